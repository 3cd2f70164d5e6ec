"""GPU: fbsa_bwd without a separate prep pass against its four stages called one by one.

For bf16 without an output gate, fbsa_bwd lets the dQ stage form each
row's statistics (lse * log2 e and sum_d dO*O) from O and lse instead of
running fbsa_bwd_prep. The stages called one by one (fbsa_bwd_prep,
fbsa_transpose_index, fbsa_bwd_dq, fbsa_bwd_dkdv) take the prep path. The row
statistics are the same values summed in the same order, so dq, dk, dv and the
gate gradient must be bit-identical between the two. (fp16 keeps the prep
stage in fbsa_bwd: there the two kernels' sums differed in the last bit; the
fp16 case checks that both calls still agree.)"""
import pytest
import torch

from _util import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _staged(q, k, v, sel, o, lse, do, mask, scale, gate=None, need_dgate=False):
    from fbsa_amd import _lib, ops
    B, Hq, L, D = q.shape
    qk = [ops._kernel_ready(t) for t in (q, k, v)]
    o_p, do_p = ops._kernel_ready(o), ops._kernel_ready(do)
    sel32 = sel.to(torch.int32).contiguous()
    gate32 = gate.to(torch.float32).contiguous() if gate is not None else None
    lse_c = lse.contiguous()
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dgate = torch.empty(sel32.shape, dtype=torch.float32, device=DEV) if need_dgate else None
    d = ops.make_desc(qk[0], qk[1], qk[2], o_p, sel32, mask=mask, scale=scale, l_valid=L, dout=do_p)
    d.flags |= _lib.FLAG_DGATE if need_dgate else 0
    lib = _lib.load()
    nbytes = lib.fbsa_bwd_workspace_bytes(d)
    assert nbytes > 0
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=DEV)
    wp = (ws.data_ptr() + 255) // 256 * 256
    P, s = ops._ptr, ops._stream()
    _lib.check(lib.fbsa_bwd_prep(d, P(o_p), P(do_p), P(lse_c), None, None, wp, nbytes, s), "fbsa_bwd_prep")
    _lib.check(lib.fbsa_transpose_index(d, P(sel32), wp, nbytes, s), "fbsa_transpose_index")
    _lib.check(lib.fbsa_bwd_dq(d, P(qk[0]), P(qk[1]), P(qk[2]), P(do_p), P(sel32), P(gate32), P(dq), P(dgate),
                               wp, nbytes, s), "fbsa_bwd_dq")
    _lib.check(lib.fbsa_bwd_dkdv(d, P(qk[0]), P(qk[1]), P(qk[2]), P(do_p), P(gate32), P(dk), P(dv), wp, nbytes, s),
               "fbsa_bwd_dkdv")
    torch.cuda.synchronize()
    return dq, dk, dv, dgate


@pytest.mark.parametrize("case", ["bf16_d64_bs64_slot_gate_dgate", "f16_d128_bs32_token_gqa", "bf16_d256_bs128_token_gqa",
                                  "bf16_d32_bs16_none"])
def test_fused_row_stats_bit_identical(case):
    from fbsa_amd import ops
    g = torch.Generator().manual_seed(41)
    dt = "f16" if case.startswith("f16") else "bf16"
    D = int(case.split("_d")[1].split("_")[0])
    bs = int(case.split("_bs")[1].split("_")[0])
    mask = {"slot": ops.MASK_SLOT_CAUSAL, "token": ops.MASK_TOKEN_CAUSAL, "none": ops.MASK_NONE}[case.split("_")[3]]
    Hq, Hkv = (8, 2) if "gqa" in case else (4, 4)
    B, nblk, kk = 2, 40, 7
    L = nblk * bs
    q, do = (randn(g, (B, Hq, L, D), dt, device=DEV) for _ in range(2))
    k, v = (randn(g, (B, Hkv, L, D), dt, device=DEV) for _ in range(2))
    i = torch.arange(nblk).view(1, 1, nblk, 1)
    past = (torch.rand(B, Hkv, nblk, kk - 1, generator=g) * (i + 1 if mask != ops.MASK_SLOT_CAUSAL else i)).long()
    if mask == ops.MASK_NONE:
        past = (torch.rand(B, Hkv, nblk, kk - 1, generator=g) * nblk).long()
    sel = torch.cat([i.expand(B, Hkv, nblk, 1), past], -1).to(torch.int32).to(DEV)
    gate = None
    need_dgate = "dgate" in case
    if "gate" in case:
        gate = torch.nn.functional.logsigmoid(torch.randn(B, Hkv, nblk, kk, generator=g)).to(DEV)
    sc = D ** -0.5
    print(f"[fused-rowstats] {case}", flush=True)
    o, lse = ops.attention_forward(q, k, v, sel, mask=mask, scale=sc, gate=gate, need_lse=True)
    fused = ops.attention_backward(q, k, v, sel, o, lse, do, mask=mask, scale=sc, gate=gate, need_dgate=need_dgate)
    staged = _staged(q, k, v, sel, o, lse, do, mask, sc, gate=gate, need_dgate=need_dgate)
    for n, a, b in zip(("dq", "dk", "dv", "dgate"), fused[:4], staged):
        if a is None:
            assert b is None
            continue
        eq = torch.equal(a, b)
        print(f"[fused-rowstats] {case} {n}: bit-identical={eq}", flush=True)
        assert eq, f"{case}: {n} differs between fbsa_bwd and its stages"
