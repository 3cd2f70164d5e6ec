"""GPU parity: atomics-free backward (libfbsa.so) vs the float64 CPU oracle."""
import numpy as np
import pytest
import torch

from oracle import attn as oattn, select as osel
from _util import randn, np64, assert_close, TOL

pytestmark = pytest.mark.gpu
DEV = "cuda"
MCODE = {"none": 0, "slot_causal": 1, "token_causal": 2}


def _gpu_bwd(q, k, v, sel, do, mask, gate=None, l_valid=None, out_gate=None, scale=None, need_dgate=False):
    from fbsa_amd import ops
    print(f"[bwd] q{tuple(q.shape)} k{tuple(k.shape)} sel{tuple(np.shape(sel))} {q.dtype} mask={mask}", flush=True)
    t = lambda x: None if x is None else torch.as_tensor(x).to(DEV)  # noqa: E731
    qd, kd, vd, sd, dod = t(q), t(k), t(v), t(sel), t(do)
    gd, ogd = t(gate), t(out_gate)
    o, lse = ops.attention_forward(qd, kd, vd, sd, mask=MCODE[mask], scale=scale, gate=gd, l_valid=l_valid,
                                   out_gate=ogd, need_lse=True)
    out = ops.attention_backward(qd, kd, vd, sd, o, lse, dod, mask=MCODE[mask], scale=scale, gate=gd,
                                 l_valid=l_valid, out_gate=ogd, need_dgate=need_dgate)
    torch.cuda.synchronize()
    return [None if x is None else np64(x) for x in out]


def _oracle(q, k, v, sel, do, mask, gate=None, l_valid=None, out_gate=None, scale=None, rows=None):
    return oattn.bwd(np64(q), np64(k), np64(v), np.asarray(sel), np64(do), mask, scale=scale,
                     gate=None if gate is None else np.asarray(gate, np.float64), L_valid=l_valid,
                     out_gate=None if out_gate is None else np64(out_gate), rows=rows)


def _cmp(got, ref, dtype, names=("dq", "dk", "dv")):
    for n, gv, rv in zip(names, got, ref):
        ma, rl = assert_close(gv, rv, dtype, n)
        print(f"  {n}: max_abs={ma:.2e} rel_l2={rl:.2e}", flush=True)


def _cmp_mag(got, ref, dtype, names=("dq", "dk", "dv")):
    # the absolute bar, printing each output's largest magnitude beside its error
    for n, gv, rv in zip(names, got, ref):
        ma, rl = assert_close(gv, rv, dtype, n)
        print(f"  {n}: max|ref|={float(np.max(np.abs(rv))):.1f} max_abs={ma:.2e} rel_l2={rl:.2e}", flush=True)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_config1_shape(dtype):
    g = torch.Generator().manual_seed(0)
    B, H, N, D, bs = 1, 4, 4096, 64, 64
    q, k, v, do = (randn(g, (B, H, N, D), dtype) for _ in range(4))
    sel, _ = osel.select_mean_pooled(np64(q), np64(k), bs, 8, True, dtype)
    got = _gpu_bwd(q, k, v, sel[:, None], do, "slot_causal")
    _cmp(got, _oracle(q, k, v, sel[:, None], do, "slot_causal"), dtype)


def test_config2_gate_bias_and_dgate():
    # config 2: B32 H8 N1024 D64 bs32 causal top-4; gate = logsigmoid(N(0,1)); dO ~ N(0,1)
    g = torch.Generator().manual_seed(0)
    B, H, N, D, bs, topk = 32, 8, 1024, 64, 32, 4
    q, k, v, do = (randn(g, (B, H, N, D), "bf16") for _ in range(4))
    sel, _ = osel.select_mean_pooled(np64(q), np64(k), bs, topk, True, "bf16")
    gate = torch.nn.functional.logsigmoid(torch.randn(B, N // bs, topk + 1, generator=g)).numpy()[:, None]
    got = _gpu_bwd(q, k, v, sel[:, None], do, "slot_causal", gate=gate, need_dgate=True)
    ref = _oracle(q, k, v, sel[:, None], do, "slot_causal", gate=gate)
    _cmp(got[:3], ref[:3], "bf16")
    # dgate (fp32 output) sums bs*bs*H = 8192 score gradients per slot, each
    # formed with the row's delta as sum P dP (the prep's 16-bit-O estimate
    # corrected by its error times the slot's probability mass): the absolute
    # bf16 bar
    dg, rdg = got[3], ref[3]
    rl = float(np.linalg.norm(dg - rdg) / np.linalg.norm(rdg))
    ma = float(np.max(np.abs(dg - rdg)))
    print(f"  dgate: max_abs={ma:.2e} max|ref|={float(np.max(np.abs(rdg))):.1f} rel_l2={rl:.2e}", flush=True)
    assert ma <= TOL["bf16"]["max_abs"] and rl <= TOL["bf16"]["rel_l2"]


def test_config2_output_gate():
    # config 2 with the sigmoid output gate o * sigmoid(g), g ~ N(0,1): dq/dk/dv and d(g)
    g = torch.Generator().manual_seed(1)
    B, H, N, D, bs, topk = 32, 8, 1024, 64, 32, 4
    q, k, v, do, og = (randn(g, (B, H, N, D), "bf16") for _ in range(5))
    sel, _ = osel.select_mean_pooled(np64(q), np64(k), bs, topk, True, "bf16")
    got = _gpu_bwd(q, k, v, sel[:, None], do, "slot_causal", out_gate=og)
    ref = _oracle(q, k, v, sel[:, None], do, "slot_causal", out_gate=og)
    _cmp(got[:3], ref[:3], "bf16")
    _cmp([got[4]], [ref[4]], "bf16", names=("dout_gate",))


@pytest.mark.parametrize("bs,D", [(16, 64), (32, 32), (64, 128), (128, 64), (64, 256), (128, 256), (16, 32),
                                  (16, 256), (32, 256)])
def test_block_and_head_sizes_random_sel_with_duplicates(bs, D):
    # make_sel-style: own + random blocks with replacement (duplicates, future blocks), no mask
    g = torch.Generator().manual_seed(2)
    B, H, nblk, kk = 1, 2, 10, 5
    N = nblk * bs
    q, k, v, do = (randn(g, (B, H, N, D), "bf16") for _ in range(4))
    rnd = torch.randint(0, nblk, (B, nblk, kk - 1), generator=g)
    sel = torch.cat([torch.arange(nblk).view(1, nblk, 1), rnd], -1).numpy()[:, None]
    gate = torch.nn.functional.logsigmoid(torch.randn(B, 1, nblk, kk, generator=g)).numpy()
    got = _gpu_bwd(q, k, v, sel, do, "none", gate=gate)
    _cmp(got, _oracle(q, k, v, sel, do, "none", gate=gate), "bf16")
    got = _gpu_bwd(q, k, v, sel, do, "slot_causal")
    _cmp(got, _oracle(q, k, v, sel, do, "slot_causal"), "bf16")


@pytest.mark.parametrize("dtype,D", [("bf16", 128), ("f32", 128), ("bf16", 256), ("f16", 256)])
def test_gqa_token_causal_padding_outgate(dtype, D):
    # bs 128 with fp32 d 128 or 16-bit d 256 splits each key block's dK/dV over two workgroups
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, N, bs, topk = 1, 8, 2, 1024, 128, 3
    q, do, og = (randn(g, (B, Hq, N, D), dtype) for _ in range(3))
    k, v = (randn(g, (B, Hkv, N, D), dtype) for _ in range(2))
    idx, _ = osel.select_quest(np64(q), np64(k), bs, topk, True, dtype)
    lv = N - 77
    got = _gpu_bwd(q, k, v, idx, do, "token_causal", l_valid=lv, out_gate=og, scale=0.0625)
    ref = _oracle(q, k, v, idx, do, "token_causal", l_valid=lv, out_gate=og, scale=0.0625)
    _cmp(got[:3], ref[:3], dtype)
    _cmp([got[4]], [ref[4]], dtype, names=("dout_gate",))


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_long_lists_walked_in_segments(dtype):
    # GQA 16:1, bs 16, d 256: one dK/dV workgroup walks at most 256 entries of a
    # transposed list. Block 0 is selected twice in odd rows and once in even rows
    # (576 entries: three segments whose fp32 partials are summed in order),
    # block 1 once in even rows (192 entries: one workgroup)
    g = torch.Generator().manual_seed(5)
    B, Hq, Hkv, N, D, bs, kk = 1, 16, 1, 6144, 256, 16, 4
    nblk = N // bs
    q, do = (randn(g, (B, Hq, N, D), dtype) for _ in range(2))
    k, v = (randn(g, (B, Hkv, N, D), dtype) for _ in range(2))
    i = torch.arange(nblk).view(1, nblk, 1)
    rnd = torch.randint(2, nblk, (B, nblk, kk - 3), generator=g)
    sel = torch.cat([i, torch.zeros_like(i), torch.where(i % 2 == 1, 0, 1), rnd], -1).numpy()[:, None]
    got = _gpu_bwd(q, k, v, sel, do, "none")
    ref = _oracle(q, k, v, sel, do, "none")
    # a split list sums at least 4096 * 16 query rows per key, so block 0's dK/dV
    # is large (|dK| ~ 40); 16-bit P and dS enter its products as hi/lo pairs,
    # so the absolute bar of the dtype holds (beyond the output's own rounding)
    _cmp_mag(got[:3], ref[:3], dtype)


def test_duplicate_heavy_list_segments_half_blocks():
    # bs 128, 16-bit d 256: each key block's dK/dV is split over two half-block
    # workgroups (two waves per key group); every non-own slot of every row picks
    # block 0 (mask none keeps duplicates), so its list has 5 * 33 + 1 = 166
    # entries, more than one segment (128 at GQA 8, four chunks per block)
    g = torch.Generator().manual_seed(6)
    B, Hq, Hkv, N, D, bs, kk = 1, 8, 1, 640, 256, 128, 34
    nblk = N // bs
    q, do = (randn(g, (B, Hq, N, D), "bf16") for _ in range(2))
    k, v = (randn(g, (B, Hkv, N, D), "bf16") for _ in range(2))
    sel = np.zeros((B, 1, nblk, kk), np.int64)
    sel[..., 0] = np.arange(nblk)
    got = _gpu_bwd(q, k, v, sel, do, "none")
    ref = _oracle(q, k, v, sel, do, "none")
    _cmp_mag(got[:3], ref[:3], "bf16")  # block 0 sums 166 * 8 * 128 rows (see above)


@pytest.mark.parametrize("dtype,D", [("bf16", 64), ("f32", 32)])
def test_segments_of_small_blocks(dtype, D):
    # bs 16 with d 64 / 32: a key block's dK and dV hold 2 * 16 * D elements, fewer
    # than one 8192-element slice of the segment reduction, so most of a reducing
    # thread's element groups lie past the block. Every content slot of every row
    # picks block 0 (mask none keeps duplicates): its list has 128 * 8 + 1 = 1025
    # entries, three segments of at most 512
    g = torch.Generator().manual_seed(8)
    B, H, N, bs, kk = 1, 2, 2048, 16, 9
    nblk = N // bs
    q, k, v, do = (randn(g, (B, H, N, D), dtype) for _ in range(4))
    sel = np.zeros((B, 1, nblk, kk), np.int64)
    sel[..., 0] = np.arange(nblk)
    got = _gpu_bwd(q, k, v, sel, do, "none")
    ref = _oracle(q, k, v, sel, do, "none")
    _cmp_mag(got[:3], ref[:3], dtype)  # block 0 sums 1025 * 16 rows per head


def test_backward_is_bitwise_repeatable():
    g = torch.Generator().manual_seed(4)
    B, H, N, D, bs, kk = 2, 4, 2048, 64, 64, 9
    nblk = N // bs
    q, k, v, do = (randn(g, (B, H, N, D), "bf16") for _ in range(4))
    # every row selects block 0 and 1: long transposed lists
    sel = torch.randint(0, nblk, (B, 1, nblk, kk), generator=g)
    sel[..., 1], sel[..., 2] = 0, 1
    a = _gpu_bwd(q, k, v, sel, do, "none")
    b = _gpu_bwd(q, k, v, sel, do, "none")
    for x, y in zip(a[:3], b[:3]):
        assert np.array_equal(x, y)
    _cmp(a, _oracle(q, k, v, sel.numpy(), do, "none"), "bf16")


def test_config3_full_size_sampled_blocks():
    # config 3: B1 H8 N262144 D64 bs64 top-16, q,k,v ~ N(0,1)/8, dO ~ N(0,1).
    # dq is checked on sampled query blocks; dk/dv on key blocks whose every
    # reading query block is included in the oracle's rows.
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(0)
    B, H, N, D, bs, topk = 1, 8, 262144, 64, 64, 16
    q, k, v = (randn(g, (B, H, N, D), "bf16", scale=0.125) for _ in range(3))
    do = randn(g, (B, H, N, D), "bf16")
    sel = selection.select_mean_pooled(q.to(DEV), k.to(DEV), bs, topk, True).cpu().numpy()[:, None]
    got = _gpu_bwd(q, k, v, sel, do, "slot_causal")
    nblk = N // bs
    keyblocks = [0, 5, 2048, nblk - 1]
    readers = set()
    for j in keyblocks:
        hit = (sel[0, 0] == j)
        valid = hit & ((np.arange(sel.shape[-1])[None, :] == 0) | (j < np.arange(nblk))[:, None])
        readers |= set(np.nonzero(valid.any(1))[0].tolist())
    qrows = [1, 100, 3000, nblk - 1]
    rows = sorted(readers | set(qrows))
    print(f"  oracle over {len(rows)} query blocks", flush=True)
    ref = _oracle(q, k, v, sel, do, "slot_causal", rows=rows)
    tsel = lambda x, blocks: np.concatenate([x[:, :, b * bs:(b + 1) * bs] for b in blocks], 2)  # noqa: E731
    _cmp([tsel(got[0], qrows)], [tsel(ref[0], qrows)], "bf16", names=("dq",))
    _cmp([tsel(got[1], keyblocks), tsel(got[2], keyblocks)], [tsel(ref[1], keyblocks), tsel(ref[2], keyblocks)],
         "bf16", names=("dk", "dv"))


def test_bsattn_reference_surface_autograd():
    # BSAttnFunction/bsattn contract (src/triton_kernel.py:237-259): grads for q,k,v; None for gate
    from fbsa_amd import autograd
    g = torch.Generator().manual_seed(5)
    B, H, N, D, bs, topk = 2, 2, 512, 64, 64, 3
    q, k, v, do = (randn(g, (B, H, N, D), "bf16") for _ in range(4))
    sel, raw = osel.select_mean_pooled(np64(q), np64(k), bs, topk, True, "bf16")
    gate = torch.nn.functional.logsigmoid(torch.as_tensor(np.take_along_axis(raw, sel, -1), dtype=torch.float32))
    qd, kd, vd = (x.to(DEV).requires_grad_(True) for x in (q, k, v))
    gd = gate.to(DEV).requires_grad_(True)
    o = autograd.bsattn(qd, kd, vd, torch.as_tensor(sel, dtype=torch.int32).to(DEV), gd, causal=True)
    o.backward(do.to(DEV))
    assert gd.grad is None
    ref = _oracle(q, k, v, sel[:, None], do, "slot_causal", gate=gate.numpy()[:, None])
    _cmp([np64(qd.grad), np64(kd.grad), np64(vd.grad)], ref[:3], "bf16")
