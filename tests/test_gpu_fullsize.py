"""GPU parity at the benchmarked shapes, every output row.

* Configuration 3 forward (B1 H8 N262144 D64 bs64, top-16 own-first,
  slot-causal): O on all rows against the fp32 torch gather path
  (``tests/_torchref.py``, pinned against the oracle by ``tests/test_torchref.py``)
  and sampled query blocks against the float64 oracle.
* Configuration 4 (B1 N65536 Hq16 Hkv2 D256 bs128, partial RoPE, ``SelectMax``
  top-32 + own + sink, token-causal, output gate): forward and backward on all
  rows against the fp32 torch gather path -- including dK/dV of the sink block 0,
  whose transposed list holds every row and is walked in segments -- and
  sampled query blocks / a whole key block against the oracle.
* The same GQA 16:2 token-causal sink path in fp32 at a smaller length (block
  0's list still split into segments), against the 1e-4 fp32 bar.

Every comparison prints its absolute max-abs (beyond the output dtype's own
rounding) and relative L2."""
import numpy as np
import pytest
import torch

from oracle import attn as oattn
from _util import randn, np64, TOL, OUT_ROUND, rel_l2
import _torchref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print("[fullsize]", *a, flush=True)


def _check(name, got, ref, dtype, tol_scale=1.0):
    """Absolute bar of the dtype (max-abs beyond the output's storage rounding,
    relative L2); prints both numbers."""
    got = got.double() if torch.is_tensor(got) else torch.as_tensor(got, dtype=torch.float64)
    ref = ref.double() if torch.is_tensor(ref) else torch.as_tensor(ref, dtype=torch.float64)
    ref = ref.to(got.device)
    t = TOL[dtype]
    excess = float((got - ref).abs().sub(OUT_ROUND[dtype] * ref.abs()).max())
    rl = float((got - ref).norm() / ref.norm().clamp_min(1e-30))
    _say(f"{name}: max_abs={excess:.3e} rel_l2={rl:.3e} max|ref|={float(ref.abs().max()):.3g}")
    assert excess <= t["max_abs"] * tol_scale and rl <= t["rel_l2"], f"{name}: {excess:.3e} / {rl:.3e}"
    return excess, rl


# The forward sums its row normalisers in fp32 from the unrounded exponentials
# (the 16-bit rounding of P enters only the P.V product), so the LSE is an fp32
# quantity for every input dtype.
LSE_TOL = {"bf16": 1e-4, "f16": 1e-4, "f32": 1e-4}


def _blocks(x, blocks, bs):
    return torch.cat([x[:, :, b * bs:(b + 1) * bs] for b in blocks], 2)


# ---------------------------------------------------------------- configuration 3
@pytest.fixture(scope="module")
def cfg3():
    # B1 H8 N262144 D64 bs64, top-16 own-first, slot-causal; q,k,v ~ N(0,1)/8, dO ~ N(0,1)
    from fbsa_amd import ops, selection
    g = torch.Generator().manual_seed(0)
    B, H, N, D, bs, topk = 1, 8, 262144, 64, 64, 16
    q, k, v = (randn(g, (B, H, N, D), "bf16", scale=0.125) for _ in range(3))
    do = randn(g, (B, H, N, D), "bf16")
    qd, kd, vd, dod = q.to(DEV), k.to(DEV), v.to(DEV), do.to(DEV)
    sel = selection.select_mean_pooled(qd, kd, bs, topk, True)[:, None]
    o, lse = ops.attention_forward(qd, kd, vd, sel, mask=ops.MASK_SLOT_CAUSAL, need_lse=True)
    grads = ops.attention_backward(qd, kd, vd, sel, o, lse, dod, mask=ops.MASK_SLOT_CAUSAL)
    ref = _torchref.attention(qd, kd, vd, sel, "slot_causal", do=dod, chunk=256)
    torch.cuda.synchronize()
    return dict(q=q, k=k, v=v, do=do, sel=sel, o=o, lse=lse, grads=grads, ref=ref, bs=bs)


def test_config3_forward_all_rows(cfg3):
    c = cfg3
    _check("config 3 o (all rows, fp32 torch)", c["o"], c["ref"][0], "bf16")
    lerr = float((c["lse"] - c["ref"][1]).abs().max())
    _say(f"config 3 lse: max_abs={lerr:.3e}")
    assert lerr <= LSE_TOL["bf16"]
    rows, bs = [0, 1, 16, 17, 1000, 2048, 4095], c["bs"]
    so, _ = oattn.fwd(np64(c["q"]), np64(c["k"]), np64(c["v"]), c["sel"].cpu().numpy(), "slot_causal", rows=rows)
    _check("config 3 o (sampled blocks, oracle)", _blocks(c["o"], rows, bs).cpu(), so, "bf16")


def test_config3_backward_all_rows(cfg3):
    # dq on every query row, dk / dv on every key block, against the fp32 torch
    # gather path's autograd (src/verify_kernel.py:15-39 compares the same three
    # gradients against the gather path)
    c = cfg3
    dq, dk, dv = c["grads"][:3]
    _, _, rdq, rdk, rdv, _ = c["ref"]
    _check("config 3 dq (all rows, fp32 torch)", dq, rdq, "bf16")
    _check("config 3 dk (all blocks, fp32 torch)", dk, rdk, "bf16")
    _check("config 3 dv (all blocks, fp32 torch)", dv, rdv, "bf16")


# ---------------------------------------------------------------- configuration 4
@pytest.fixture(scope="module")
def cfg4():
    import qwen_blocksparse as qb
    from bench import rope_partial
    from fbsa_amd import ops
    B, Hq, Hkv, N, D, bs, topk = 1, 16, 2, 65536, 256, 128, 32
    g = torch.Generator(device=DEV).manual_seed(4)
    rn = lambda *s: torch.randn(*s, generator=g, device=DEV).to(torch.bfloat16)  # noqa: E731
    q = rope_partial(rn(B, Hq, N, D))
    k = rope_partial(rn(B, Hkv, N, D))
    v, og, do = rn(B, Hkv, N, D), rn(B, Hq, N, D), rn(B, Hq, N, D)
    idx = qb.SelectMax(topk=topk, bs=bs, sink=True).select(q, k)
    nblk = N // bs
    assert idx.shape == (B, Hkv, nblk, topk + 2) and bool((idx[..., 0] == 0).all())
    sc = D ** -0.5
    idx32 = idx.to(torch.int32).contiguous()
    o, lse = ops.attention_forward(q, k, v, idx32, mask=ops.MASK_TOKEN_CAUSAL, scale=sc, out_gate=og,
                                   need_lse=True)
    grads = ops.attention_backward(q, k, v, idx32, o, lse, do, mask=ops.MASK_TOKEN_CAUSAL, scale=sc,
                                   out_gate=og)
    ref = _torchref.attention(q, k, v, idx, "token_causal", scale=sc, out_gate=og, do=do, chunk=16)
    torch.cuda.synchronize()
    lens = [int((idx[0, h] == j).any(-1).sum()) for h in range(Hkv) for j in (0,)]
    _say("config 4: sink block 0 read by", lens, "rows per KV head")
    return dict(q=q, k=k, v=v, og=og, do=do, idx=idx, o=o, lse=lse, grads=grads, ref=ref, bs=bs, sc=sc)


def test_config4_forward_all_rows(cfg4):
    c = cfg4
    _check("config 4 o (all rows, fp32 torch)", c["o"], c["ref"][0], "bf16")
    lerr = float((c["lse"] - c["ref"][1]).abs().max())
    _say(f"config 4 lse: max_abs={lerr:.3e}")
    assert lerr <= LSE_TOL["bf16"]
    # sampled query blocks of KV group 0 (heads 0..7) against the oracle
    rows, grp = [0, 255, 511], 8
    so, _ = oattn.fwd(np64(c["q"][:, :grp]), np64(c["k"][:, :1]), np64(c["v"][:, :1]),
                      c["idx"][:, :1].cpu().numpy(), "token_causal", scale=c["sc"],
                      out_gate=np64(c["og"][:, :grp]), rows=rows)
    _check("config 4 o (sampled blocks, oracle)", _blocks(c["o"][:, :grp], rows, c["bs"]).cpu(), so, "bf16")


def test_config4_backward_all_rows(cfg4):
    c = cfg4
    dq, dk, dv, _, dog = c["grads"]
    _, _, rdq, rdk, rdv, rdog = c["ref"]
    bs = c["bs"]
    _check("config 4 dq (all rows, fp32 torch)", dq, rdq, "bf16")
    _check("config 4 dout_gate (all rows, fp32 torch)", dog, rdog, "bf16")
    _check("config 4 dk (all blocks, fp32 torch)", dk, rdk, "bf16")
    _check("config 4 dv (all blocks, fp32 torch)", dv, rdv, "bf16")
    _check("config 4 dk of sink block 0 (segmented list)", dk[:, :, :bs], rdk[:, :, :bs], "bf16")
    _check("config 4 dv of sink block 0 (segmented list)", dv[:, :, :bs], rdv[:, :, :bs], "bf16")
    # the oracle: dq of the last query block and the complete dK/dV of the last key
    # block (token-causal: only the last query block can read it), KV group 0
    grp, last = 8, c["idx"].shape[2] - 1
    r = oattn.bwd(np64(c["q"][:, :grp]), np64(c["k"][:, :1]), np64(c["v"][:, :1]),
                  c["idx"][:, :1].cpu().numpy(), np64(c["do"][:, :grp]), "token_causal", scale=c["sc"],
                  out_gate=np64(c["og"][:, :grp]), rows=[last])
    _check("config 4 dq (last block, oracle)", _blocks(dq[:, :grp], [last], bs).cpu(), _blocks(
        torch.as_tensor(r[0]), [last], bs), "bf16")
    _check("config 4 dk (last block, oracle)", _blocks(dk[:, :1], [last], bs).cpu(),
           _blocks(torch.as_tensor(r[1]), [last], bs), "bf16")
    _check("config 4 dv (last block, oracle)", _blocks(dv[:, :1], [last], bs).cpu(),
           _blocks(torch.as_tensor(r[2]), [last], bs), "bf16")


# ------------------------------------------- GQA token-causal sink path, fp32 and bf16
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_gqa_token_causal_sink_segments(dtype):
    # Hq 16 / Hkv 2, bs 128, d 256, hsel = Hkv, sorted own + sink + 8 random past
    # blocks per row: block 0's transposed list holds all 300 rows (+ duplicates
    # in the first rows), more than one segment of 4096 work chunks
    from fbsa_amd import ops
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, nblk, D, bs, kr = 1, 16, 2, 300, 256, 128, 8
    N = nblk * bs
    q, do, og = (randn(g, (B, Hq, N, D), dtype) for _ in range(3))
    k, v = (randn(g, (B, Hkv, N, D), dtype) for _ in range(2))
    i = torch.arange(nblk).view(1, 1, nblk, 1)
    past = (torch.rand(B, Hkv, nblk, kr, generator=g) * (i + 1)).long()        # blocks <= i
    idx = torch.cat([past, i.expand(B, Hkv, nblk, 1), torch.zeros(B, Hkv, nblk, 1, dtype=torch.long)], -1)
    idx = idx.sort(-1).values
    qd, kd, vd, dod, ogd = (x.to(DEV) for x in (q, k, v, do, og))
    sc = D ** -0.5
    idx32 = idx.to(torch.int32).to(DEV)
    o, lse = ops.attention_forward(qd, kd, vd, idx32, mask=ops.MASK_TOKEN_CAUSAL, scale=sc, out_gate=ogd,
                                   need_lse=True)
    dq, dk, dv, _, dog = ops.attention_backward(qd, kd, vd, idx32, o, lse, dod, mask=ops.MASK_TOKEN_CAUSAL,
                                                scale=sc, out_gate=ogd)
    ro, _, rdq, rdk, rdv, rdog = _torchref.attention(qd, kd, vd, idx.to(DEV), "token_causal", scale=sc,
                                                     out_gate=ogd, do=dod, chunk=25)
    torch.cuda.synchronize()
    for name, got, ref in (("o", o, ro), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv),
                           ("dout_gate", dog, rdog), ("dk block 0", dk[:, :, :bs], rdk[:, :, :bs]),
                           ("dv block 0", dv[:, :, :bs], rdv[:, :, :bs])):
        _check(f"sink segments {dtype} {name} (fp32 torch)", got, ref, dtype)
    # the oracle on KV group 1: dq of two query blocks and the complete dK/dV of
    # the last key block (only the last query block reads it)
    rows = [5, nblk - 1]
    r = oattn.bwd(np64(q[:, 8:]), np64(k[:, 1:]), np64(v[:, 1:]), idx[:, 1:].numpy(), np64(do[:, 8:]),
                  "token_causal", scale=sc, out_gate=np64(og[:, 8:]), rows=rows)
    _check(f"sink segments {dtype} dq (oracle)", _blocks(dq[:, 8:], rows, bs).cpu(),
           _blocks(torch.as_tensor(r[0]), rows, bs), dtype)
    _check(f"sink segments {dtype} dk last block (oracle)", _blocks(dk[:, 1:], [nblk - 1], bs).cpu(),
           _blocks(torch.as_tensor(r[1]), [nblk - 1], bs), dtype)
    _check(f"sink segments {dtype} dv last block (oracle)", _blocks(dv[:, 1:], [nblk - 1], bs).cpu(),
           _blocks(torch.as_tensor(r[2]), [nblk - 1], bs), dtype)


# ---------------------------------------------------------------- configuration 5
def test_config5_forward_sampled_blocks():
    # B1 H8 D64 N4194304 bs64 (nblk 65536), top-16 own-first, slot-causal: the
    # selection-scaling stress shape. O of the first and last 8 query blocks and
    # 40 random ones against the float64 oracle. Each sampled row is checked on
    # a small problem made of its own block and the blocks it selects,
    # renumbered in ascending order (the slot-causal rule only compares block
    # indices, so an order-preserving renumbering keeps every mask decision).
    from fbsa_amd import ops, selection
    B, H, N, D, bs, topk = 1, 8, 4194304, 64, 64, 16
    nblk = N // bs
    g = torch.Generator(device=DEV).manual_seed(5)
    q, k, v = ((torch.randn(B, H, N, D, generator=g, device=DEV) * D ** -0.5).to(torch.bfloat16) for _ in range(3))
    sel = selection.select_mean_pooled(q, k, bs, topk, True)[:, None]
    o = ops.attention_forward(q, k, v, sel, mask=ops.MASK_SLOT_CAUSAL)
    torch.cuda.synchronize()
    _say("config 5 forward done")
    sel_np = sel.cpu().numpy()
    rows = np.unique(np.concatenate([np.arange(8), np.arange(nblk - 8, nblk),
                                     np.random.default_rng(5).integers(8, nblk - 8, 40)]))
    worst = 0.0
    for i in rows.tolist():
        srow = sel_np[0, 0, i]
        blocks = np.unique(np.concatenate([srow, [i]]))
        rank = {int(b): r for r, b in enumerate(blocks)}
        nb = len(blocks)
        take = torch.as_tensor(blocks, device=DEV)
        kb = k.view(B, H, nblk, bs, D)[:, :, take].reshape(B, H, nb * bs, D)
        vb = v.view(B, H, nblk, bs, D)[:, :, take].reshape(B, H, nb * bs, D)
        qb = torch.zeros(B, H, nb, bs, D, dtype=q.dtype, device=DEV)
        qb[:, :, rank[i]] = q.view(B, H, nblk, bs, D)[:, :, i]
        smini = np.zeros((B, 1, nb, srow.size), np.int64)
        smini[0, 0, rank[i]] = [rank[int(j)] for j in srow]
        so, _ = oattn.fwd(np64(qb.reshape(B, H, nb * bs, D)), np64(kb), np64(vb), smini, "slot_causal",
                          rows=[rank[i]])
        ex, _ = _check(f"config 5 o block {i} (oracle)", o[:, :, i * bs:(i + 1) * bs].cpu(), so, "bf16")
        worst = max(worst, ex)
    _say(f"config 5 o over {len(rows)} sampled blocks: worst max_abs={worst:.3e}")
