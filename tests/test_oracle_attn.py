"""Pins for the attention oracle (CPU, float64).

Each check is independent of the oracle's own vectorised formula:
brute-force per-token enumeration of the reference's per-slot mask rules,
the all-blocks == dense closed forms (``scripts/run_all.sh:7-21``,
``src/test_qwen_blocksparse.py:17-34``), torch's own SDPA for the dense form,
gate-bias identities, and central finite differences for the backward."""
import numpy as np
import pytest
import torch

from oracle import attn as oattn

RNG = np.random.default_rng(0)


def _qkv(B, Hq, Hkv, N, D, rng=RNG):
    return (rng.standard_normal((B, Hq, N, D)), rng.standard_normal((B, Hkv, N, D)),
            rng.standard_normal((B, Hkv, N, D)))


def _rand_sel(B, Hs, nblk, kk, rng=RNG, own_first=True):
    sel = rng.integers(0, nblk, (B, Hs, nblk, kk))
    if own_first:
        sel[..., 0] = np.arange(nblk)
    return sel


@pytest.mark.parametrize("mask", oattn.MASKS)
@pytest.mark.parametrize("Hq,Hkv,Hs", [(2, 2, 1), (4, 2, 2), (4, 1, 1)])
def test_fwd_matches_bruteforce(mask, Hq, Hkv, Hs):
    B, N, D, bs, kk = 2, 48, 8, 8, 4
    nblk = N // bs
    q, k, v = _qkv(B, Hq, Hkv, N, D)
    sel = _rand_sel(B, Hs, nblk, kk)       # random with replacement: duplicates and future blocks
    gate = RNG.standard_normal((B, Hs, nblk, kk))
    lv = N - 5 if mask == "token_causal" else None
    o, _ = oattn.fwd(q, k, v, sel, mask, gate=gate, L_valid=lv)
    ob = oattn.fwd_bruteforce(q, k, v, sel, mask, gate=gate, L_valid=lv)
    np.testing.assert_allclose(o, ob, rtol=1e-12, atol=1e-12)


def test_dense_matches_torch_sdpa():
    q, k, v = _qkv(1, 4, 2, 40, 16)
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    for causal in (False, True):
        ref = torch.nn.functional.scaled_dot_product_attention(
            tq, tk.repeat_interleave(2, 1), tv.repeat_interleave(2, 1), is_causal=causal).numpy()
        np.testing.assert_allclose(oattn.dense(q, k, v, causal), ref, rtol=1e-10, atol=1e-12)


def test_all_blocks_equal_dense():
    B, Hq, Hkv, N, D, bs = 1, 4, 2, 64, 16, 16
    nblk = N // bs
    q, k, v = _qkv(B, Hq, Hkv, N, D)
    # SelectAll + token-causal rule (src/qwen_blocksparse.py:155-165) == causal dense
    sel = np.broadcast_to(np.arange(nblk), (B, Hkv, nblk, nblk))
    o, _ = oattn.fwd(q, k, v, sel, "token_causal")
    np.testing.assert_allclose(o, oattn.dense(q, k, v, True), rtol=1e-10, atol=1e-12)
    # convention A with topk >= nblk-1: non-causal -> dense, slot-causal -> causal dense
    own = np.arange(nblk)[:, None]
    rest = np.array([[j for j in range(nblk) if j != i] for i in range(nblk)])
    selA = np.concatenate([own, rest], 1)[None, None]
    qa, ka, va = _qkv(B, 2, 2, N, D)
    o, _ = oattn.fwd(qa, ka, va, selA, "none")
    np.testing.assert_allclose(o, oattn.dense(qa, ka, va, False), rtol=1e-10, atol=1e-12)
    o, _ = oattn.fwd(qa, ka, va, selA, "slot_causal")
    np.testing.assert_allclose(o, oattn.dense(qa, ka, va, True), rtol=1e-10, atol=1e-12)
    # padding: keys at positions >= L_valid are ignored
    o, _ = oattn.fwd(q, k, v, sel, "token_causal", L_valid=50)
    np.testing.assert_allclose(o[:, :, :50], oattn.dense(q, k, v, True, L_valid=50)[:, :, :50], rtol=1e-10, atol=1e-12)


def test_gate_identities():
    B, H, N, D, bs, kk = 1, 2, 32, 8, 8, 3
    nblk = N // bs
    q, k, v = _qkv(B, H, H, N, D)
    sel = _rand_sel(B, 1, nblk, kk)
    base, lse0 = oattn.fwd(q, k, v, sel, "none")
    # a constant bias on every slot cancels in the softmax and shifts the lse
    o, lse = oattn.fwd(q, k, v, sel, "none", gate=np.full(sel.shape, -1.7))
    np.testing.assert_allclose(o, base, rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(lse, lse0 - 1.7, rtol=1e-12, atol=1e-12)
    # a -inf bias on a slot removes it; the same as masking it out of the row
    g = np.zeros(sel.shape)
    g[..., 2] = -np.inf
    o, _ = oattn.fwd(q, k, v, sel, "none", gate=g)
    np.testing.assert_allclose(o, oattn.fwd(q, k, v, sel[..., :2], "none")[0], rtol=1e-12, atol=1e-13)
    # bias log(2) on a slot == that slot's keys counted twice
    g = np.zeros(sel.shape)
    g[..., 1] = np.log(2.0)
    o, _ = oattn.fwd(q, k, v, sel, "none", gate=g)
    dup = np.concatenate([sel, sel[..., 1:2]], -1)
    np.testing.assert_allclose(o, oattn.fwd(q, k, v, dup, "none")[0], rtol=1e-12, atol=1e-13)


def test_out_gate_and_empty_rows():
    B, H, N, D, bs = 1, 1, 32, 8, 8
    q, k, v = _qkv(B, H, H, N, D)
    og = RNG.standard_normal((B, H, N, D))
    sel = np.array([[[[0], [1], [2], [3]]]])
    o, lse = oattn.fwd(q, k, v, sel, "token_causal", out_gate=og, L_valid=9)
    plain, _ = oattn.fwd(q, k, v, sel, "token_causal", L_valid=9)
    np.testing.assert_allclose(o, plain / (1 + np.exp(-og)), rtol=1e-12)
    # blocks 2 and 3 only see keys >= 16 > L_valid: empty rows give 0 and -inf
    assert np.all(o[:, :, 16:] == 0) and np.all(np.isneginf(lse[:, :, 16:]))


def _fd_check(mask, Hq, Hkv, Hs, with_og, lv=None):
    rng = np.random.default_rng(7)
    B, N, D, bs, kk = 1, 16, 4, 4, 3
    nblk = N // bs
    q, k, v = _qkv(B, Hq, Hkv, N, D, rng)
    sel = _rand_sel(B, Hs, nblk, kk, rng)
    gate = rng.standard_normal(sel.shape)
    do = rng.standard_normal(q.shape)
    og = rng.standard_normal(q.shape) if with_og else None

    def f(q_, k_, v_, g_, og_):
        o, _ = oattn.fwd(q_, k_, v_, sel, mask, gate=g_, L_valid=lv, out_gate=og_)
        return float((o * do).sum())

    dq, dk, dv, dg, dog = oattn.bwd(q, k, v, sel, do, mask, gate=gate, L_valid=lv, out_gate=og)
    eps = 1e-6
    args = [q, k, v, gate, og]
    grads = [dq, dk, dv, dg, dog]
    for ai in range(5 if with_og else 4):
        x = args[ai]
        for idx in [tuple(rng.integers(0, s) for s in x.shape) for _ in range(12)]:
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            ap, am = list(args), list(args)
            ap[ai], am[ai] = xp, xm
            num = (f(*ap) - f(*am)) / (2 * eps)
            assert abs(num - grads[ai][idx]) < 1e-6 * max(1.0, abs(num)), (ai, idx, num, grads[ai][idx])


@pytest.mark.parametrize("mask", oattn.MASKS)
def test_bwd_matches_finite_differences(mask):
    _fd_check(mask, 2, 2, 1, False)
    _fd_check(mask, 4, 2, 2, True, lv=13 if mask == "token_causal" else None)


def test_bwd_row_partition_sums_to_full():
    rng = np.random.default_rng(3)
    B, H, N, D, bs, kk = 1, 2, 48, 8, 8, 4
    nblk = N // bs
    q, k, v = _qkv(B, H, H, N, D, rng)
    sel = _rand_sel(B, 1, nblk, kk, rng)
    do = rng.standard_normal(q.shape)
    full = oattn.bwd(q, k, v, sel, do, "slot_causal")
    a = oattn.bwd(q, k, v, sel, do, "slot_causal", rows=[0, 2, 5])
    b = oattn.bwd(q, k, v, sel, do, "slot_causal", rows=[1, 3, 4])
    for x, y, z in zip(full[:4], a[:4], b[:4]):
        np.testing.assert_allclose(x, y + z, rtol=1e-12, atol=1e-12)


def test_block_mass_closed_forms():
    # q = 0: every score is 0, so row t attends uniformly to keys 0..t
    B, Hq, Hkv, L, D, bs = 1, 2, 1, 128, 16, 32
    rng = np.random.default_rng(7)
    k = rng.standard_normal((B, Hkv, L, D))
    m0 = oattn.block_mass(np.zeros((B, Hq, L, D)), k, bs, 0.25, "bf16")
    nblk = L // bs
    ref = np.zeros((nblk, nblk))
    for i in range(nblk):
        for t in range(bs):
            T = i * bs + t
            for j in range(i + 1):
                ref[i, j] += min(bs, T + 1 - j * bs) / (T + 1) / bs
    np.testing.assert_allclose(m0[0, 0], ref, rtol=0, atol=1e-15)
    # any input: each row of blocks sums to 1, zero above the diagonal
    q = rng.standard_normal((B, Hq, L, D))
    m = oattn.block_mass(q, k, bs, 0.25, "bf16")
    np.testing.assert_allclose(m.sum(-1), 1.0, atol=1e-12)
    assert np.all(np.triu(m[0, 0], 1) == 0)


def test_block_mass_matches_reference_loop_in_torch_cpu():
    # the capture_mass loop (src/eval_qwen_ppl.py:84-95) run by torch on the same bf16 data
    B, Hq, Hkv, L, D, bs, scaling = 1, 4, 2, 256, 32, 64, 0.2
    g = torch.Generator().manual_seed(8)
    q = torch.randn(B, Hq, L, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16)
    grp, nblk = Hq // Hkv, L // bs
    kr = k.repeat_interleave(grp, 1)
    kpos = torch.arange(L)
    ablk = torch.zeros(B, Hq, nblk, nblk)
    for i in range(nblk):
        qi = q[:, :, i * bs:(i + 1) * bs, :]
        s = (qi @ kr.transpose(-1, -2)) * scaling
        qpos = i * bs + torch.arange(bs)
        s = s.float().masked_fill(kpos[None, None, None, :] > qpos[None, None, :, None], float("-inf"))
        ablk[:, :, i, :] = s.softmax(-1).view(B, Hq, bs, nblk, bs).sum(-1).mean(2)
    ref = ablk.view(B, Hkv, grp, nblk, nblk).mean(2).double().numpy()
    got = oattn.block_mass(q.double().numpy(), k.double().numpy(), bs, scaling, "bf16")
    # fp32 softmax and torch's fp32 accumulator vs exact products: a bf16 score may sit one ulp apart
    np.testing.assert_allclose(got, ref, atol=2e-4)
    assert np.abs(got - ref).mean() < 5e-6
