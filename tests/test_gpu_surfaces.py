"""GPU tests of the reference-compatible surfaces: ``triton_kernel``,
``ssa_model.BlockSparseSSA`` and ``qwen_blocksparse`` (drop-ins for the
reference's modules of the same names), against the CPU oracle and the
reference's own closed-form checks."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attn as oattn, select as osel
from _util import randn, np64, assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print("[surface]", *a, flush=True)


# ---------------------------------------------------------------- triton_kernel
def test_triton_kernel_forward_backward_match_oracle():
    import triton_kernel as tk
    g = torch.Generator().manual_seed(0)
    B, H, N, D, bs, kk = 2, 2, 512, 64, 32, 5
    nblk = N // bs
    q, k, v, do = (randn(g, (B, H, N, D), "bf16") for _ in range(4))
    rnd = torch.randint(0, nblk, (B, nblk, kk - 1), generator=g)
    sel = torch.cat([torch.arange(nblk).view(1, nblk, 1).expand(B, nblk, 1), rnd], -1)
    gate = F.logsigmoid(torch.randn(B, nblk, kk, generator=g))
    for causal in (False, True):
        _say("bsattn_forward/backward causal", causal)
        mask = "slot_causal" if causal else "none"
        o = tk.bsattn_forward(q.to(DEV), k.to(DEV), v.to(DEV), sel.to(DEV), gate.to(DEV), causal=causal)
        ro, _ = oattn.fwd(np64(q), np64(k), np64(v), sel.numpy()[:, None], mask, gate=gate.numpy()[:, None])
        assert o.dtype == q.dtype and o.shape == q.shape
        assert_close(np64(o), ro, "bf16", "o")
        dq, dk, dv = tk.bsattn_backward(q.to(DEV), k.to(DEV), v.to(DEV), sel.to(DEV), o, do.to(DEV),
                                        gate.to(DEV), causal=causal)
        r = oattn.bwd(np64(q), np64(k), np64(v), sel.numpy()[:, None], np64(do), mask, gate=gate.numpy()[:, None])
        for n, a, b in (("dq", dq, r[0]), ("dk", dk, r[1]), ("dv", dv, r[2])):
            assert_close(np64(a), b, "bf16", n)


def test_triton_kernel_rejects_bad_length():
    import triton_kernel as tk
    q = torch.zeros(1, 1, 100, 64, dtype=torch.bfloat16, device=DEV)
    sel = torch.zeros(1, 3, 1, dtype=torch.int32, device=DEV)
    with pytest.raises(AssertionError):
        tk.bsattn_forward(q, q, q, sel)


# ---------------------------------------------------------------- ssa_model
def test_blocksparse_all_blocks_equals_dense_gate():
    # the reference's correctness gate (scripts/run_all.sh:7-21), on the GPU
    from ssa_model import BlockSparseSSA, DenseAttention
    torch.manual_seed(0)
    B, L, D, H = 2, 512, 128, 4
    x = torch.randn(B, L, D, device=DEV)
    sp = BlockSparseSSA(D, H, block=64, topk=10_000, sel_dim=16).to(DEV)
    dn = DenseAttention(D, H).to(DEV)
    dn.qkv.load_state_dict(sp.qkv.state_dict())
    dn.o.load_state_dict(sp.o.state_dict())
    with torch.no_grad():
        diff = (dn(x) - sp(x)).abs().max().item()
    _say("max|dense - sparse(all blocks)| =", diff)
    assert diff < 1e-3
    # causal, topk >= nblk-1 (every past block) == causal dense
    sp.causal, dn.causal = True, True
    with torch.no_grad():
        diff = (dn(x) - sp(x)).abs().max().item()
    _say("causal: max|dense - sparse(all blocks)| =", diff)
    assert diff < 1e-3
    # more blocks than the streaming top-k holds: own + every other block
    sp = BlockSparseSSA(D, H, block=16, topk=10_000, sel_dim=16, causal=True, gate=False).to(DEV)
    dn = DenseAttention(D, H, causal=True).to(DEV)
    dn.qkv.load_state_dict(sp.qkv.state_dict())
    dn.o.load_state_dict(sp.o.state_dict())
    x = torch.randn(1, 16 * 80, D, device=DEV)
    with torch.no_grad():
        diff = (dn(x) - sp(x)).abs().max().item()
    _say("nblk=80 causal: max|dense - sparse(all blocks)| =", diff)
    assert diff < 1e-3


def _module_oracle(m, x):
    """The reference module's computation restated on the oracle: q,k,v and the
    pooled selector features come from the module's own layers (torch, GPU);
    selection, gate and attention from the oracle; output projection in fp64."""
    B, L, D = x.shape
    Bs, H, dh = m.block, m.h, m.dh
    nblk = L // Bs
    dt = osel.__dict__  # noqa: F841
    name = {torch.float32: "f32", torch.bfloat16: "bf16"}[x.dtype]
    with torch.no_grad():
        q, k, v = (t.view(B, L, H, dh).transpose(1, 2) for t in m.qkv(x).chunk(3, -1))
        sq, skm, skx = m._pooled(x, B, nblk, Bs)
    raw = osel.scores(np64(sq), np64(skm), name, "max2", b2=np64(skx))
    sel = osel.select_conv_a(raw, m.topk, m.causal)
    gate = None
    if m.gate:
        from oracle.numerics import round_to
        gate = round_to(osel.gate_from_scores(raw, sel), name)[:, None]
    o, _ = oattn.fwd(np64(q), np64(k), np64(v), sel[:, None], "slot_causal" if m.causal else "none", gate=gate)
    o = o.transpose(0, 2, 1, 3).reshape(B, L, D)
    W, b = np64(m.o.weight), np64(m.o.bias)
    return o @ W.T + b, sel


@pytest.mark.parametrize("causal,gate", [(True, True), (False, False), (True, False)])
def test_blocksparse_module_matches_oracle(causal, gate):
    # verify_kernel.py's "small" case shape: d256 h4 B2 L1024 block64 top-4, bf16
    from ssa_model import BlockSparseSSA
    torch.manual_seed(0)
    m = BlockSparseSSA(256, 4, block=64, topk=4, causal=causal, gate=gate).to(DEV).to(torch.bfloat16).eval()
    x = torch.randn(2, 1024, 256, device=DEV, dtype=torch.bfloat16)
    _say("module", causal, gate)
    with torch.no_grad():
        m.use_triton = False
        a = m(x)
        m.use_triton = True
        b = m(x)
    assert torch.equal(a, b)
    ref, _ = _module_oracle(m, x)
    assert_close(np64(a), ref, "bf16", "module out")


@pytest.mark.parametrize("dtype,L,autocast", [("bf16", 1024, False), ("bf16", 1000, True), ("f32", 512, False)])
def test_blocksparse_distill_target_matches_oracle(dtype, L, autocast):
    # self-distillation target (src/ssa_model.py:140-149): dense causal softmax of
    # the module's own q, k summed per key block, averaged over each query
    # block's rows and the heads; 16-bit models take the fused block-mass kernel
    from ssa_model import BlockSparseSSA
    torch.manual_seed(4)
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    m = BlockSparseSSA(256, 4, block=64, topk=3, causal=True).to(DEV).to(tdt)
    m.distill = True
    x = torch.randn(1, L, 256, device=DEV, dtype=tdt)
    _say("distill", dtype, L, autocast)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        m(x)
        Lp = (L + 63) // 64 * 64
        xp = F.pad(x, (0, 0, 0, Lp - L))
        q, k, _ = (t.view(1, Lp, 4, 64).transpose(1, 2) for t in m.qkv(xp).chunk(3, -1))
    tgt = m.distill_target
    assert tgt.shape == (1, Lp // 64, Lp // 64)
    assert tgt.dtype == (torch.float32 if autocast or dtype == "f32" else tdt)
    ref = oattn.block_mass(np64(q), np64(k), 64, 64 ** -0.5, "f32" if q.dtype == torch.float32 else "bf16")
    ref = ref.mean(1)
    atol = 5e-5 if tgt.dtype == torch.float32 else 4e-3  # a bf16 target carries its own rounding
    np.testing.assert_allclose(np64(tgt), ref, atol=atol, rtol=0)
    np.testing.assert_allclose(np64(tgt).sum(-1), 1.0, atol=atol * 64)
    assert m.distill_logits.shape == tgt.shape


def _slot_module_oracle(m, x, slots, gval, causal):
    """Attention over routed slots on the oracle: q, k, v from the module's
    own projection (torch); empty places (-1) removed by a -inf gate; with
    m.gate, logsigmoid of the slot scores added; output projection in fp64."""
    B, L, D = x.shape
    H, dh = m.h, m.dh
    with torch.no_grad():
        q, k, v = (t.view(B, L, H, dh).transpose(1, 2) for t in m.qkv(x).chunk(3, -1))
    valid = slots >= 0
    gate = np.where(valid, 0.0, -np.inf)
    if m.gate:
        gate = gate + np.where(valid, -np.logaddexp(0.0, -np.asarray(gval, dtype=np.float64)), 0.0)
    o, _ = oattn.fwd(np64(q), np64(k), np64(v), np.maximum(slots, 0)[:, None], "slot_causal" if causal else "none",
                     gate=gate[:, None])
    o = o.transpose(0, 2, 1, 3).reshape(B, L, D)
    return o @ np64(m.o.weight).T + np64(m.o.bias)


@pytest.mark.parametrize("gate,refine", [(False, None), (True, None), (True, 3)])
def test_centroid_module_matches_oracle(gate, refine):
    # CentroidSSA (src/ssa_model.py:204-336): O(nblk*C) routing, non-causal attention
    from ssa_model import CentroidSSA
    torch.manual_seed(5)
    B, L, d, h, Bs, s = 2, 1024, 128, 2, 32, 16
    m = CentroidSSA(d, h, block=Bs, sel_dim=s, n_centroids=6, cpq=2, cap=3, gate=gate, refine_topk=refine).to(DEV)
    x = torch.randn(B, L, d, device=DEV)
    _say("centroid", gate, refine)
    with torch.no_grad():
        out = m(x, needle_pos=torch.tensor([100, 900], device=DEV))
        nblk = L // Bs
        sq = m.sel_q(x).view(B, nblk, Bs, s).mean(2)
        kf = m.sel_k(x).view(B, nblk, Bs, s)
        sk = torch.maximum(kf.mean(2), kf.max(2).values)
        q, k, _ = (t.view(B, L, h, d // h).transpose(1, 2) for t in m.qkv(x).chunk(3, -1))
        qm = q.reshape(B, h, nblk, Bs, -1).mean(3).mean(1)
        km = k.reshape(B, h, nblk, Bs, -1).mean(3).mean(1)
    slots, qc, kc, home = osel.centroid_route(np64(sq), np64(sk), np64(m.cent), 2, 3, refine, np64(qm), np64(km))
    gval = np.take_along_axis(qc, home[np.arange(B)[:, None], np.maximum(slots, 0).reshape(B, -1)].reshape(
        slots.shape), 2)
    assert_close(np64(out), _slot_module_oracle(m, x, slots, gval, False), "f32", "centroid out")
    assert m.last_block_logits.shape == (B, nblk) and m.align_q.shape == (B, 6)
    assert m.last_hit is not None


def test_centroid_module_single_centroid_is_dense():
    # the reference's exactness check (src/ssa_model.py:212): one centroid, one
    # route, capacity >= nblk selects every block, i.e. dense non-causal attention
    from ssa_model import CentroidSSA
    torch.manual_seed(6)
    m = CentroidSSA(128, 2, block=32, sel_dim=16, n_centroids=1, cpq=1, cap=64).to(DEV)
    x = torch.randn(1, 1024, 128, device=DEV)
    with torch.no_grad():
        out = m(x)
        q, k, v = (t.view(1, 1024, 2, 64).transpose(1, 2) for t in m.qkv(x).chunk(3, -1))
        ref = m.o(F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(1, 1024, 128))
    assert_close(np64(out), np64(ref), "f32", "centroid dense")


@pytest.mark.parametrize("causal,gate,dense", [(False, True, False), (True, True, False), (True, False, True),
                                               (False, True, True)])
def test_lsh_module_matches_oracle(causal, gate, dense):
    # LSHBucketSSA (src/ssa_model.py:339-513): bucketed (eval) or dense (train) selection
    from ssa_model import LSHBucketSSA
    torch.manual_seed(7)
    B, L, d, h, Bs, s, topk = 2, 1024, 128, 2, 32, 16, 4
    m = LSHBucketSSA(d, h, block=Bs, topk=topk, sel_dim=s, n_rounds=3, n_buckets=4, cap=4, gate=gate,
                     causal=causal).to(DEV)
    m.dense_select = dense
    x = torch.randn(B, L, d, device=DEV)
    _say("lsh", causal, gate, dense)
    with torch.no_grad():
        out = m(x, needle_pos=torch.tensor([50, 700], device=DEV))
        nblk = L // Bs
        sq = F.normalize(m.sel_q(x).view(B, nblk, Bs, s).mean(2), dim=-1)
        kf = m.sel_k(x).view(B, nblk, Bs, s)
        sk = F.normalize(torch.maximum(kf.mean(2), kf.max(2).values), dim=-1)
    if dense:
        slots, gval = osel.lsh_dense(np64(sq), np64(sk), m.scale, causal, topk)
    else:
        slots, gval = osel.lsh_route(np64(sq), np64(sk), np64(m.R), 4, m.scale, causal, topk)
    assert_close(np64(out), _slot_module_oracle(m, x, slots, gval, causal), "f32", "lsh out")
    assert m.last_block_logits.shape == (B, nblk) and m.last_hit is not None


def test_routed_modules_train_their_selectors():
    # gradients reach the centroids (through the gate) and the learned hash planes
    from ssa_model import CentroidSSA, LSHBucketSSA
    torch.manual_seed(8)
    x = torch.randn(1, 512, 128, device=DEV)
    c = CentroidSSA(128, 2, block=32, sel_dim=16, n_centroids=4, cpq=2, cap=4, gate=True).to(DEV)
    c(x).square().sum().backward()
    assert c.cent.grad is not None and c.cent.grad.abs().sum() > 0 and c.qkv.weight.grad.abs().sum() > 0
    lsh = LSHBucketSSA(128, 2, block=32, topk=3, sel_dim=16, gate=True, causal=True, learn_hash=True).to(DEV)
    lsh.dense_select = True
    lsh.train()
    out = lsh(x)
    assert lsh.last_hash_loss is not None and torch.isfinite(lsh.last_hash_loss)
    (out.square().sum() + lsh.last_hash_loss).backward()
    assert lsh.R.grad is not None and lsh.R.grad.abs().sum() > 0
    assert lsh.sel_q[0].weight.grad.abs().sum() > 0


def test_tiny_transformer_centroid_align_trains_centroids():
    # TinyTransformer.centroid_align (src/ssa_model.py:560-562) hands train.py
    # (src/train.py:56-63) one (align_q, align_k_all) pair per CentroidSSA
    # layer; the InfoNCE routing loss built from them reaches the centroids
    from ssa_model import TinyTransformer
    torch.manual_seed(3)
    B, L, blk = 2, 512, 32
    nblk = L // blk
    m = TinyTransformer(64, 10, d=128, h=2, layers=2, max_len=L, attn="centroid",
                        block=blk, sel_dim=16, n_centroids=4, cpq=2, cap=4).to(DEV)
    toks = torch.randint(0, 64, (B, L), device=DEV)
    npos = torch.tensor([37, 300], device=DEV)
    assert m.centroid_align() == []                   # nothing stashed before a needle pass
    m(toks, needle_pos=npos)
    aligns = m.centroid_align()
    assert len(aligns) == 2
    tau, nb = 0.5, (npos // blk).long()
    loss = 0.0
    for aq, ak_all in aligns:
        assert aq.shape == (B, 4) and ak_all.shape == (B, nblk, 4)
        q_dist = F.softmax(aq.float() / tau, -1)
        k_dist = F.softmax(ak_all.float() / tau, -1)
        sim = (q_dist.unsqueeze(1) * k_dist).sum(-1) / tau
        loss = loss + F.cross_entropy(sim, nb)
    loss.backward()
    for b in m.blocks:
        g = b["attn"].cent.grad
        assert g is not None and torch.isfinite(g).all() and g.abs().sum() > 0


def test_blocksparse_gate_gradient_paths():
    # gather path (use_triton=False) trains the selector through the gate; the
    # fused op (use_triton=True) returns no gate gradient (src/triton_kernel.py:254)
    from ssa_model import BlockSparseSSA
    torch.manual_seed(1)
    m = BlockSparseSSA(128, 2, block=32, topk=3, causal=True, gate=True).to(DEV)
    x = torch.randn(2, 512, 128, device=DEV, requires_grad=True)
    m.use_triton = False
    m(x).square().sum().backward()
    gq = m.sel_q[0].weight.grad
    assert gq is not None and gq.abs().sum() > 0 and m.qkv.weight.grad.abs().sum() > 0
    m.zero_grad(set_to_none=True)
    m.use_triton = True
    m(x).square().sum().backward()
    assert m.sel_q[0].weight.grad is None and m.qkv.weight.grad.abs().sum() > 0


def test_blocksparse_gate_gradient_matches_finite_difference():
    # d(loss)/d(selector params) through logsigmoid(raw[i, sel]) on the fused backward, fp32
    from ssa_model import BlockSparseSSA
    torch.manual_seed(2)
    # a bias on the key-side selector output shifts every block's pooled mean
    # and max alike, so the selected blocks do not change under the perturbation
    m = BlockSparseSSA(64, 2, block=16, topk=2, sel_dim=16, causal=True, gate=True).to(DEV)
    x = torch.randn(1, 128, 64, device=DEV)
    w = torch.randn(1, 128, 64, device=DEV)
    loss = lambda: (m(x).double() * w.double()).sum()  # noqa: E731
    loss().backward()
    p = m.sel_k[2].bias
    gp = p.grad.clone()
    eps = 5e-2
    for idx in range(4):
        with torch.no_grad():
            p[idx] += eps
            lp = loss().item()
            p[idx] -= 2 * eps
            lm = loss().item()
            p[idx] += eps
        num = (lp - lm) / (2 * eps)
        _say("fd", idx, num, gp[idx].item())
        assert abs(num - gp[idx].item()) <= 2e-2 * max(1.0, abs(num))


def test_blocksparse_padding_and_needle_hooks():
    from ssa_model import BlockSparseSSA
    torch.manual_seed(3)
    m = BlockSparseSSA(128, 2, block=64, topk=2, causal=True).to(DEV)
    x = torch.randn(2, 1000, 128, device=DEV)          # L % block != 0: zero-padded like the reference
    with torch.no_grad():
        y = m(x, needle_pos=torch.tensor([5, 900], device=DEV))
    assert y.shape == x.shape and torch.isfinite(y).all()
    assert m.last_block_logits.shape == (2, 16)
    assert 0.0 <= m.last_hit <= 1.0
    xp = F.pad(x, (0, 0, 0, 24))
    ref, sel = _module_oracle(m, xp)
    assert_close(np64(y), ref[:, :1000], "f32", "padded module out")


# ---------------------------------------------------------------- qwen_blocksparse
def _ref_sdpa(q, k, v, causal=True):
    grp = q.shape[1] // k.shape[1]
    return F.scaled_dot_product_attention(q.float(), k.repeat_interleave(grp, 1).float(),
                                          v.repeat_interleave(grp, 1).float(), is_causal=causal)


@pytest.mark.parametrize("L", [256, 200])
def test_qwen_fastpath_matches_sdpa(L):
    from qwen_blocksparse import blocksparse_forward
    torch.manual_seed(0)
    B, Hq, Hkv, d = 1, 16, 2, 64
    q, k, v = torch.randn(B, Hq, L, d, device=DEV), torch.randn(B, Hkv, L, d, device=DEV), torch.randn(B, Hkv, L, d, device=DEV)
    for causal in (True, False):
        out = blocksparse_forward(q, k, v, selector=None, topk=9999, bs=32, causal=causal)
        assert out.shape == (B, Hq, L, d)
        assert torch.allclose(out, _ref_sdpa(q, k, v, causal), atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("L", [192, 200])
def test_qwen_gather_allcausal_matches_sdpa(L):
    from qwen_blocksparse import blocksparse_forward, SelectAll
    torch.manual_seed(0)
    B, Hq, Hkv, d = 1, 8, 2, 48
    q, k, v = torch.randn(B, Hq, L, d, device=DEV), torch.randn(B, Hkv, L, d, device=DEV), torch.randn(B, Hkv, L, d, device=DEV)
    out = blocksparse_forward(q, k, v, selector=SelectAll(bs=32), topk=0, bs=32, causal=True, q_chunk=3)
    assert out.shape == (B, Hq, L, d)
    assert torch.allclose(out, _ref_sdpa(q, k, v), atol=1e-3, rtol=1e-3)


def test_qwen_selectors_causal_and_budget():
    from qwen_blocksparse import SelectMax, SelectOracle, SelectRandom, blocksparse_forward
    torch.manual_seed(0)
    B, Hq, Hkv, L, d = 1, 16, 2, 256, 64
    q, k, v = torch.randn(B, Hq, L, d, device=DEV), torch.randn(B, Hkv, L, d, device=DEV), torch.randn(B, Hkv, L, d, device=DEV)
    nblk = L // 32
    qb = torch.arange(nblk, device=DEV).view(1, 1, nblk, 1)
    for S in (SelectMax(topk=4, bs=32, sink=True), SelectRandom(topk=4, bs=32, sink=True, seed=1)):
        idx = S.select(q, k)
        assert idx.shape == (B, Hkv, nblk, 6) and (idx <= qb).all() and (idx >= 0).all()
        assert (idx == 0).any(-1).all() and (idx == qb).any(-1).all()
        assert torch.equal(idx, idx.sort(-1).values)
        out = blocksparse_forward(q, k, v, selector=S, topk=4, bs=32, q_chunk=2)
        assert out.shape == (B, Hq, L, d) and torch.isfinite(out).all()
    mass = torch.rand(B, Hkv, 8, 8, device=DEV) * 0.01
    mass[..., 0] = 1.0
    idx = SelectOracle(topk=1, bs=32, sink=False).select_from_mass(mass)
    assert (idx == 0).any(-1).all()


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_qwen_selectmax_forward_matches_oracle_with_outgate(dtype):
    # config-4-like: GQA 8/2, d128, bs64, Quest top-6 + own + sink, padded L, output gate
    from qwen_blocksparse import blocksparse_forward, SelectMax
    g = torch.Generator().manual_seed(4)
    B, Hq, Hkv, L, d, bs, topk = 1, 8, 2, 1000, 128, 64, 6
    q, og = randn(g, (B, Hq, L, d), dtype), randn(g, (B, Hq, L, d), dtype)
    k, v = randn(g, (B, Hkv, L, d), dtype), randn(g, (B, Hkv, L, d), dtype)
    S = SelectMax(topk=topk, bs=bs, sink=True)
    idx = S.select(q.to(DEV), k.to(DEV)).cpu().numpy()
    Lp = 1024
    pad = lambda t: np.pad(np64(t), ((0, 0), (0, 0), (0, Lp - L), (0, 0)))  # noqa: E731
    ref_idx, _ = osel.select_quest(pad(q), pad(k), bs, topk, True, dtype)
    assert np.array_equal(idx, ref_idx)
    out = blocksparse_forward(q.to(DEV), k.to(DEV), v.to(DEV), selector=S, topk=topk, bs=bs, scale=0.1,
                              out_gate=og.to(DEV))
    ro, _ = oattn.fwd(pad(q), pad(k), pad(v), ref_idx, "token_causal", scale=0.1, L_valid=L, out_gate=pad(og))
    assert_close(np64(out), ro[:, :, :L], dtype, "out")


@pytest.mark.parametrize("L,d,dtype", [(2048, 64, "bf16"), (2000, 128, "bf16"), (1024, 64, "f32")])
def test_qwen_select_lasttok_matches_oracle(L, d, dtype):
    # SelectLastTok (src/qwen_blocksparse.py:244-264): Quest score of each block's
    # last-token group mean; the ragged block's last token is zero padding
    from qwen_blocksparse import SelectLastTok
    g = torch.Generator().manual_seed(21)
    B, Hq, Hkv, bs, topk = 1, 8, 2, 64, 6
    q, k = randn(g, (B, Hq, L, d), dtype), randn(g, (B, Hkv, L, d), dtype)
    _say("lasttok", L, d, dtype)
    idx = SelectLastTok(topk=topk, bs=bs, sink=True).select(q.to(DEV), k.to(DEV)).cpu().numpy()
    ref, _ = osel.select_quest_lasttok(np64(q), np64(k), bs, topk, True, dtype)
    assert idx.shape == ref.shape and np.array_equal(idx, ref)


@pytest.mark.parametrize("minmax", [False, True])
@pytest.mark.parametrize("sel_dim,dtype", [(64, "bf16"), (32, "bf16"), (64, "f32")])
def test_qwen_select_learned_matches_oracle(minmax, sel_dim, dtype):
    # SelectLearned / SelectLearnedMinMax (src/qwen_blocksparse.py:168-213): pooled
    # features (checked against the oracle's pools) projected by torch as in the
    # reference, then the streaming top-k of scale * sq.sk^T. With sel_dim 64 the
    # default scale is 1/8 (exact); with 32 it rounds, and may merge neighbouring
    # scores into exact ties, where the chosen score multiset must still agree.
    from fbsa_amd import selection
    from qwen_blocksparse import SelectLearned, SelectLearnedMinMax
    g = torch.Generator().manual_seed(22)
    B, Hq, Hkv, L, d, bs, topk = 1, 8, 2, 4096, 64, 64, 8
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    q, k = randn(g, (B, Hq, L, d), dtype).to(DEV), randn(g, (B, Hkv, L, d), dtype).to(DEV)
    Wq = (torch.randn(d, sel_dim, generator=g) / 8).to(tdt).to(DEV)
    Wk = (torch.randn(2 * d if minmax else d, sel_dim, generator=g) / 8).to(tdt).to(DEV)
    S = (SelectLearnedMinMax if minmax else SelectLearned)(Wq, Wk, topk=topk, bs=bs, sink=True)
    _say("learned", minmax, sel_dim, dtype)
    idx = S.select(q, k).cpu().numpy()
    qpool = selection.pool(q, bs, "mean_grp_then_tok", grp=Hq // Hkv)
    np.testing.assert_array_equal(np64(qpool), osel.pool_mean_grp_then_tok(np64(q), Hkv, bs, dtype))
    if minmax:
        kmin, kmax = selection.pool(k, bs, "minmax")
        kfeat = torch.cat([kmin, kmax], -1)
        omin, omax = osel.pool_minmax(np64(k), bs)
        np.testing.assert_array_equal(np64(kfeat), np.concatenate([omin, omax], -1))
    else:
        kfeat = selection.pool(k, bs, "mean_tok_then_grp", grp=1)
        np.testing.assert_array_equal(np64(kfeat), osel.pool_mean_tok(np64(k), bs, dtype))
    sq, sk = np64(qpool @ Wq), np64(kfeat @ Wk)
    ref, sc, _ = osel.select_learned_features(sq, sk, topk, True, dtype, S.scale)
    if sel_dim == 64:
        assert np.array_equal(idx, ref)
    else:
        got_sc = np.sort(np.take_along_axis(sc, idx, -1), -1)
        ref_sc = np.sort(np.take_along_axis(sc, ref, -1), -1)
        assert np.array_equal(got_sc, ref_sc)
        assert (idx == ref).all(-1).mean() > 0.9


@pytest.mark.parametrize("dtype,L,d,bs", [("bf16", 512, 64, 64), ("bf16", 1024, 256, 128),
                                          ("f16", 512, 128, 64), ("bf16", 768, 64, 128)])
def test_qwen_block_mass_matches_oracle(dtype, L, d, bs):
    # the true block mass of capture_mass (src/eval_qwen_ppl.py:84-95) on the fused kernel
    from qwen_blocksparse import SelectOracle, block_mass
    g = torch.Generator().manual_seed(23)
    B, Hq, Hkv, scale = 1, 4, 2, 0.1
    q, k = randn(g, (B, Hq, L, d), dtype), randn(g, (B, Hkv, L, d), dtype)
    _say("block mass", dtype, L, d, bs)
    got = block_mass(q.to(DEV), k.to(DEV), bs, scale)
    ref = oattn.block_mass(np64(q), np64(k), bs, scale, dtype)
    m = got.cpu().numpy().astype(np.float64)
    assert m.shape == ref.shape
    assert np.all(np.triu(m, 1) == 0)
    np.testing.assert_allclose(m.sum(-1), 1.0, atol=1e-4)
    np.testing.assert_allclose(m, ref, atol=5e-5)
    assert np.abs(m - ref).mean() < 2e-6
    # SelectOracle on it (src/qwen_blocksparse.py:124-137)
    topk = 3
    idx = SelectOracle(topk=topk, bs=bs, sink=True, mass=got).select(None, None).cpu().numpy()
    ridx = osel.select_conv_b(ref, topk, True)
    assert (idx == ridx).all(-1).mean() > 0.97  # rows apart only at near-equal masses


@pytest.mark.parametrize("which", ["ssa", "lsh", "lsh_dense", "qwen"])
def test_causal_modules_do_not_leak(which):
    # src/check_lsh_causal.py: perturbing the inputs from block p on must leave
    # every output before position p unchanged (here: bit for bit)
    from ssa_model import BlockSparseSSA, LSHBucketSSA
    from qwen_blocksparse import SelectMax, blocksparse_forward
    torch.manual_seed(9)
    d, h, B, L, block = 128, 4, 2, 1024, 32
    if which == "qwen":
        q, k, v = (torch.randn(B, s, L, 64, device=DEV, dtype=torch.bfloat16) for s in (8, 2, 2))

        def run(qq, kk_, vv):
            return blocksparse_forward(qq, kk_, vv, selector=SelectMax(topk=4, bs=block), topk=4, bs=block)
    else:
        m = (BlockSparseSSA(d, h, block=block, topk=4, causal=True, gate=True) if which == "ssa" else
             LSHBucketSSA(d, h, block=block, topk=4, causal=True, gate=True)).to(DEV).eval()
        m.dense_select = which == "lsh_dense"
        x = torch.randn(B, L, d, device=DEV)
    for pb in (L // block - 1, L // block // 2, 3):
        p = pb * block
        _say("leak", which, pb)
        with torch.no_grad():
            if which == "qwen":
                o1 = run(q, k, v)
                q2, k2, v2 = q.clone(), k.clone(), v.clone()
                for t in (q2, k2, v2):
                    t[:, :, p:] += 3.0
                o2 = run(q2, k2, v2)
                before, after = o1[:, :, :p], o2[:, :, :p]
                changed = (o1[:, :, p:] - o2[:, :, p:]).abs().max()
            else:
                o1 = m(x)
                x2 = x.clone()
                x2[:, p:] += 10.0
                o2 = m(x2)
                before, after = o1[:, :p], o2[:, :p]
                changed = (o1[:, p:] - o2[:, p:]).abs().max()
        assert torch.equal(before, after), f"{which}: outputs before block {pb} changed"
        assert changed > 0


def test_blocksparse_module_large_nblk():
    # src/verify_kernel.py's large case: d64 h2 L=1,120,000 block 16 -> nblk 70000
    # (> 65535), top-2, causal, gated, bf16; sampled query blocks against the oracle
    from ssa_model import BlockSparseSSA
    from oracle.numerics import round_to
    torch.manual_seed(0)
    d, h, B, L, Bs, topk = 64, 2, 1, 70000 * 16, 16, 2
    m = BlockSparseSSA(d, h, block=Bs, topk=topk, causal=True, gate=True).to(DEV).to(torch.bfloat16).eval()
    x = torch.randn(B, L, d, device=DEV, dtype=torch.bfloat16)
    nblk, dh = L // Bs, d // h
    _say("large nblk")
    with torch.no_grad():
        out = m(x)
        q, k, v = (t.view(B, L, h, dh).transpose(1, 2) for t in m.qkv(x).chunk(3, -1))
        sq, skm, skx = m._pooled(x, B, nblk, Bs)
    assert torch.isfinite(out.float()).all()
    rows = np.array([0, 1, 2, 5, 65534, 65535, 65536, 69999])
    raw = osel.scores(np64(sq), np64(skm), "bf16", "max2", b2=np64(skx), rows=rows)   # (B, R, nblk)
    sel_r = osel.select_conv_a(raw, topk, True, rows=rows)                              # (B, R, kk)
    gate_r = round_to(osel.gate_from_scores(raw, sel_r), "bf16")
    kk = sel_r.shape[-1]
    sel = np.tile(np.arange(nblk)[None, :, None], (B, 1, kk))
    gate = np.zeros((B, nblk, kk))
    sel[:, rows], gate[:, rows] = sel_r, gate_r
    o, _ = oattn.fwd(np64(q), np64(k), np64(v), sel[:, None], "slot_causal", gate=gate[:, None], rows=rows)
    o = o.reshape(B, h, len(rows), Bs, dh).transpose(0, 2, 3, 1, 4).reshape(B, len(rows) * Bs, d)
    ref = o @ np64(m.o.weight).T + np64(m.o.bias)
    pos = (rows[:, None] * Bs + np.arange(Bs)[None, :]).ravel()
    assert_close(np64(out[:, pos]), ref, "bf16", "large-nblk out")
