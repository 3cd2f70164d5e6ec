"""GPU parity: pooling and streaming selection (libfbsa.so) vs the CPU oracle.

Block indices must match bit for bit (ties break to the lower index in both);
pooled values must match exactly (same rounding points)."""
import numpy as np
import pytest
import torch

from oracle import select as osel
from _util import randn, np64

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print("[select]", *a, flush=True)


@pytest.mark.parametrize("dtype,H,D,bs", [("f32", 4, 64, 64), ("bf16", 4, 64, 64), ("f16", 4, 64, 64),
                                          ("bf16", 6, 64, 64), ("bf16", 12, 64, 64), ("f16", 13, 64, 64),
                                          ("f32", 1, 64, 64), ("bf16", 1, 64, 64), ("f16", 1, 64, 64),
                                          ("f32", 1, 256, 128), ("bf16", 1, 128, 32), ("f16", 1, 16, 16),
                                          ("bf16", 1, 32, 128)])
def test_pool_mean_tok_then_heads_exact(dtype, H, D, bs):
    """Mean over tokens, then over H heads. A wave takes heads w, w + 4, ... and
    loads two of them together: 6, 12 and 13 heads leave waves with an odd count.
    One head (a plain token mean) runs one block per wave, four per workgroup,
    at every head dim and block size it takes."""
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(0)
    B, N = 2, 1000                               # N % bs != 0: zero-padded tail block
    x = randn(g, (B, H, N, D), dtype)
    _say("pool mean_tok_then_grp", dtype, H)
    got = np64(selection.pool(x.to(DEV), bs, "mean_tok_then_grp", grp=H))
    ref = osel.pool_mean_tok_then_heads(np64(x), bs, dtype)[:, None]
    assert np.array_equal(got, ref), np.abs(got - ref).max()


@pytest.mark.parametrize("op,H,grp,D,bs", [("mean_tok_then_grp", 2, 1, 64, 64), ("mean_tok_then_grp", 4, 4, 64, 32),
                                           ("mean_grp_then_tok", 4, 2, 128, 128), ("minmax", 2, 1, 32, 16)])
def test_pool_l_valid_past_whole_blocks(op, H, grp, D, bs):
    """Tokens at positions >= l_valid count as zeros, also in blocks that lie
    wholly past l_valid (their rows are read at the last valid row's address
    and discarded): the result equals pooling the input with those rows zeroed."""
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(7)
    B, N, lv = 2, 1000, 77                       # blocks from lv // bs + 1 on hold no valid token
    x = randn(g, (B, H, N, D), "bf16")
    xz = x.clone()
    xz[:, :, lv:] = 0
    _say("pool l_valid", op, H, grp, D, bs)
    got = selection.pool(x.to(DEV), bs, op, grp=grp, l_valid=lv)
    if op == "minmax":
        rmin, rmax = osel.pool_minmax(np64(xz), bs)
        assert np.array_equal(np64(got[0]), rmin) and np.array_equal(np64(got[1]), rmax)
        return
    if op == "mean_tok_then_grp":
        ref = np.concatenate([osel.pool_mean_tok_then_heads(np64(xz[:, h0:h0 + grp]), bs, "bf16")[:, None]
                              for h0 in range(0, H, grp)], axis=1)
    else:
        ref = osel.pool_mean_grp_then_tok(np64(xz), H // grp, bs, "bf16")
    assert np.array_equal(np64(got), ref), np.abs(np64(got) - ref).max()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_pool_quest_exact(dtype):
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(1)
    B, Hq, Hkv, N, D, bs = 1, 8, 2, 700, 128, 128
    q = randn(g, (B, Hq, N, D), dtype)
    k = randn(g, (B, Hkv, N, D), dtype)
    _say("pool quest", dtype)
    qp = np64(selection.pool(q.to(DEV), bs, "mean_grp_then_tok", grp=Hq // Hkv))
    kmin, kmax = selection.pool(k.to(DEV), bs, "minmax")
    assert np.array_equal(qp, osel.pool_mean_grp_then_tok(np64(q), Hkv, bs, dtype))
    rmin, rmax = osel.pool_minmax(np64(k), bs)
    assert np.array_equal(np64(kmin), rmin) and np.array_equal(np64(kmax), rmax)


def _check_sel(got, ref, what):
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"{what}: {len(bad)} mismatching slots, first at {bad[:3].tolist()}: " \
                          f"got {got[tuple(bad[0][:-1])]} ref {ref[tuple(bad[0][:-1])]}"


@pytest.mark.parametrize("engine", ["auto", "fp64"])
@pytest.mark.parametrize("dtype,B,H,N,bs,topk,causal", [
    ("f32", 1, 4, 4096, 64, 8, True),      # config 1
    ("bf16", 32, 8, 1024, 32, 4, True),    # config 2
    ("bf16", 1, 2, 8192, 16, 16, True),    # many blocks, small block
    ("bf16", 2, 2, 2048, 64, 5, False),    # non-causal
    ("f16", 1, 2, 2048, 32, 12, True),
])
def test_select_mean_pooled_exact(dtype, B, H, N, bs, topk, causal, engine):
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(2)
    D = 64
    q, k = (randn(g, (B, H, N, D), dtype) for _ in range(2))
    _say("mean-pooled", dtype, B, H, N, bs, topk, causal, engine)
    sel, sc = selection.select_mean_pooled(q.to(DEV), k.to(DEV), bs, topk, causal, need_scores=True, engine=engine)
    ref, raw = osel.select_mean_pooled(np64(q), np64(k), bs, topk, causal, dtype)
    _check_sel(sel.cpu().numpy(), ref, "sel")
    ref_sc = np.take_along_axis(raw, ref, axis=-1)
    assert np.array_equal(sc.cpu().numpy().astype(np.float64), ref_sc)


@pytest.mark.parametrize("dtype,B,Hq,Hk,N,D,bs,topk,scale", [
    ("bf16", 1, 8, 8, 16384, 64, 64, 16, 1.0),     # config 3's shape, shorter
    ("bf16", 2, 4, 2, 3000, 64, 32, 32, 1.0),      # ragged tail block, largest fused budget
    ("bf16", 2, 4, 2, 3000, 64, 32, 48, 1.0),      # past it: pool, pool, fp64 select
    ("f16", 1, 2, 1, 2048, 32, 16, 8, 1.0),
    ("bf16", 1, 2, 2, 4096, 64, 128, 20, 1.0),
    ("bf16", 1, 4, 4, 4096, 64, 64, 49, 1.0),      # budget past the MFMA engine: pool, pool, select
    ("bf16", 1, 2, 2, 4096, 64, 64, 16, 1e19),     # norms past 1e18: every pair takes the exact path
    ("bf16", 1, 2, 2, 4096, 32, 64, 16, 1e-20),    # norms below 2^-40: likewise
    ("bf16", 3, 1, 1, 3000, 64, 32, 16, 1.0),      # one head: plain token means, a block per wave
    ("f16", 1, 1, 1, 4000, 32, 128, 8, 1.0),
])
def test_select_mean_pooled_fused_equals_separate_calls(dtype, B, Hq, Hk, N, D, bs, topk, scale):
    """fbsa_select_mean_pooled (q and k pooled by one launch that also writes the
    selection's row norms) against fbsa_pool twice + fbsa_select: same blocks,
    same chosen-slot scores."""
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(31)
    q = (randn(g, (B, Hq, N, D), "f32") * scale).to(getattr(torch, {"bf16": "bfloat16", "f16": "float16"}[dtype]))
    k = (randn(g, (B, Hk, N, D), "f32") * scale).to(q.dtype)
    q, k = q.to(DEV), k.to(DEV)
    _say("mean-pooled fused vs separate", dtype, B, Hq, Hk, N, D, bs, topk, scale)
    sel1, sc1 = selection.select_mean_pooled(q, k, bs, topk, True, need_scores=True)
    qp = selection.pool(q, bs, "mean_tok_then_grp", grp=Hq)
    kp = selection.pool(k, bs, "mean_tok_then_grp", grp=Hk)
    sel2, sc2 = selection.select(qp, kp, score="dot", convention="own_first", topk=topk, causal=True,
                                 need_scores=True)
    torch.cuda.synchronize()
    assert torch.equal(sel1, sel2[:, 0])
    assert torch.equal(sc1, sc2[:, 0])


def test_select_config3_full_size_sampled_rows():
    # config 3: B1 H8 N262144 D64 bs64 top-16; q,k ~ N(0,1)/8 in bf16. The oracle
    # pools the full tensors and scores a sample of rows (each row i depends
    # only on qpool[i] and kpool[0..i]).
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(0)
    B, H, N, D, bs, topk = 1, 8, 262144, 64, 64, 16
    q = randn(g, (B, H, N, D), "bf16", scale=0.125)
    k = randn(g, (B, H, N, D), "bf16", scale=0.125)
    _say("config 3 selection")
    sel = selection.select_mean_pooled(q.to(DEV), k.to(DEV), bs, topk, True).cpu().numpy()
    qp = osel.pool_mean_tok_then_heads(np64(q), bs, "bf16")
    kp = osel.pool_mean_tok_then_heads(np64(k), bs, "bf16")
    rows = np.unique(np.concatenate([np.arange(0, 40), np.arange(4096 - 40, 4096),
                                     np.random.default_rng(0).integers(0, 4096, 200)]))
    raw = osel.scores(qp, kp, "bf16", "dot", rows=rows)
    ref = osel.select_conv_a(raw, topk, True, rows=rows)
    _check_sel(sel[:, rows], ref, "sel (sampled rows)")


@pytest.mark.parametrize("dtype,engine", [("bf16", "auto"), ("bf16", "fp64"), ("f32", "auto")])
def test_select_quest_config4_shape(dtype, engine):
    # config 4 selector: Hq16 Hkv2 D256 bs128 nblk512 top-32 + own + sink
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, N, D, bs, topk = 1, 16, 2, 65536, 256, 128, 32
    q = randn(g, (B, Hq, N, D), dtype)
    k = randn(g, (B, Hkv, N, D), dtype)
    _say("quest config 4", dtype, engine)
    idx = selection.select_quest(q.to(DEV), k.to(DEV), bs, topk, sink=True, engine=engine).cpu().numpy()
    ref, _ = osel.select_quest(np64(q), np64(k), bs, topk, True, dtype)
    _check_sel(idx, ref, "idx")


@pytest.mark.parametrize("D,ties,sink,topk", [(128, False, True, 8), (256, True, True, 62), (128, True, False, 30),
                                               (256, False, False, 16)])
def test_select_quest_wide_rows(D, ties, sink, topk):
    # Quest + _finish at D >= 128 without chosen-slot scores runs on the row-per-
    # workgroup exact kernel; with scores requested, on the streaming fp64 kernel:
    # both must give the oracle's blocks
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(9)
    B, H, nblk = 1, 2, 700
    if ties:
        mk = lambda: torch.randint(-2, 3, (B, H, nblk, D), generator=g).to(torch.bfloat16)  # noqa: E731
    else:
        mk = lambda: randn(g, (B, H, nblk, D), "bf16")  # noqa: E731
    a, b1, b2 = mk(), mk(), mk()
    b1, b2 = torch.maximum(b1, b2), torch.minimum(b1, b2)
    _say("quest wide", D, ties, sink, topk)
    kw = dict(score="quest", convention="sorted_sink", topk=topk, sink=sink)
    sel = selection.select(a.to(DEV), b1.to(DEV), b2.to(DEV), **kw)
    sel2, _ = selection.select(a.to(DEV), b1.to(DEV), b2.to(DEV), need_scores=True, **kw)
    raw = osel.scores(np64(a), np64(b1), "bf16", "quest", b2=np64(b2))
    ref = osel.select_conv_b(raw, topk, sink)
    _check_sel(sel.cpu().numpy(), ref, "sel (row kernel)")
    _check_sel(sel2.cpu().numpy(), ref, "sel (streaming kernel)")


@pytest.mark.parametrize("engine", ["auto", "fp64"])
def test_select_max2_module_scores(engine):
    # BlockSparseSSA._scores: max(sq . sk_mean, sq . sk_max) (src/ssa_model.py:113-119)
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(4)
    B, L, S, bs, topk = 2, 2048, 32, 64, 8
    sq = randn(g, (B, 1, L, S), "bf16")
    sk = randn(g, (B, 1, L, S), "bf16")
    _say("max2")
    a = selection.pool(sq.to(DEV), bs, "mean_tok_then_grp")
    km = selection.pool(sk.to(DEV), bs, "mean_tok_then_grp")
    kx = selection.pool(sk.to(DEV), bs, "max")
    sel, sc = selection.select(a, km, kx, score="max2", topk=topk, causal=True, need_scores=True, engine=engine)
    ra = osel.pool_tok(np64(sq)[:, 0], bs, "bf16", "mean")
    rkm = osel.pool_tok(np64(sk)[:, 0], bs, "bf16", "mean")
    rkx = osel.pool_tok(np64(sk)[:, 0], bs, "bf16", "max")
    raw = osel.scores(ra, rkm, "bf16", "max2", b2=rkx)
    ref = osel.select_conv_a(raw, topk, True)
    _check_sel(sel.cpu().numpy()[:, 0], ref, "sel")
    assert np.array_equal(sc.cpu().numpy()[:, 0].astype(np.float64), np.take_along_axis(raw, ref, -1))


@pytest.mark.parametrize("engine", ["auto", "fp64"])
@pytest.mark.parametrize("nblk,topk,conv", [(1, 4, "own_first"), (3, 8, "own_first"), (5, 0, "own_first"),
                                            (1, 4, "sorted_sink"), (4, 9, "sorted_sink"), (70, 62, "own_first"),
                                            (200, 62, "sorted_sink")])
def test_select_edge_budgets(nblk, topk, conv, engine):
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(5)
    a = randn(g, (1, 2, nblk, 32), "bf16")
    b = randn(g, (1, 2, nblk, 32), "bf16")
    _say("edge", nblk, topk, conv)
    sel = selection.select(a.to(DEV), b.to(DEV), topk=topk, convention=conv, sink=conv == "sorted_sink",
                           engine=engine).cpu().numpy()
    raw = osel.scores(np64(a), np64(b), "bf16", "dot")
    if conv == "own_first":
        ref = np.stack([osel.select_conv_a(raw[:, h], topk, True) for h in range(2)], 1)
    else:
        ref = osel.select_conv_b(raw, topk, True)
    _check_sel(sel, ref, "sel")


@pytest.mark.parametrize("D", [16, 64])
def test_select_ties_break_to_lower_index(D):
    # all-equal scores: every candidate ties; lowest indices must win
    from fbsa_amd import selection
    nblk, topk = 200, 7
    a = torch.ones(1, 1, nblk, D, dtype=torch.bfloat16)
    sel = selection.select(a.to(DEV), a.to(DEV), topk=topk, causal=True).cpu().numpy()[0, 0]
    for i in range(nblk):
        want = [i] + [j for j in range(min(i, topk))] + [i] * max(0, topk - i)
        assert sel[i].tolist() == want, (i, sel[i])


def test_select_config5_prefix_invariance_and_sampled_rows():
    # config 5: B1 H8 D64 N4194304 bs64 (nblk 65536) top-16. The streaming selection
    # on the full sequence must give the 262144-token prefix run's blocks for the
    # first 4096 rows (causal), and the oracle's blocks on sampled later rows.
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(5)
    B, H, N, D, bs, topk = 1, 8, 4194304, 64, 64, 16
    q = randn(g, (B, H, N, D), "bf16")
    k = randn(g, (B, H, N, D), "bf16")
    _say("config 5 selection")
    qd, kd = q.to(DEV), k.to(DEV)
    sel = selection.select_mean_pooled(qd, kd, bs, topk, True).cpu().numpy()
    pre = selection.select_mean_pooled(qd[:, :, :262144].contiguous(), kd[:, :, :262144].contiguous(),
                                       bs, topk, True).cpu().numpy()
    _check_sel(sel[:, :4096], pre, "prefix rows")
    qp = selection.pool(qd, bs, "mean_tok_then_grp", grp=H)[:, 0].float().cpu().numpy().astype(np.float64)
    kp = selection.pool(kd, bs, "mean_tok_then_grp", grp=H)[:, 0].float().cpu().numpy().astype(np.float64)
    rows = np.unique(np.concatenate([np.arange(65536 - 8, 65536),
                                     np.random.default_rng(1).integers(4096, 65536, 40)]))
    raw = osel.scores(qp, kp, "bf16", "dot", rows=rows)
    ref = osel.select_conv_a(raw, topk, True, rows=rows)
    _check_sel(sel[:, rows], ref, "sampled rows")


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("score", ["dot", "max2", "quest"])
@pytest.mark.parametrize("conv,causal,topk", [("own_first", True, 16), ("own_first", False, 16),
                                              ("sorted_sink", True, 16), ("own_first", True, 32),
                                              ("own_first", True, 48)])
@pytest.mark.parametrize("ties,chunk", [(False, 0), (True, 0), (False, 4), (True, 1)])
def test_select_tiled_modes(dtype, D, score, conv, causal, topk, ties, chunk):
    # The MFMA engine over every score mode / convention / width it takes, with
    # nblk = 700 (11 candidate tiles, a ragged last tile). chunk > 0 splits the
    # candidates of a row block over several workgroups (partial lists + merge).
    # ties=True uses small integer operands, so scores are exact integers with
    # many exact ties (tie-break and exact-bracket paths).
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(6)
    B, H, nblk = 1, 2, 700
    if ties:
        mk = lambda: torch.randint(-2, 3, (B, H, nblk, D), generator=g).to(getattr(torch, {"bf16": "bfloat16", "f16": "float16"}[dtype]))
    else:
        mk = lambda: randn(g, (B, H, nblk, D), dtype)
    a, b1, b2 = mk(), mk(), mk()
    if score == "quest":  # kmax >= kmin element-wise, as the pooled operands are
        b1, b2 = torch.maximum(b1, b2), torch.minimum(b1, b2)
    _say("tiled", dtype, D, score, conv, causal, topk, ties, chunk)
    sink = conv == "sorted_sink"
    sel, sc = selection.select(a.to(DEV), b1.to(DEV), b2.to(DEV) if score != "dot" else None, score=score,
                               convention=conv, topk=topk, causal=causal, sink=sink, need_scores=True,
                               chunk_tiles=chunk)
    raw = osel.scores(np64(a), np64(b1), dtype, score, b2=np64(b2))
    if conv == "own_first":
        ref = np.stack([osel.select_conv_a(raw[:, h], topk, causal) for h in range(H)], 1)
    else:
        ref = osel.select_conv_b(raw, topk, sink)
    _check_sel(sel.cpu().numpy(), ref, "sel")
    assert np.array_equal(sc.cpu().numpy().astype(np.float64), np.take_along_axis(raw, ref, -1))


@pytest.mark.parametrize("dtype,score,conv,causal,topk,nblk,ties", [
    ("bf16", "dot", "own_first", True, 64, 900, False),
    ("bf16", "dot", "own_first", True, 128, 900, True),
    ("bf16", "dot", "own_first", False, 63, 300, False),
    ("f32", "dot", "own_first", True, 128, 600, False),
    ("bf16", "max2", "own_first", True, 100, 700, False),
    ("bf16", "dot", "sorted_sink", True, 64, 900, True),
    ("f16", "quest", "sorted_sink", True, 128, 700, False),
    ("bf16", "dot", "sorted_sink", True, 700, 700, False),
    ("bf16", "quest", "sorted_sink", True, 300, 1200, True),
])
def test_select_wide_budgets(dtype, score, conv, causal, topk, nblk, ties):
    # top-k budgets past one wave-wide list (> 62): one workgroup per row with
    # its keys in LDS; blocks and chosen-slot scores bit-exact against the oracle
    # (src/ssa_model.py:158-161 and src/qwen_blocksparse.py:90 take any topk)
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(31)
    B, H, D = 1, 2, 64
    if ties:
        mk = lambda: torch.randint(-2, 3, (B, H, nblk, D), generator=g).to(torch.bfloat16 if dtype == "bf16" else torch.float16 if dtype == "f16" else torch.float32)  # noqa: E731
    else:
        mk = lambda: randn(g, (B, H, nblk, D), dtype)  # noqa: E731
    a, b1, b2 = mk(), mk(), mk()
    if score == "quest":
        b1, b2 = torch.maximum(b1, b2), torch.minimum(b1, b2)
    _say("wide", dtype, score, conv, causal, topk, nblk, ties)
    sel, sc = selection.select(a.to(DEV), b1.to(DEV), None if score == "dot" else b2.to(DEV), score=score,
                               convention=conv, topk=topk, causal=causal, sink=conv == "sorted_sink",
                               need_scores=True)
    raw = osel.scores(np64(a), np64(b1), dtype, score, b2=None if score == "dot" else np64(b2))
    if conv == "own_first":
        ref = np.stack([osel.select_conv_a(raw[:, h], topk, causal) for h in range(H)], 1)
    else:
        ref = osel.select_conv_b(raw, topk, True)
    _check_sel(sel.cpu().numpy(), ref, "sel")
    assert np.array_equal(sc.cpu().numpy().astype(np.float64), np.take_along_axis(raw, ref, -1))


def test_select_quest_topk_100_config4_rows():
    # SelectMax with a budget of 100 at D 256 (the row-per-workgroup Quest kernel)
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(32)
    B, Hq, Hkv, N, D, bs, topk = 1, 4, 2, 128 * 300, 256, 128, 100
    q = randn(g, (B, Hq, N, D), "bf16")
    k = randn(g, (B, Hkv, N, D), "bf16")
    idx = selection.select_quest(q.to(DEV), k.to(DEV), bs, topk, sink=True).cpu().numpy()
    ref, _ = osel.select_quest(np64(q), np64(k), bs, topk, True, "bf16")
    _check_sel(idx, ref, "idx")
