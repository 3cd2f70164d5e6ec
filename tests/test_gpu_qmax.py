"""GPU parity of the row-block max Quest selection (``fbsa_select_qmax``):
``SelectMaxQMax`` and ``SelectTwoStage`` (``src/qwen_blocksparse.py:216-241``,
``:267-299``) against the CPU oracle, bit-exact block indices (ties to the
lower block index). Both engines are checked: MFMA brackets with exact
resolution ("auto") and float64 for every score ("fp64")."""
import time

import numpy as np
import pytest
import torch

from oracle import select as osel
from _util import randn, np64

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print("[qmax]", *a, flush=True)


def _inputs(seed, B, Hq, Hkv, L, D, dtype, ties=False):
    g = torch.Generator().manual_seed(seed)
    q, k = randn(g, (B, Hq, L, D), dtype), randn(g, (B, Hkv, L, D), dtype)
    if ties:
        # values in {-1/4, 0, 1/4}: many exactly equal scores
        q = (torch.round(q.float().clamp(-1, 1)) / 4).to(q.dtype)
        k = (torch.round(k.float().clamp(-1, 1)) / 4).to(k.dtype)
    return q, k


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_pool_token_group_mean_matches_oracle(dtype):
    from fbsa_amd import selection
    q, _ = _inputs(40, 2, 8, 2, 999, 64, dtype)
    _say("pool bs=1", dtype)
    got = selection.pool(q.to(DEV), 1, "mean_grp_then_tok", grp=4)
    np.testing.assert_array_equal(np64(got), osel.pool_grp_mean_tok(np64(q), 2, dtype))


# (B, Hq, Hkv, L, D, bs, topk, sink, dtype, ties)
QMAX_CASES = [
    (1, 8, 2, 4096, 256, 128, 6, True, "bf16", False),     # the Qwen shape class (tok 128, D 256)
    (2, 4, 2, 2000, 128, 64, 5, False, "bf16", False),     # ragged last block
    (1, 2, 1, 3072, 64, 64, 8, True, "f16", False),
    (1, 4, 4, 1024, 32, 128, 3, True, "bf16", False),
    (1, 4, 2, 2048, 64, 64, 7, True, "bf16", True),        # exact ties everywhere
    (1, 2, 2, 1024, 128, 64, 40, True, "bf16", False),     # topk > nblk: every block
    (1, 4, 2, 1000, 64, 32, 4, True, "bf16", False),       # bs 32: float64 engine only
    (1, 2, 1, 1024, 64, 64, 5, True, "f32", False),        # fp32 operands: float64 engine
]


@pytest.mark.parametrize("case", QMAX_CASES, ids=lambda c: "-".join(map(str, c)))
def test_select_qmax_matches_oracle(case):
    from fbsa_amd import selection
    B, Hq, Hkv, L, D, bs, topk, sink, dtype, ties = case
    q, k = _inputs(41, B, Hq, Hkv, L, D, dtype, ties)
    ref, _ = osel.select_quest_qmax(np64(q), np64(k), bs, topk, sink, dtype)
    for engine in ("auto", "fp64"):
        _say("qmax", case, engine)
        got = selection.select_quest_qmax(q.to(DEV), k.to(DEV), bs, topk, sink=sink, engine=engine)
        assert got.dtype == torch.int32 and tuple(got.shape) == ref.shape
        np.testing.assert_array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("case", [(1, 8, 2, 4096, 128, 64, 6, 4, "bf16", False),
                                  (1, 8, 2, 4096, 256, 128, 4, 4, "bf16", False),
                                  (2, 4, 2, 1900, 64, 64, 5, 2, "f16", False),
                                  (1, 4, 2, 2048, 64, 64, 6, 3, "bf16", True),
                                  (1, 2, 1, 1024, 64, 64, 3, 1, "f32", False)],
                         ids=lambda c: "-".join(map(str, c)))
def test_select_two_stage_matches_oracle(case):
    from fbsa_amd import selection
    B, Hq, Hkv, L, D, bs, topk, over, dtype, ties = case
    q, k = _inputs(42, B, Hq, Hkv, L, D, dtype, ties)
    ref, _, _ = osel.select_two_stage(np64(q), np64(k), bs, topk, True, over, dtype)
    for engine in ("auto", "fp64"):
        _say("two-stage", case, engine)
        got = selection.select_two_stage(q.to(DEV), k.to(DEV), bs, topk, sink=True, over=over, engine=engine)
        np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_qwen_selector_classes():
    from qwen_blocksparse import SelectMaxQMax, SelectTwoStage, blocksparse_forward
    q, k = _inputs(43, 1, 8, 2, 2048, 128, "bf16")
    v = randn(torch.Generator().manual_seed(44), (1, 2, 2048, 128), "bf16")
    bs, topk = 64, 5
    for S, ref in ((SelectMaxQMax(topk=topk, bs=bs), osel.select_quest_qmax(np64(q), np64(k), bs, topk, True, "bf16")[0]),
                   (SelectTwoStage(topk=topk, bs=bs, over=3),
                    osel.select_two_stage(np64(q), np64(k), bs, topk, True, 3, "bf16")[0])):
        _say("class", type(S).__name__)
        idx = S.select(q.to(DEV), k.to(DEV))
        assert idx.dtype == torch.long
        np.testing.assert_array_equal(idx.cpu().numpy(), ref)
        out = blocksparse_forward(q.to(DEV), k.to(DEV), v.to(DEV), selector=S, topk=topk, bs=bs)
        assert out.shape == q.shape and torch.isfinite(out.float()).all()


def test_select_qmax_candidate_list_rules():
    # candidate rows with repeats and entries outside [0, i]: those are skipped
    from fbsa_amd import selection
    q, k = _inputs(45, 1, 2, 1, 1024, 64, "bf16")
    bs, topk = 64, 3
    qg = selection.pool(q.to(DEV), 1, "mean_grp_then_tok", grp=2)
    kmin, kmax = selection.pool(k.to(DEV), bs, "minmax")
    nblk = kmax.shape[2]
    rng = np.random.default_rng(0)
    cand = np.sort(rng.integers(-3, nblk + 3, size=(1, 1, nblk, 9)), axis=-1).astype(np.int32)
    _say("candidate rules")
    got = selection.select_qmax(qg, kmax, kmin, bs, topk=topk, cand=torch.from_numpy(cand).to(DEV)).cpu().numpy()
    qgo = osel.pool_grp_mean_tok(np64(q), 1, "bf16")
    omin, omax = osel.pool_minmax(np64(k), bs)
    listed = np.zeros((nblk, nblk), dtype=bool)
    for i in range(nblk):
        c = cand[0, 0, i]
        listed[i, c[(c >= 0) & (c <= i)]] = True
    assert not listed.any(-1).all()  # some rows list no valid block
    sc = np.where(listed[None, None], osel.scores_qmax(qgo, omax, omin, bs, "bf16"), -np.inf)
    np.testing.assert_array_equal(got, osel.select_conv_b(sc, topk, True))


@pytest.mark.parametrize("two_stage", [False, True])
def test_select_qmax_f16_overflow(two_stage):
    # fp16 scores past 65504 round to inf (and inf - inf to NaN), as torch's fp16
    # einsums make them; NaN ranks first and non-finite picks become the own block
    from fbsa_amd import selection
    q, k = _inputs(47, 1, 4, 2, 2048, 128, "f16")
    # every third key block large (its scores overflow to inf), block 7 large
    # and positive (its min is large too: inf - inf = NaN), the rest moderate
    kf = k.float().view(1, 2, 32, 64, 128)
    scale = torch.full((32,), 8.0)
    scale[::3] = 30.0
    kf = kf * scale.view(1, 1, 32, 1, 1)
    kf[:, :, 7] = kf[:, :, 7].abs() + 100
    q, k = (q.float() * 16).half(), kf.view(1, 2, 2048, 128).half()
    if two_stage:
        ref, sc, _ = osel.select_two_stage(np64(q), np64(k), 64, 5, True, 2, "f16")
    else:
        ref, sc = osel.select_quest_qmax(np64(q), np64(k), 64, 5, True, "f16")
    past = np.arange(32)[None, :] <= np.arange(32)[:, None]
    assert np.isinf(sc[..., past]).any() and np.isnan(sc[..., past]).any() and np.isfinite(sc[..., past]).any()
    for engine in ("auto", "fp64"):
        _say("f16 overflow", two_stage, engine)
        fn = selection.select_two_stage if two_stage else selection.select_quest_qmax
        kw = dict(over=2) if two_stage else {}
        got = fn(q.to(DEV), k.to(DEV), 64, 5, sink=True, engine=engine, **kw)
        np.testing.assert_array_equal(got.cpu().numpy(), ref)


def test_select_qmax_full_qwen_shape_properties():
    # configuration-4 shape (L 65536, Hq 16, Hkv 2, D 256, bs 128, top-32): the
    # two engines agree, and rows of a causal prefix do not depend on the rest
    from fbsa_amd import selection
    g = torch.Generator(device=DEV).manual_seed(46)
    B, Hq, Hkv, L, D, bs, topk = 1, 16, 2, 65536, 256, 128, 32
    q = torch.randn(B, Hq, L, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, Hkv, L, D, generator=g, device=DEV).to(torch.bfloat16)
    _say("qwen shape auto")
    a = selection.select_quest_qmax(q, k, bs, topk)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        a = selection.select_quest_qmax(q, k, bs, topk)
    torch.cuda.synchronize()
    _say(f"SelectMaxQMax at the config-4 shape: {(time.perf_counter() - t0) / 3 * 1e3:.2f} ms per call")
    _say("qwen shape fp64")
    f = selection.select_quest_qmax(q, k, bs, topk, engine="fp64")
    assert torch.equal(a, f)
    _say("qwen shape prefix")
    n = 16384
    p = selection.select_quest_qmax(q[:, :, :n].contiguous(), k[:, :, :n].contiguous(), bs, topk)
    assert torch.equal(a[:, :, :n // bs], p)
    _say("qwen shape two-stage")
    t = selection.select_two_stage(q, k, bs, topk, over=4)
    t64 = selection.select_two_stage(q, k, bs, topk, over=4, engine="fp64")
    assert torch.equal(t, t64)
    # the first over*topk rows have every past block as a candidate
    assert torch.equal(t[:, :, :4 * topk], a[:, :, :4 * topk])


def test_select_qmax_8192_columns():
    # the largest row the kernel takes (nblk 8192: 1M tokens at block 128, here
    # 512K at block 64): rows of the 262144-token prefix match the prefix run,
    # and sampled late rows match the oracle row by row
    from fbsa_amd import selection
    g = torch.Generator(device=DEV).manual_seed(48)
    B, Hq, Hkv, L, D, bs, topk = 1, 2, 1, 524288, 64, 64, 16
    q = torch.randn(B, Hq, L, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B, Hkv, L, D, generator=g, device=DEV).to(torch.bfloat16)
    _say("8192 columns")
    full = selection.select_quest_qmax(q, k, bs, topk)
    n = 262144
    pre = selection.select_quest_qmax(q[:, :, :n].contiguous(), k[:, :, :n].contiguous(), bs, topk)
    assert torch.equal(full[:, :, :n // bs], pre)
    qg = np64(selection.pool(q, 1, "mean_grp_then_tok", grp=2))
    kmin, kmax = (np64(t) for t in selection.pool(k, bs, "minmax"))
    got = full.cpu().numpy()
    for i in (4096, 6000, 8191):
        tok = osel.scores(qg[:, :, i * bs:(i + 1) * bs], kmax, "bf16", "quest", b2=kmin)  # (B,H,bs,nblk)
        row = tok.max(axis=2)[:, :, None, :]
        ref = osel.select_conv_b(row, topk, True, rows=[i])
        np.testing.assert_array_equal(got[:, :, i:i + 1], ref)
