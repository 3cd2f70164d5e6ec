"""Pins for the selection oracle (CPU).

* rounding helpers against torch's own dtype conversions;
* pooling against closed forms (constant blocks, min <= x <= max) and torch's
  CPU reductions (``view(...).mean(3).mean(1)``, ``src/ssa_model.py:287-288``;
  ``src/qwen_blocksparse.py:113-116``);
* the Quest bound (``src/qwen_blocksparse.py:8-10``);
* conventions A and B against brute-force per-row sorting and against
  torch.topk / sort on tie-free scores (the reference's own routines,
  ``src/ssa_model.py:151-165``, ``src/qwen_blocksparse.py:87-99``);
* budget/causality invariants and the planted-mass check
  (``src/test_qwen_blocksparse.py:37-71``);
* causal-prefix invariance and the near-tie census.
"""
import numpy as np
import pytest
import torch

from oracle import numerics as on, select as osel

RNG = np.random.default_rng(0)


# ---------------------------------------------------------------- numerics
def test_round_bf16_matches_torch():
    x = np.concatenate([RNG.standard_normal(100000) * 10.0 ** RNG.integers(-8, 4, 100000),
                        # exact bf16 midpoints (ties to even) and their neighbours
                        (np.arange(1, 2000, dtype=np.float32) * 2 ** -7 + 2 ** -8) * 3.0])
    x32 = x.astype(np.float32)
    ref = torch.from_numpy(x32).to(torch.bfloat16).float().numpy().astype(np.float64)
    np.testing.assert_array_equal(on.round_bf16(x32.astype(np.float64)), ref)
    ref16 = torch.from_numpy(x32).to(torch.float16).float().numpy().astype(np.float64)
    np.testing.assert_array_equal(on.round_f16(x32.astype(np.float64)), ref16)
    np.testing.assert_array_equal(on.round_f32(x), x.astype(np.float32).astype(np.float64))


def test_round_bf16_double_rounding_point():
    # torch rounds an fp32 accumulator; a float64 value just above a bf16
    # midpoint that rounds to the midpoint in fp32 must then tie to even
    mid = 1.0 + 2 ** -8                   # midpoint between 1 and 1 + 2^-7
    x = mid + 2 ** -40                    # rounds to exactly `mid` in fp32
    assert on.round_bf16(np.array([x]))[0] == 1.0
    assert on.round_bf16(np.array([mid + 2 ** -20]))[0] == 1.0 + 2 ** -7


# ---------------------------------------------------------------- pooling
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_pool_mean_matches_torch_cpu(dtype):
    tdt = {"bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    B, H, N, D, bs = 2, 4, 512, 32, 64
    x = torch.randn(B, H, N, D, generator=torch.Generator().manual_seed(1)).to(tdt)
    ref = x.view(B, H, N // bs, bs, D).mean(3).mean(1).double().numpy()
    got = osel.pool_mean_tok_then_heads(x.double().numpy(), bs, dtype)
    # torch's CPU accumulator may differ from the exact sum in the last fp32 bits;
    # a different bf16 result is only possible at a rounding midpoint (1 ulp)
    ref2 = x.view(B, 2, 2, N // bs, bs, D).mean(2).mean(3).double().numpy()   # SelectMax's order
    got2 = osel.pool_mean_grp_then_tok(x.double().numpy(), 2, bs, dtype)
    for g_, r_ in ((got, ref), (got2, ref2)):
        if dtype == "bf16":
            diff = g_ != r_
            assert diff.mean() < 2e-3
            ulp = 2.0 ** (np.floor(np.log2(np.abs(r_[diff]))) - 7)
            assert np.all(np.abs(g_[diff] - r_[diff]) <= ulp)
        else:
            # the oracle is the exactly rounded mean; torch's fp32 accumulator is within a few ulps
            np.testing.assert_allclose(g_, r_, rtol=4e-7 * 64, atol=1e-8)


@pytest.mark.parametrize("N", [512, 500])
def test_pool_last_token_and_token_mean_match_torch_cpu(N):
    # the reference's expressions (src/qwen_blocksparse.py:259, :183) on the same bf16 data
    B, Hq, Hkv, D, bs = 2, 4, 2, 32, 64
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, Hq, N, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, N, D, generator=g).to(torch.bfloat16)
    nblk = (N + bs - 1) // bs
    qp = torch.nn.functional.pad(q, (0, 0, 0, nblk * bs - N))
    kp = torch.nn.functional.pad(k, (0, 0, 0, nblk * bs - N))
    ref_last = qp.view(B, Hkv, Hq // Hkv, nblk, bs, D).mean(2)[:, :, :, -1, :].double().numpy()
    ref_mean = kp.view(B, Hkv, nblk, bs, D).mean(3).double().numpy()
    got_last = osel.pool_last_token_grp(q.double().numpy(), Hkv, bs, "bf16")
    got_mean = osel.pool_mean_tok(k.double().numpy(), bs, "bf16")
    # a 2-term group mean is exact in fp32 before the bf16 rounding: identical
    np.testing.assert_array_equal(got_last, ref_last)
    if N % bs:
        assert np.all(got_last[:, :, -1] == 0)  # the ragged block's last token is padding
    diff = got_mean != ref_mean  # a 64-term fp32 sum may round differently at a bf16 midpoint
    assert diff.mean() < 2e-3
    ulp = 2.0 ** (np.floor(np.log2(np.abs(ref_mean[diff]))) - 7)
    assert np.all(np.abs(got_mean[diff] - ref_mean[diff]) <= ulp)


def test_learned_scale_rounding_and_order():
    # a positive scale keeps the order of rnd(sq.sk); it can only merge neighbours
    # into exact ties (then the lower index wins); scale = 1/8 changes nothing
    rng = np.random.default_rng(3)
    sq = on.round_bf16(rng.standard_normal((1, 1, 40, 32)))
    sk = on.round_bf16(rng.standard_normal((1, 1, 40, 32)))
    idx8, sc8, raw = osel.select_learned_features(sq, sk, 6, True, "bf16", 0.125)
    np.testing.assert_array_equal(sc8, raw * 0.125)
    np.testing.assert_array_equal(idx8, osel.select_conv_b(raw, 6, True))
    idx3, sc3, _ = osel.select_learned_features(sq, sk, 6, True, "bf16", 3 ** -0.5)
    assert np.all(np.diff(np.sort(sc3.ravel())) >= 0)
    order_ok = (np.sign(np.subtract.outer(raw.ravel(), raw.ravel())) * np.sign(np.subtract.outer(sc3.ravel(), sc3.ravel()))) >= 0
    assert order_ok.all()  # no inversions, only merges


def test_pool_closed_forms():
    B, H, N, D, bs = 1, 2, 96, 8, 32
    c = RNG.standard_normal((B, H, N // bs, 1, D))
    x = np.broadcast_to(c, (B, H, N // bs, bs, D)).reshape(B, H, N, D)
    x = on.round_bf16(x)
    pm = osel.pool_mean_tok_then_heads(x, bs, "bf16")
    np.testing.assert_array_equal(pm, on.round_bf16(x.reshape(B, H, -1, bs, D)[:, :, :, 0].mean(1)))
    k = RNG.standard_normal((B, H, N, D))
    kmin, kmax = osel.pool_minmax(k, bs)
    kb = k.reshape(B, H, N // bs, bs, D)
    assert np.all(kmin[:, :, :, None] <= kb) and np.all(kb <= kmax[:, :, :, None])
    assert np.all((kb == kmin[:, :, :, None]).any(3)) and np.all((kb == kmax[:, :, :, None]).any(3))
    # zero padding takes part (src/qwen_blocksparse.py:112-116)
    kmin2, kmax2 = osel.pool_minmax(k[:, :, :80], bs)
    assert np.all(kmin2[:, :, 2] <= 0) and np.all(kmax2[:, :, 2] >= 0)
    tk = torch.from_numpy(k)
    np.testing.assert_array_equal(kmax, tk.view(B, H, -1, bs, D).max(3).values.numpy())


def test_quest_score_upper_bounds_token_products():
    B, Hq, Hkv, N, D, bs = 1, 4, 2, 128, 16, 16
    q = RNG.standard_normal((B, Hq, N, D))
    k = RNG.standard_normal((B, Hkv, N, D))
    qpool = osel.pool_mean_grp_then_tok(q, Hkv, bs, "f32")
    kmin, kmax = osel.pool_minmax(k, bs)
    exact = (np.maximum(qpool, 0)[..., :, None, :] * kmax[..., None, :, :]
             + np.minimum(qpool, 0)[..., :, None, :] * kmin[..., None, :, :]).sum(-1)
    kb = k.reshape(B, Hkv, N // bs, bs, D)
    prod = np.einsum("bhid,bhjsd->bhijs", qpool, kb).max(-1)      # max_s qpool_i . k_s over block j
    assert np.all(exact >= prod - 1e-12)
    sc = osel.scores(qpool, kmax, "f32", "quest", b2=kmin)
    np.testing.assert_allclose(sc, exact, rtol=1e-6, atol=1e-6)


def test_scores_match_torch_matmul_rounding():
    a = on.round_bf16(RNG.standard_normal((2, 40, 32)))
    b = on.round_bf16(RNG.standard_normal((2, 40, 32)))
    ta, tb = (torch.from_numpy(x).to(torch.bfloat16) for x in (a, b))
    ref = (ta @ tb.transpose(-1, -2)).double().numpy()
    got = osel.scores(a, b, "bf16", "dot")
    assert (got != ref).mean() < 5e-3      # only accumulator-order midpoints may differ
    b2 = on.round_bf16(RNG.standard_normal((2, 40, 32)))
    ref2 = torch.maximum(ta @ tb.transpose(-1, -2), ta @ torch.from_numpy(b2).to(torch.bfloat16).transpose(-1, -2))
    assert (osel.scores(a, b, "bf16", "max2", b2=b2) != ref2.double().numpy()).mean() < 5e-3


# ---------------------------------------------------------------- conventions
def _brute_a(raw_row, i, topk, causal):
    nblk = len(raw_row)
    cand = [j for j in range(nblk) if j != i and (not causal or j < i)]
    cand.sort(key=lambda j: (-raw_row[j], j))
    kk_c = min(topk, nblk - 1)
    picks = cand[:kk_c]
    return [i] + picks + [i] * (kk_c - len(picks))


@pytest.mark.parametrize("causal", [True, False])
def test_convention_a_bruteforce_with_ties(causal):
    raw = np.round(RNG.standard_normal((2, 23, 23)) * 2) / 2     # many exact ties
    for topk in (0, 1, 5, 22, 40):
        sel = osel.select_conv_a(raw, topk, causal)
        for b in range(2):
            for i in range(23):
                assert sel[b, i].tolist() == _brute_a(raw[b, i], i, topk, causal)


@pytest.mark.parametrize("causal", [True, False])
def test_convention_a_matches_torch_topk(causal):
    # the reference's selection code path on tie-free scores
    nblk, topk = 50, 7
    raw = torch.from_numpy(RNG.standard_normal((3, nblk, nblk)))
    diag = torch.arange(nblk)
    content = raw.clone()
    content[:, diag, diag] = float("-inf")
    if causal:
        content = content.masked_fill((diag.view(nblk, 1) < diag.view(1, nblk)).unsqueeze(0), float("-inf"))
    sel_ref = torch.cat([diag.view(1, nblk, 1).expand(3, nblk, 1), content.topk(topk, dim=-1).indices], -1).numpy()
    sel = osel.select_conv_a(raw.numpy(), topk, causal)
    valid = np.isfinite(np.take_along_axis(content.numpy(), sel_ref, -1))
    valid[..., 0] = True
    np.testing.assert_array_equal(np.where(valid, sel, -1), np.where(valid, sel_ref, -1))


def test_convention_b_matches_torch_finish():
    B, H, nblk = 2, 3, 40
    score = torch.from_numpy(RNG.standard_normal((B, H, nblk, nblk)))
    for topk, sink in ((4, True), (4, False), (45, True)):
        ar = torch.arange(nblk)
        sc = score.masked_fill(ar.view(1, 1, nblk, 1) < ar.view(1, 1, 1, nblk), float("-inf"))
        k = min(topk, nblk)
        tv, ti = sc.topk(k, dim=-1)
        own = ar.view(1, 1, nblk, 1).expand(B, H, nblk, 1)
        ti = torch.where(torch.isfinite(tv), ti, own.expand_as(ti))
        parts = [ti, own] + ([torch.zeros(B, H, nblk, 1, dtype=torch.long)] if sink else [])
        ref = torch.cat(parts, -1).sort(-1).values.numpy()
        got = osel.select_conv_b(score.numpy(), topk, sink)
        np.testing.assert_array_equal(got, ref)


def test_convention_invariants_and_planted_mass():
    B, H, nblk = 1, 2, 16
    score = RNG.standard_normal((B, H, nblk, nblk))
    idx = osel.select_conv_b(score, 4, True)
    qb = np.arange(nblk)[None, None, :, None]
    assert idx.shape == (B, H, nblk, 6) and np.all(idx <= qb) and np.all(idx >= 0)
    assert np.all(np.diff(idx, axis=-1) >= 0) and np.all((idx == 0).any(-1)) and np.all((idx == qb).any(-1))
    mass = RNG.random((B, H, 8, 8)) * 0.01
    mass[..., 0] = 1.0
    assert np.all((osel.select_conv_b(mass, 1, False) == 0).any(-1))
    raw = RNG.standard_normal((B, nblk, nblk))
    sel = osel.select_conv_a(raw, 5, True)
    assert np.all(sel[..., 0] == np.arange(nblk))
    content = sel[..., 1:]
    rows = np.arange(nblk)[None, :, None]
    assert np.all((content < rows) | (content == rows))     # fills are the own block
    for i in range(6, nblk):                                 # enough past blocks: distinct, all past
        assert len(set(content[0, i].tolist())) == 5 and np.all(content[0, i] < i)


def test_causal_prefix_invariance():
    # rows i < n' depend only on blocks <= i: selection on a prefix equals the full run's rows
    q = RNG.standard_normal((1, 4, 64 * 40, 16))
    k = RNG.standard_normal((1, 4, 64 * 40, 16))
    full, _ = osel.select_mean_pooled(q, k, 64, 6, True, "bf16")
    pre, _ = osel.select_mean_pooled(q[:, :, :64 * 25], k[:, :, :64 * 25], 64, 6, True, "bf16")
    np.testing.assert_array_equal(full[:, :25], pre)
    rows = np.array([3, 17, 24])
    qp = osel.pool_mean_tok_then_heads(q, 64, "bf16")
    kp = osel.pool_mean_tok_then_heads(k, 64, "bf16")
    part = osel.select_conv_a(osel.scores(qp, kp, "bf16", "dot", rows=rows), 6, True, rows=rows)
    np.testing.assert_array_equal(part, full[:, rows])


def test_near_tie_census():
    score = np.array([[[5.0, 3.0, 3.0 + 1e-9, 1.0, 2.0]]])
    valid = np.ones_like(score, dtype=bool)
    assert osel.near_tie_rows(score, np.array([[[0, 1]]]), 2, valid)[0, 0]
    assert not osel.near_tie_rows(score, np.array([[[0, 4]]]), 2, valid)[0, 0]
    score2 = np.array([[[5.0, 3.0, 2.5, 1.0, 2.0]]])
    assert not osel.near_tie_rows(score2, np.array([[[0, 1]]]), 2, valid)[0, 0]


# ---------------------------------------------------------------- token-max Quest (SelectMaxQMax / SelectTwoStage)
def _torch_token_max_parts(q, k, bs):
    """Padded per-token group means and per-block key extremes, as the
    reference forms them (src/qwen_blocksparse.py:228-234, :278-283)."""
    B, Hq, L, D = q.shape
    Hkv = k.shape[1]
    nblk = (L + bs - 1) // bs
    qp = torch.nn.functional.pad(q, (0, 0, 0, nblk * bs - L))
    kp = torch.nn.functional.pad(k, (0, 0, 0, nblk * bs - L))
    qg = qp.view(B, Hkv, Hq // Hkv, nblk, bs, D).mean(2)
    kb = kp.view(B, Hkv, nblk, bs, D)
    return qg, kb.min(3).values, kb.max(3).values, nblk


def _torch_qmax_scores(qg, kmin, kmax):
    # the per-query-block loop of SelectMaxQMax (src/qwen_blocksparse.py:235-240) on the CPU
    B, H, nblk = kmin.shape[:3]
    score = torch.empty(B, H, nblk, nblk)
    for i in range(nblk):
        qi = qg[:, :, i]
        s = (torch.einsum("bhtd,bhjd->bhtj", qi.clamp(min=0), kmax)
             + torch.einsum("bhtd,bhjd->bhtj", qi.clamp(max=0), kmin))
        score[:, :, i] = s.max(2).values
    return score


def _torch_finish(score, topk, sink):
    B, H, nblk, _ = score.shape
    ar = torch.arange(nblk)
    sc = score.masked_fill(ar.view(1, 1, nblk, 1) < ar.view(1, 1, 1, nblk), float("-inf"))
    tv, ti = sc.topk(min(topk, nblk), dim=-1)
    own = ar.view(1, 1, nblk, 1).expand(B, H, nblk, 1)
    ti = torch.where(torch.isfinite(tv), ti, own.expand_as(ti))
    parts = [ti, own] + ([torch.zeros(B, H, nblk, 1, dtype=torch.long)] if sink else [])
    return torch.cat(parts, -1).sort(-1).values.numpy()


@pytest.mark.parametrize("L", [512, 470])
def test_qmax_scores_match_reference_loop_torch_cpu(L):
    B, Hq, Hkv, D, bs = 1, 4, 2, 32, 64
    g = torch.Generator().manual_seed(11)
    q = torch.randn(B, Hq, L, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, L, D, generator=g).to(torch.bfloat16)
    qg, kmin, kmax, nblk = _torch_token_max_parts(q, k, bs)
    ref = _torch_qmax_scores(qg, kmin, kmax).double().numpy()
    idx, sc = osel.select_quest_qmax(q.double().numpy(), k.double().numpy(), bs, 3, True, "bf16")
    # torch's CPU accumulator may round a token's score differently at a bf16
    # midpoint: at most one ulp, rarely
    diff = sc != ref
    assert diff.mean() < 5e-3
    ulp = 2.0 ** (np.floor(np.log2(np.abs(ref[diff]))) - 7)
    assert np.all(np.abs(sc[diff] - ref[diff]) <= ulp)
    if L % bs:
        assert np.all(sc[:, :, -1] >= 0)  # padding tokens score 0 and take part in the max
    assert idx.shape == (B, Hkv, nblk, 5)


@pytest.mark.parametrize("over", [1, 2, 4])
def test_qmax_and_two_stage_match_reference_torch_cpu_fp32(over):
    # fp32 data (no exact ties): the whole selection equals the reference's
    # algorithm run by torch on the CPU, gather/scatter of the candidates included
    B, Hq, Hkv, L, D, bs, topk = 1, 4, 2, 24 * 32, 16, 32, 4
    g = torch.Generator().manual_seed(12)
    q, k = torch.randn(B, Hq, L, D, generator=g), torch.randn(B, Hkv, L, D, generator=g)
    qg, kmin, kmax, nblk = _torch_token_max_parts(q, k, bs)
    ref_qmax = _torch_finish(_torch_qmax_scores(qg, kmin, kmax), topk, True)
    got_qmax, _ = osel.select_quest_qmax(q.numpy(), k.numpy(), bs, topk, True, "f32")
    np.testing.assert_array_equal(got_qmax, ref_qmax)
    # SelectTwoStage (src/qwen_blocksparse.py:284-299)
    qpool = qg.mean(3)
    s1 = (torch.einsum("bhid,bhjd->bhij", qpool.clamp(min=0), kmax)
          + torch.einsum("bhid,bhjd->bhij", qpool.clamp(max=0), kmin))
    diag = torch.arange(nblk)
    s1 = s1.masked_fill(diag.view(1, 1, nblk, 1) < diag.view(1, 1, 1, nblk), float("-inf"))
    M = min(over * topk, nblk)
    cand = s1.topk(M, dim=-1).indices
    ci = cand.unsqueeze(-1).expand(B, Hkv, nblk, M, D)
    kmax_c = torch.gather(kmax.unsqueeze(2).expand(B, Hkv, nblk, nblk, D), 3, ci)
    kmin_c = torch.gather(kmin.unsqueeze(2).expand(B, Hkv, nblk, nblk, D), 3, ci)
    s2 = (torch.einsum("bhitd,bhimd->bhitm", qg.clamp(min=0), kmax_c)
          + torch.einsum("bhitd,bhimd->bhitm", qg.clamp(max=0), kmin_c)).max(3).values
    full = torch.full((B, Hkv, nblk, nblk), float("-inf")).scatter_(3, cand, s2)
    ref_two = _torch_finish(full, topk, True)
    got_two, _, got_cand = osel.select_two_stage(q.numpy(), k.numpy(), bs, topk, True, over, "f32")
    np.testing.assert_array_equal(got_two, ref_two)
    past = [set(r[r <= i].tolist()) for i, r in enumerate(cand[0, 0].numpy())]
    assert [set(r.tolist()) for r in got_cand[0, 0]] == [p | ({i} if len(p) < M else set()) for i, p in enumerate(past)]


def test_qmax_closed_forms():
    # tokens constant within each block: the token max is the block mean, so
    # SelectMaxQMax reduces to SelectMax; candidates covering every block make
    # SelectTwoStage reduce to SelectMaxQMax
    B, Hq, Hkv, D, bs, nblk = 1, 4, 2, 32, 32, 20
    c = on.round_bf16(RNG.standard_normal((B, Hq, nblk, 1, D)))
    q = np.broadcast_to(c, (B, Hq, nblk, bs, D)).reshape(B, Hq, nblk * bs, D)
    k = on.round_bf16(RNG.standard_normal((B, Hkv, nblk * bs, D)))
    for topk, sink in ((3, True), (5, False), (25, True)):
        iq, sq = osel.select_quest_qmax(q, k, bs, topk, sink, "bf16")
        im, sm = osel.select_quest(q, k, bs, topk, sink, "bf16")
        np.testing.assert_array_equal(sq, sm)
        np.testing.assert_array_equal(iq, im)
    q2 = on.round_bf16(RNG.standard_normal((B, Hq, nblk * bs, D)))
    iq2, sq2 = osel.select_quest_qmax(q2, k, bs, 4, True, "bf16")
    i2, s2, cand = osel.select_two_stage(q2, k, bs, 4, True, 5, "bf16")
    np.testing.assert_array_equal(i2, iq2)
    fut = np.arange(nblk)[None, :] > np.arange(nblk)[:, None]
    np.testing.assert_array_equal(np.where(fut, -np.inf, s2), np.where(fut, -np.inf, sq2))
    assert all(set(cand[0, 0, i].tolist()) == set(range(i + 1)) for i in range(nblk))


# ---------------------------------------------------------------- centroid / LSH routing
def test_bucket_members_matches_cumcount_idiom():
    # the reference builds the buckets with one_hot + cumsum (src/ssa_model.py:269-275)
    home = RNG.integers(0, 5, size=(3, 40))
    for cap in (1, 3, 40):
        ref = torch.full((3, 5, cap), -1, dtype=torch.long)
        h = torch.from_numpy(home)
        oh = torch.nn.functional.one_hot(h, 5)
        within = (oh.cumsum(1) - oh).gather(2, h.unsqueeze(-1)).squeeze(-1)
        keep = within < cap
        bI = torch.arange(3).view(3, 1).expand(3, 40)
        jI = torch.arange(40).view(1, 40).expand(3, 40)
        ref[bI[keep], h[keep], within[keep]] = jI[keep]
        np.testing.assert_array_equal(osel.bucket_members(home, 5, cap), ref.numpy())


def test_centroid_route_closed_form_and_invariants():
    B, nblk, s = 2, 12, 8
    sq, sk = RNG.standard_normal((B, nblk, s)), RNG.standard_normal((B, nblk, s))
    # one centroid, one route, capacity >= nblk: every block (the reference's exactness check)
    slots, _, _, _ = osel.centroid_route(sq, sk, RNG.standard_normal((1, s)), 1, nblk)
    for i in range(nblk):
        row = slots[0, i]
        assert row[0] == i and sorted(row[row >= 0].tolist()) == list(range(nblk))
    cent = RNG.standard_normal((5, s))
    slots, qc, kc, home = osel.centroid_route(sq, sk, cent, 2, 3)
    assert slots.shape == (B, nblk, 1 + 6)
    for b in range(B):
        for i in range(nblk):
            picks = slots[b, i, 1:][slots[b, i, 1:] >= 0]
            routes = set(np.argsort(-qc[b, i])[:2].tolist())
            assert all(home[b, j] in routes for j in picks) and i not in picks
            assert len(set(picks.tolist())) == len(picks)
    qm, km = RNG.standard_normal((B, nblk, 4)), RNG.standard_normal((B, nblk, 4))
    r2, _, _, _ = osel.centroid_route(sq, sk, cent, 2, 3, refine_topk=2, qm=qm, km=km)
    for b in range(B):
        for i in range(nblk):
            full = slots[b, i, 1:][slots[b, i, 1:] >= 0]
            best = sorted(full.tolist(), key=lambda j: -(qm[b, i] @ km[b, j]))[:2]
            got = [j for j in r2[b, i, 1:].tolist() if j >= 0]
            assert got == best


@pytest.mark.parametrize("causal", [False, True])
def test_lsh_routes_reduce_to_dense_and_match_torch_topk(causal):
    B, nblk, s, topk, scale = 2, 20, 8, 4, 2.5
    sq, sk = RNG.standard_normal((B, nblk, s)), RNG.standard_normal((B, nblk, s))
    sq /= np.linalg.norm(sq, axis=-1, keepdims=True)
    sk /= np.linalg.norm(sk, axis=-1, keepdims=True)
    dense, dsc = osel.lsh_dense(sq, sk, scale, causal, topk)
    # one round, one bucket, capacity nblk: every block is a candidate
    slots, sc = osel.lsh_route(sq, sk, RNG.standard_normal((s, 1, 1)), nblk, scale, causal, topk)
    np.testing.assert_array_equal(slots, dense)
    np.testing.assert_allclose(sc, dsc, rtol=1e-12)
    # the reference's dense top-k (src/ssa_model.py:397-405) on these tie-free scores
    t_sq, t_sk = torch.from_numpy(sq), torch.from_numpy(sk)
    raw = scale * (t_sq @ t_sk.transpose(-1, -2))
    diag = torch.arange(nblk)
    raw = raw.masked_fill(diag.view(1, nblk, 1) == diag.view(1, 1, nblk), float("-inf"))
    if causal:
        raw = raw.masked_fill(diag.view(1, 1, nblk) > diag.view(1, nblk, 1), float("-inf"))
    topv, topi = raw.topk(min(topk, nblk - 1), dim=-1)
    ref = torch.where(torch.isfinite(topv), topi, torch.full_like(topi, -1)).numpy()
    np.testing.assert_array_equal(dense[..., 1:], ref)
    # several rounds and buckets: picks come from the query's buckets, distinct, past only when causal
    R = RNG.standard_normal((s, 3, 4))
    slots, _ = osel.lsh_route(sq, sk, R, 3, scale, causal, topk)
    kb = np.einsum("bns,src->bnrc", sk, R).argmax(-1)
    qb = np.einsum("bns,src->bnrc", sq, R).argmax(-1)
    for b in range(B):
        for i in range(nblk):
            picks = [j for j in slots[b, i, 1:].tolist() if j >= 0]
            assert len(set(picks)) == len(picks) and i not in picks
            assert all((kb[b, j] == qb[b, i]).any() for j in picks)
            if causal:
                assert all(j < i for j in picks)
