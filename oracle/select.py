"""Selection oracle: pooling, pooled scores, conventions A and B (test infrastructure only).

Restates, in numpy, the reference's block-pair selection:

* ``pool_mean_tok_then_heads`` -- ``q.view(B,H,nblk,Bs,dh).mean(3).mean(1)``
  (``src/ssa_model.py:287-288``): the mean-pooled q/k selector used by the
  synthetic configurations (the contraction is ``src/scale_sel.py:33-35``).
* ``pool_mean_grp_then_tok`` / ``pool_minmax`` -- ``SelectMax.select``
  (``src/qwen_blocksparse.py:111-116``).
* ``pool_tok`` -- ``BlockSparseSSA._scores`` pooling (``src/ssa_model.py:114-117``).
* ``pool_last_token_grp`` / ``pool_mean_tok`` -- the ``SelectLastTok`` and
  ``SelectLearned`` poolings (``src/qwen_blocksparse.py:259``, ``:183``).
* ``scores`` -- the nblk x nblk contraction: plain dot (``src/scale_sel.py:33``),
  max of two dots (``src/ssa_model.py:118-119``), Quest q+/q- split
  (``src/qwen_blocksparse.py:117-120``), each rounded where torch rounds.
* ``select_conv_a`` -- own block first + top-k content blocks
  (``src/ssa_model.py:151-165``; ``src/bench_crossover.py:41-54``).
* ``select_conv_b`` -- ``_finish`` (``src/qwen_blocksparse.py:87-99``).
* ``bucket_members`` / ``centroid_route`` / ``lsh_route`` / ``lsh_dense`` -- the
  routing of ``CentroidSSA`` and ``LSHBucketSSA`` (``src/ssa_model.py:204-513``).
* ``pool_grp_mean_tok`` / ``scores_qmax`` / ``select_topk_set`` -- the
  token-max Quest score of ``SelectMaxQMax`` and the two stages of
  ``SelectTwoStage`` (``src/qwen_blocksparse.py:216-241``, ``:267-299``).

Tie-break: candidates are ranked NaN first (torch.topk treats NaN as the
largest value), then by descending score, then by ascending block index.
torch.topk's order among exactly equal scores is implementation-defined; the
lowest-index rule is this build's canonical choice and ``near_tie_rows``
implements the parity procedure for comparing against any other order.
"""
import numpy as np

from .numerics import round_to


def _pad_tokens(x, bs, axis):
    """Zero-pad the token axis to a multiple of bs (``_pad_blocks``,
    ``src/qwen_blocksparse.py:20-26``; ``F.pad`` in ``src/ssa_model.py:124-126``)."""
    n = x.shape[axis]
    nblk = (n + bs - 1) // bs
    pad = nblk * bs - n
    if pad:
        widths = [(0, 0)] * x.ndim
        widths[axis] = (0, pad)
        x = np.pad(x, widths)
    return x, nblk


def pool_mean_tok_then_heads(x, bs, dtype):
    """(B,H,N,D) -> (B,nblk,D): mean over the block's tokens (rounded), then
    over heads (rounded). ``src/ssa_model.py:287-288``."""
    x = np.asarray(x, dtype=np.float64)
    B, H, N, D = x.shape
    x, nblk = _pad_tokens(x, bs, 2)
    tok = round_to(x.reshape(B, H, nblk, bs, D).sum(axis=3) / bs, dtype)
    return round_to(tok.sum(axis=1) / H, dtype)


def pool_mean_grp_then_tok(q, hkv, bs, dtype):
    """(B,Hq,N,D) -> (B,Hkv,nblk,D): mean over the GQA group (rounded), then
    over the block's tokens (rounded). ``src/qwen_blocksparse.py:113``."""
    q = np.asarray(q, dtype=np.float64)
    B, Hq, N, D = q.shape
    grp = Hq // hkv
    q, nblk = _pad_tokens(q, bs, 2)
    g = round_to(q.reshape(B, hkv, grp, nblk, bs, D).sum(axis=2) / grp, dtype)
    return round_to(g.sum(axis=3) / bs, dtype)


def pool_minmax(k, bs):
    """(B,H,N,D) -> kmin, kmax (B,H,nblk,D), exact. Padding rows are zeros and
    take part, as in ``src/qwen_blocksparse.py:112-116``."""
    k = np.asarray(k, dtype=np.float64)
    B, H, N, D = k.shape
    k, nblk = _pad_tokens(k, bs, 2)
    kb = k.reshape(B, H, nblk, bs, D)
    return kb.min(axis=3), kb.max(axis=3)


def pool_last_token_grp(q, hkv, bs, dtype):
    """(B,Hq,N,D) -> (B,Hkv,nblk,D): the GQA-group mean (rounded) of each
    block's last token; a ragged last block's last token is the zero padding.
    ``q.view(B,Hkv,grp,nblk,bs,d).mean(2)[:, :, :, -1, :]``
    (``src/qwen_blocksparse.py:259``)."""
    q = np.asarray(q, dtype=np.float64)
    B, Hq, N, D = q.shape
    grp = Hq // hkv
    q, nblk = _pad_tokens(q, bs, 2)
    last = q.reshape(B, Hq, nblk, bs, D)[:, :, :, -1, :]
    return round_to(last.reshape(B, hkv, grp, nblk, D).sum(axis=2) / grp, dtype)


def pool_mean_tok(x, bs, dtype):
    """(B,H,N,D) -> (B,H,nblk,D): per-head token mean (rounded), zero padding
    counted: ``kp.view(B,Hkv,nblk,bs,d).mean(3)`` (``src/qwen_blocksparse.py:183``)."""
    x = np.asarray(x, dtype=np.float64)
    B, H, N, D = x.shape
    x, nblk = _pad_tokens(x, bs, 2)
    return round_to(x.reshape(B, H, nblk, bs, D).sum(axis=3) / bs, dtype)


def pool_tok(x, bs, dtype, op):
    """(B,N,S) -> (B,nblk,S): per-block token mean (rounded) or max (exact).
    ``src/ssa_model.py:114-117`` (N is already a multiple of bs there)."""
    x = np.asarray(x, dtype=np.float64)
    B, N, S = x.shape
    x, nblk = _pad_tokens(x, bs, 1)
    xb = x.reshape(B, nblk, bs, S)
    if op == "mean":
        return round_to(xb.sum(axis=2) / bs, dtype)
    if op == "max":
        return xb.max(axis=2)
    if op == "min":
        return xb.min(axis=2)
    raise ValueError(op)


def _seq_dot(a, b, rows=None):
    """Exact-order dot products: s = sum_d a[..,i,d]*b[..,j,d] accumulated
    sequentially over d in float64 (the GPU kernel uses the same order with
    fp64 FMA, and the bf16/fp32 products are exact in fp64)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if rows is not None:
        a = a[..., rows, :]
    out = np.zeros(a.shape[:-1] + (b.shape[-2],), dtype=np.float64)
    for d in range(a.shape[-1]):
        out += a[..., :, None, d] * b[..., None, :, d]
    return out


def scores(a, b1, dtype, combine="dot", b2=None, rows=None):
    """Pooled block-pair scores (..., nblk_q, nblk_k), rounded like torch.

    combine='dot'   : rnd(a . b1)                                (src/scale_sel.py:33)
    combine='max2'  : max(rnd(a . b1), rnd(a . b2))              (src/ssa_model.py:118-119)
    combine='quest' : rnd(rnd(relu(a) . b1) + rnd(min(a,0) . b2)) with b1=kmax,
                      b2=kmin                                    (src/qwen_blocksparse.py:117-120)
    ``rows`` restricts the query-block rows computed (for large nblk).
    """
    if combine == "dot":
        return round_to(_seq_dot(a, b1, rows), dtype)
    if combine == "max2":
        return np.maximum(round_to(_seq_dot(a, b1, rows), dtype),
                          round_to(_seq_dot(a, b2, rows), dtype))
    if combine == "quest":
        a = np.asarray(a, dtype=np.float64)
        s1 = round_to(_seq_dot(np.maximum(a, 0.0), b1, rows), dtype)
        s2 = round_to(_seq_dot(np.minimum(a, 0.0), b2, rows), dtype)
        return round_to(s1 + s2, dtype)
    raise ValueError(combine)


def _rank(score, valid):
    """Per-row candidate order: valid NaN first, then valid by descending
    score, then invalid; ties by ascending index (stable)."""
    score = np.asarray(score, dtype=np.float64)
    nan = np.isnan(score)
    cls = np.where(valid, np.where(nan, 0, 1), 2)
    neg = np.where(nan, 0.0, -score)
    idx = np.broadcast_to(np.arange(score.shape[-1]), score.shape)
    return np.lexsort((idx, neg, cls), axis=-1)


def select_conv_a(raw, topk, causal, rows=None):
    """Convention A (``src/ssa_model.py:151-165``).

    raw: (B, nblk_rows, nblk) scores for query-block rows ``rows`` (all rows by
    default). Returns sel (B, R, kk) int64 with kk = 1 + min(topk, nblk-1):
    slot 0 = own block i; slots 1.. = content blocks by descending score with
    the diagonal (and, if causal, every j > i) excluded. Rows with fewer valid
    candidates than the budget (causal, i < kk-1) are filled with i; the
    slot-causal mask rule (slot s>0 valid iff sel < i) masks those fills, as it
    masks torch.topk's -inf picks in the reference.
    """
    raw = np.asarray(raw, dtype=np.float64)
    B, R, nblk = raw.shape
    rows = np.arange(R) if rows is None else np.asarray(rows)
    j = np.arange(nblk)
    valid = j[None, :] != rows[:, None]
    if causal:
        valid &= j[None, :] < rows[:, None]
    valid = np.broadcast_to(valid, raw.shape)
    kk_c = min(topk, nblk - 1)
    own = np.broadcast_to(rows[None, :, None], (B, R, 1)).astype(np.int64)
    if kk_c <= 0:
        return own.copy()
    order = _rank(raw, valid)[..., :kk_c]
    ok = np.take_along_axis(valid, order, axis=-1)
    picks = np.where(ok, order, own)
    return np.concatenate([own, picks], axis=-1).astype(np.int64)


def select_conv_b(score, topk, sink, rows=None):
    """Convention B, ``_finish`` (``src/qwen_blocksparse.py:87-99``).

    score: (B, H, R, nblk). Future blocks j > i are masked to -inf (own NOT
    excluded); the top min(topk, nblk) picks whose score is not finite become
    the own block; own (and block 0 when ``sink``) are appended and each row is
    sorted ascending. Duplicates are kept (the attention rule dedups them).
    """
    score = np.asarray(score, dtype=np.float64)
    B, H, R, nblk = score.shape
    rows = np.arange(R) if rows is None else np.asarray(rows)
    j = np.arange(nblk)
    fut = j[None, :] > rows[:, None]
    masked = np.where(fut, -np.inf, score)
    kk_t = min(topk, nblk)
    order = _rank(masked, np.ones_like(masked, dtype=bool))[..., :kk_t]
    vals = np.take_along_axis(masked, order, axis=-1)
    own = np.broadcast_to(rows[None, None, :, None], (B, H, R, 1)).astype(np.int64)
    picks = np.where(np.isfinite(vals), order, own)
    parts = [picks, own]
    if sink:
        parts.append(np.zeros((B, H, R, 1), dtype=np.int64))
    return np.sort(np.concatenate(parts, axis=-1), axis=-1).astype(np.int64)


def gate_from_scores(raw, sel):
    """gate[b,i,s] = logsigmoid(raw[b,i,sel[b,i,s]]) (``src/ssa_model.py:189-191``),
    float64 (the caller rounds to the score dtype if it mirrors torch)."""
    g = np.take_along_axis(np.asarray(raw, dtype=np.float64), np.asarray(sel), axis=-1)
    return -np.logaddexp(0.0, -g)


def select_mean_pooled(q, k, bs, topk, causal, dtype):
    """Configs 1/2/3/5 selector: mean-pooled q.k scores + convention A.
    Returns (sel (B,nblk,kk) int64, raw (B,nblk,nblk))."""
    qp = pool_mean_tok_then_heads(q, bs, dtype)
    kp = pool_mean_tok_then_heads(k, bs, dtype)
    raw = scores(qp, kp, dtype, "dot")
    return select_conv_a(raw, topk, causal), raw


def select_quest(q, k, bs, topk, sink, dtype):
    """``SelectMax.select`` (``src/qwen_blocksparse.py:107-121``).
    Returns (idx (B,Hkv,nblk,kk) int64, score (B,Hkv,nblk,nblk))."""
    hkv = k.shape[1]
    qpool = pool_mean_grp_then_tok(q, hkv, bs, dtype)
    kmin, kmax = pool_minmax(k, bs)
    sc = scores(qpool, kmax, dtype, "quest", b2=kmin)
    return select_conv_b(sc, topk, sink), sc


def select_quest_lasttok(q, k, bs, topk, sink, dtype):
    """``SelectLastTok.select`` (``src/qwen_blocksparse.py:244-264``): Quest
    scores of each block's last-token group mean, then ``_finish``."""
    hkv = k.shape[1]
    qlast = pool_last_token_grp(q, hkv, bs, dtype)
    kmin, kmax = pool_minmax(k, bs)
    sc = scores(qlast, kmax, dtype, "quest", b2=kmin)
    return select_conv_b(sc, topk, sink), sc


def select_learned_features(sq, sk, topk, sink, dtype, scale):
    """``SelectLearned`` / ``SelectLearnedMinMax`` from their projected features
    (``src/qwen_blocksparse.py:184-187``, ``:210-213``): score =
    rnd(scale * rnd(sq . sk)) in the feature dtype, then ``_finish``. Returns
    (idx, score, unscaled rnd(sq . sk))."""
    raw = scores(sq, sk, dtype, "dot")
    sc = round_to(scale * raw, dtype)
    return select_conv_b(sc, topk, sink), sc, raw


def pool_grp_mean_tok(q, hkv, dtype):
    """(B,Hq,N,D) -> (B,Hkv,N,D): the GQA-group mean of every token (rounded),
    ``qp.view(B,Hkv,grp,nblk,bs,d).mean(2)`` (``src/qwen_blocksparse.py:231``,
    ``:281``) before the block padding (padding tokens are zeros)."""
    q = np.asarray(q, dtype=np.float64)
    B, Hq, N, D = q.shape
    grp = Hq // hkv
    return round_to(q.reshape(B, hkv, grp, N, D).sum(axis=2) / grp, dtype)


def scores_qmax(qg, kmax, kmin, bs, dtype, cand=None):
    """Row-block max Quest scores (B,H,nblk,nblk): score(i,j) = max over the bs
    tokens t of block i (zero padded) of rnd(rnd(relu(q_t).kmax_j) +
    rnd(min(q_t,0).kmin_j)) -- the per-block loop of ``SelectMaxQMax``
    (``src/qwen_blocksparse.py:236-240``). With ``cand`` (B,H,nblk,M) only the
    candidate columns keep their score and every other entry is -inf (the
    scatter into a -inf matrix of ``SelectTwoStage``, ``:297-298``)."""
    qg, nblk = _pad_tokens(np.asarray(qg, dtype=np.float64), bs, 2)
    B, H, _, D = qg.shape
    tok = scores(qg, kmax, dtype, "quest", b2=kmin)              # (B,H,nblk*bs,nblk)
    sc = tok.reshape(B, H, nblk, bs, -1).max(axis=3)
    if cand is not None:
        keep = np.zeros(sc.shape, dtype=bool)
        np.put_along_axis(keep, np.asarray(cand, dtype=np.int64), True, axis=-1)
        sc = np.where(keep, sc, -np.inf)
    return sc


def select_topk_set(score, topk):
    """Candidate stage of ``SelectTwoStage`` (``src/qwen_blocksparse.py:288-290``):
    the top min(topk, nblk) blocks over j <= i (future blocks are -inf), used
    as a set -- non-finite picks become the own block (a -inf pick is a future
    block, which the final ``_finish`` masks anyway), sorted ascending, nothing
    appended. score: (B,H,R,nblk); returns (B,H,R,min(topk,nblk)) int64."""
    score = np.asarray(score, dtype=np.float64)
    B, H, R, nblk = score.shape
    rows = np.arange(R)
    masked = np.where(np.arange(nblk)[None, :] > rows[:, None], -np.inf, score)
    kk_t = min(topk, nblk)
    order = _rank(masked, np.ones_like(masked, dtype=bool))[..., :kk_t]
    vals = np.take_along_axis(masked, order, axis=-1)
    own = np.broadcast_to(rows[None, None, :, None], order.shape)
    return np.sort(np.where(np.isfinite(vals), order, own), axis=-1).astype(np.int64)


def select_quest_qmax(q, k, bs, topk, sink, dtype):
    """``SelectMaxQMax.select`` (``src/qwen_blocksparse.py:216-241``).
    Returns (idx (B,Hkv,nblk,kk) int64, score (B,Hkv,nblk,nblk))."""
    hkv = k.shape[1]
    qg = pool_grp_mean_tok(q, hkv, dtype)
    kmin, kmax = pool_minmax(k, bs)
    sc = scores_qmax(qg, kmax, kmin, bs, dtype)
    return select_conv_b(sc, topk, sink), sc


def select_two_stage(q, k, bs, topk, sink, over, dtype):
    """``SelectTwoStage.select`` (``src/qwen_blocksparse.py:267-299``): block-mean
    Quest scores pick M = min(over*topk, nblk) candidates, the token-max Quest
    score re-ranks them, then ``_finish``. Returns (idx, final scores, cand)."""
    hkv = k.shape[1]
    qg = pool_grp_mean_tok(q, hkv, dtype)
    qpool = pool_mean_tok(qg, bs, dtype)                      # qg.mean(3), :284
    kmin, kmax = pool_minmax(k, bs)
    nblk = kmax.shape[2]
    s1 = scores(qpool, kmax, dtype, "quest", b2=kmin)
    cand = select_topk_set(s1, min(over * topk, nblk))
    s2 = scores_qmax(qg, kmax, kmin, bs, dtype, cand=cand)
    return select_conv_b(s2, topk, sink), s2, cand


def bucket_members(home, n_buckets, cap):
    """(B, n) bucket id per block -> (B, n_buckets, cap) ids of each bucket's
    first cap members in block order, -1 for unused places (the fixed-capacity
    buckets of ``src/ssa_model.py:269-275``, ``:430-436``), by a plain loop."""
    home = np.asarray(home)
    B, n = home.shape
    out = np.full((B, n_buckets, cap), -1, dtype=np.int64)
    for b in range(B):
        fill = np.zeros(n_buckets, dtype=np.int64)
        for j in range(n):
            c = home[b, j]
            if fill[c] < cap:
                out[b, c, fill[c]] = j
                fill[c] += 1
    return out


def centroid_route(sq, sk, cent, cpq, cap, refine_topk=None, qm=None, km=None):
    """``CentroidSSA`` routing (``src/ssa_model.py:256-301``) on float64 values:
    qc = sq.cent^T, kc = sk.cent^T, each key block's centroid argmax(kc), each
    query block's top-cpq centroids, their buckets' members (own block
    removed), optional re-rank of the candidates by qm.km (block means of the
    main q, k) to refine_topk. Returns (slots (B,nblk,kk) int64 with -1 for
    empty places, qc, kc, home)."""
    sq, sk, cent = (np.asarray(a, dtype=np.float64) for a in (sq, sk, cent))
    B, nblk, _ = sq.shape
    C = cent.shape[0]
    cpq, cap = min(cpq, C), min(cap, nblk)
    qc, kc = sq @ cent.T, sk @ cent.T
    home = kc.argmax(-1)
    routes = np.argsort(-qc, axis=-1, kind="stable")[..., :cpq]
    members = bucket_members(home, C, cap)
    slots = np.stack([np.concatenate([members[b, routes[b, i]].ravel() for i in range(nblk)]).reshape(nblk, -1)
                      for b in range(B)])
    own = np.arange(nblk)[None, :, None]
    slots = np.where(slots == own, -1, slots)
    if refine_topk is not None and refine_topk < cpq * cap:
        qm, km = np.asarray(qm, dtype=np.float64), np.asarray(km, dtype=np.float64)
        sc = np.einsum("bid,bipd->bip", qm, km[np.arange(B)[:, None, None], np.maximum(slots, 0)])
        sc = np.where(slots >= 0, sc, -np.inf)
        order = np.argsort(-sc, axis=-1, kind="stable")[..., :min(refine_topk, cpq * cap)]
        slots = np.take_along_axis(slots, order, -1)
    slots = np.concatenate([np.broadcast_to(own, (B, nblk, 1)), slots], -1)
    return slots, qc, kc, home


def lsh_route(sq, sk, R, cap, scale, causal, topk):
    """``LSHBucketSSA`` bucketed selection (``src/ssa_model.py:425-452``): per
    round, hash = argmax of the projection on R[:, r, :]; candidates = the
    first cap members of the query block's bucket, concatenated over rounds;
    a place is dropped if empty, a repeat of an earlier place (compared on
    ids with empty places read as block 0, as the reference compares them),
    the own block or (causal) a future block; the rest are scored
    scale * sq.sk and the top min(k, places) kept. Returns (slots (B,nblk,kk)
    with -1 for invalid picks, own first; their scores, own score first)."""
    sq, sk, R = (np.asarray(a, dtype=np.float64) for a in (sq, sk, R))
    B, nblk, _ = sq.shape
    NR, NB = R.shape[1], R.shape[2]
    cap = min(cap, nblk)
    kb = np.einsum("bns,src->bnrc", sk, R).argmax(-1)
    qb = np.einsum("bns,src->bnrc", sq, R).argmax(-1)
    cand = np.concatenate([bucket_members(kb[..., r], NB, cap)[np.arange(B)[:, None], qb[..., r]]
                           for r in range(NR)], -1)                      # (B, nblk, P)
    P = cand.shape[-1]
    cc = np.maximum(cand, 0)
    rows = np.arange(nblk)[None, :, None]
    ok = cand >= 0
    for p in range(1, P):
        ok[..., p] &= ~(cc[..., :p] == cc[..., p:p + 1]).any(-1)
    ok &= cand != rows
    if causal:
        ok &= cand < rows
    sc = np.where(ok, scale * np.einsum("bis,bips->bip", sq, sk[np.arange(B)[:, None, None], cc]), -np.inf)
    kk_c = min(topk, max(1, nblk - 1))
    order = np.argsort(-sc, axis=-1, kind="stable")[..., :min(kk_c, P)]
    topv = np.take_along_axis(sc, order, -1)
    picks = np.where(np.isfinite(topv), np.take_along_axis(cc, order, -1), -1)
    own_sc = scale * (sq * sk).sum(-1)[..., None]
    slots = np.concatenate([np.broadcast_to(rows, (B, nblk, 1)), picks], -1)
    return slots, np.concatenate([own_sc, np.where(np.isfinite(topv), topv, 0.0)], -1)


def lsh_dense(sq, sk, scale, causal, topk):
    """``LSHBucketSSA`` train-time dense selection (``src/ssa_model.py:397-405``):
    top-k of scale * sq.sk^T over j != i (and j < i when causal), own first,
    -inf picks invalid (-1). Returns (slots, scores) like ``lsh_route``."""
    sq, sk = np.asarray(sq, dtype=np.float64), np.asarray(sk, dtype=np.float64)
    B, nblk, _ = sq.shape
    raw = scale * np.einsum("bis,bjs->bij", sq, sk)
    j = np.arange(nblk)
    bad = j[None, :] == j[:, None]
    if causal:
        bad |= j[None, :] > j[:, None]
    raw = np.where(bad[None], -np.inf, raw)
    kk_c = min(topk, max(1, nblk - 1))
    order = np.argsort(-raw, axis=-1, kind="stable")[..., :kk_c]
    topv = np.take_along_axis(raw, order, -1)
    picks = np.where(np.isfinite(topv), order, -1)
    own_sc = scale * (sq * sk).sum(-1)[..., None]
    slots = np.concatenate([np.broadcast_to(j[None, :, None], (B, nblk, 1)), picks], -1)
    return slots, np.concatenate([own_sc, np.where(np.isfinite(topv), topv, 0.0)], -1)


def near_tie_rows(score, sel_valid_sets, k_eff, valid_mask, rel=1e-6):
    """Parity procedure for selected-set comparison (near-tie census).

    score: (..., R, nblk) oracle scores; valid_mask: candidate validity of the
    same shape; sel_valid_sets: (..., R, k_eff) chosen candidate indices (the
    valid content picks). A row is a near-tie row if some valid candidate
    outside the chosen set has |s - s_k| < rel * max(1, |s_k|), where s_k is
    the k-th best chosen score. Returns a bool array (..., R).
    """
    score = np.asarray(score, dtype=np.float64)
    chosen = np.zeros(score.shape, dtype=bool)
    np.put_along_axis(chosen, np.asarray(sel_valid_sets), True, axis=-1)
    chosen &= valid_mask
    s_chosen = np.where(chosen, score, np.inf)
    s_k = s_chosen.min(axis=-1, keepdims=True)
    others = valid_mask & ~chosen & np.isfinite(score)
    tol = rel * np.maximum(1.0, np.abs(s_k))
    close = others & (np.abs(score - s_k) < tol)
    has_k = np.isfinite(s_k[..., 0])
    return close.any(axis=-1) & has_k
