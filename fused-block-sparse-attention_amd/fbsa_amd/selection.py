"""Block pooling and streaming block-pair selection over the C ABI (gfx950).

The pooled-score matrix (nblk x nblk) is never materialised: ``select`` streams
the candidates through a per-row top-k held in registers. Scores are computed
exactly (float64) and rounded to the operand dtype where torch rounds, so the
chosen blocks match the oracle bit for bit; ties break towards the lower block
index.
"""
import torch

from . import _lib
from .ops import _dtype_code, _ptr, _require_cuda, _stream

POOL_OPS = {"mean_tok_then_grp": _lib.POOL_MEAN_TOK_THEN_GRP,
            "mean_grp_then_tok": _lib.POOL_MEAN_GRP_THEN_TOK,
            "max": _lib.POOL_MAX, "min": _lib.POOL_MIN, "minmax": _lib.POOL_MINMAX}
SCORES = {"dot": _lib.SCORE_DOT, "max2": _lib.SCORE_MAX2, "quest": _lib.SCORE_QUEST}
MAX_TOPK = 4096  # largest top-k budget of fbsa_select (past 62: one workgroup per row, keys in LDS)


def _pool_desc(x, bs, op, grp, l_valid):
    B, H, L, D = x.shape
    d = _lib.PoolDesc()
    d.dtype = _dtype_code(x)
    d.op = POOL_OPS[op]
    d.B, d.H, d.L, d.D, d.bs, d.nblk, d.grp = B, H, L, D, bs, (L + bs - 1) // bs, grp
    d.l_valid = L if l_valid is None else int(l_valid)
    d.sx[:] = (x.stride(0), x.stride(1), x.stride(2))
    return d


def _pool_input(x):
    if x.stride(-1) != 1 or any((s * x.element_size()) % 16 for s in x.stride()[:-1]) or x.data_ptr() % 16:
        return x.contiguous()
    return x


def pool(x, bs, op, grp=1, l_valid=None):
    """Pool x (B,H,L,D) over blocks of bs tokens (and groups of grp heads).

    op: 'mean_tok_then_grp' (src/ssa_model.py:287-288 with grp=H),
    'mean_grp_then_tok' (src/qwen_blocksparse.py:113), 'max', 'min' or
    'minmax' (src/qwen_blocksparse.py:115-116; returns (min, max)).
    Tokens at positions >= l_valid (default L) count as zeros, like the
    reference's zero padding. Returns (B, H//grp, ceil(L/bs), D) in x's dtype.
    """
    _require_cuda(x)
    if x.dim() != 4:
        raise ValueError("fbsa.pool: x must be (B, H, L, D)")
    B, H, L, D = x.shape
    x = _pool_input(x)
    nblk = (L + bs - 1) // bs
    d = _pool_desc(x, bs, op, grp, l_valid)
    out = torch.empty(B, H // grp if H % grp == 0 else 1, nblk, D, dtype=x.dtype, device=x.device)
    out2 = torch.empty_like(out) if op == "minmax" else None
    _lib.check(_lib.load().fbsa_pool(d, _ptr(x), _ptr(out), _ptr(out2), _stream()), "fbsa_pool")
    return (out, out2) if op == "minmax" else out


def budget(convention, topk, nblk, sink=False):
    """Slots per query block: A: 1 + min(topk, nblk-1); B: min(topk, nblk) + 1 + sink."""
    if convention == "own_first":
        return 1 + min(topk, nblk - 1)
    return min(topk, nblk) + 1 + (1 if sink else 0)


def select(a, b1, b2=None, *, score="dot", convention="own_first", topk, causal=True, sink=False,
           need_scores=False, engine="auto", chunk_tiles=0, rows=None, out=None, workspace=None):
    """Top-k key blocks per query block from pooled operands (B,H,nblk,D).

    convention 'own_first' (A, src/ssa_model.py:151-165): [i, top-k content
    blocks by descending score]; 'sorted_sink' (B, ``_finish``,
    src/qwen_blocksparse.py:87-99): top-k over j <= i, + own (+ sink 0), sorted.
    Returns sel int32 (B,H,nblk,kk) (and fp32 scores of the chosen slots).
    engine: "auto" forms 16-bit scores on MFMA with exact verification (fp64
    only where an MFMA bracket is ambiguous); "fp64" scores everything in fp64.
    Both return identical blocks. chunk_tiles (tuning/tests): candidate tiles
    of 64 blocks per workgroup on the MFMA path, 0 = chosen from the sizes.
    rows=(r0, r1) selects query blocks [r0, r1) only, writing those rows of
    `out` (an int32 (B,H,nblk,kk) tensor); `workspace` may pass a uint8
    tensor of at least select_workspace_bytes() bytes to reuse.
    """
    _require_cuda(a, b1, b2)
    if a.dim() != 4 or a.shape != b1.shape or (b2 is not None and b2.shape != a.shape):
        raise ValueError("fbsa.select: operands must be (B, H, nblk, D) of equal shape")
    if a.dtype != b1.dtype or (b2 is not None and b2.dtype != a.dtype):
        raise ValueError("fbsa.select: operands must share a dtype")
    B, H, nblk, D = a.shape
    a, b1 = a.contiguous(), b1.contiguous()
    b2 = b2.contiguous() if b2 is not None else None
    conv = {"own_first": _lib.SEL_OWN_FIRST, "sorted_sink": _lib.SEL_SORTED_SINK}[convention]
    kk = budget(convention, topk, nblk, sink)
    d = _lib.SelectDesc()
    d.dtype = _dtype_code(a)
    d.score = SCORES[score]
    d.convention = conv
    d.causal = 1 if causal else 0
    d.sink = 1 if sink else 0
    if not 0 <= chunk_tiles < 65536:
        raise ValueError("fbsa.select: chunk_tiles must be in [0, 65536)")
    d.flags = chunk_tiles << _lib.SEL_CHUNK_SHIFT
    d.B, d.H, d.nblk, d.D, d.topk, d.kk = B, H, nblk, D, topk, kk
    if out is not None:
        if out.shape != (B, H, nblk, kk) or out.dtype != torch.int32 or not out.is_contiguous():
            raise ValueError(f"fbsa.select: out must be contiguous int32 {(B, H, nblk, kk)}")
        sel = out
    else:
        sel = torch.empty(B, H, nblk, kk, dtype=torch.int32, device=a.device)
    sc = torch.empty(B, H, nblk, kk, dtype=torch.float32, device=a.device) if need_scores else None
    lib = _lib.load()
    nbytes = lib.fbsa_select_workspace_bytes(d) if engine == "auto" else 0
    if workspace is not None and nbytes and workspace.numel() >= nbytes:
        ws = workspace
    else:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
    r0, r1 = (0, nblk) if rows is None else rows
    _lib.check(lib.fbsa_select_rows(d, r0, r1, _ptr(a), _ptr(b1), _ptr(b2), _ptr(sel), _ptr(sc), _ptr(ws), nbytes,
                                    _stream()), "fbsa_select")
    return (sel, sc) if need_scores else sel


def select_workspace_bytes(a, *, score="dot", convention="own_first", topk, sink=False, chunk_tiles=0):
    """Workspace bytes the MFMA engine needs for pooled operands shaped like `a`."""
    B, H, nblk, D = a.shape
    d = _lib.SelectDesc()
    d.dtype = _dtype_code(a)
    d.score = SCORES[score]
    d.convention = {"own_first": _lib.SEL_OWN_FIRST, "sorted_sink": _lib.SEL_SORTED_SINK}[convention]
    d.causal, d.sink, d.flags = 1, 1 if sink else 0, chunk_tiles << _lib.SEL_CHUNK_SHIFT
    d.B, d.H, d.nblk, d.D, d.topk, d.kk = B, H, nblk, D, topk, budget(convention, topk, nblk, sink)
    return _lib.load().fbsa_select_workspace_bytes(d)


def select_mean_pooled(q, k, bs, topk, causal=True, need_scores=False, engine="auto"):
    """Synthetic-config selector: mean-pooled q.k block scores, convention A.

    qpool = q.view(B,H,nblk,bs,D).mean(3).mean(1) (src/ssa_model.py:287-288),
    raw = qpool kpool^T (src/scale_sel.py:33), then own block + top-k content
    blocks (src/ssa_model.py:151-165). Returns sel (B, nblk, kk) int32.
    """
    if engine == "fp64" or q.dim() != 4 or k.dim() != 4 or q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:] \
            or q.dtype != k.dtype:
        H = q.shape[1]
        qp = pool(q, bs, "mean_tok_then_grp", grp=H)
        kp = pool(k, bs, "mean_tok_then_grp", grp=k.shape[1])
        out = select(qp, kp, score="dot", convention="own_first", topk=topk, causal=causal, need_scores=need_scores,
                     engine=engine)
        if need_scores:
            return out[0][:, 0], out[1][:, 0]
        return out[:, 0]
    # one call: q and k pooled by one launch that also writes the selection's
    # row norms (fbsa_select_mean_pooled), then the MFMA selection
    _require_cuda(q, k)
    q, k = _pool_input(q), _pool_input(k)
    B, H, L, D = q.shape
    nblk = (L + bs - 1) // bs
    dq = _pool_desc(q, bs, "mean_tok_then_grp", H, None)
    dk = _pool_desc(k, bs, "mean_tok_then_grp", k.shape[1], None)
    kk = budget("own_first", topk, nblk)
    d = _lib.SelectDesc()
    d.dtype = _dtype_code(q)
    d.score, d.convention = _lib.SCORE_DOT, _lib.SEL_OWN_FIRST
    d.causal, d.sink, d.flags = 1 if causal else 0, 0, 0
    d.B, d.H, d.nblk, d.D, d.topk, d.kk = B, 1, nblk, D, topk, kk
    qp = torch.empty(B, 1, nblk, D, dtype=q.dtype, device=q.device)
    kp = torch.empty_like(qp)
    sel = torch.empty(B, 1, nblk, kk, dtype=torch.int32, device=q.device)
    sc = torch.empty(B, 1, nblk, kk, dtype=torch.float32, device=q.device) if need_scores else None
    lib = _lib.load()
    nbytes = lib.fbsa_select_workspace_bytes(d)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
    _lib.check(lib.fbsa_select_mean_pooled(dq, _ptr(q), _ptr(qp), dk, _ptr(k), _ptr(kp), d, _ptr(sel), _ptr(sc),
                                           _ptr(ws), nbytes, _stream()), "fbsa_select_mean_pooled")
    if need_scores:
        return sel[:, 0], sc[:, 0]
    return sel[:, 0]


def select_quest(q, k, bs, topk, sink=True, l_valid=None, engine="auto"):
    """SelectMax (src/qwen_blocksparse.py:107-121): Quest upper-bound scores
    relu(qpool).kmax + min(qpool,0).kmin per KV head, then ``_finish``.
    Returns idx (B, Hkv, nblk, kk) int32."""
    Hkv = k.shape[1]
    grp = q.shape[1] // Hkv
    qpool = pool(q, bs, "mean_grp_then_tok", grp=grp, l_valid=l_valid)
    kmin, kmax = pool(k, bs, "minmax", l_valid=l_valid)
    return select(qpool, kmax, kmin, score="quest", convention="sorted_sink", topk=topk, sink=sink, engine=engine)


def _pool_last_token(q, bs, grp):
    """Last token of every query block, averaged over the GQA group:
    ``q.view(B,Hkv,grp,nblk,bs,d).mean(2)[:, :, :, -1, :]``
    (src/qwen_blocksparse.py:259). A ragged last block's last token is the zero
    padding. Pools the strided view of those tokens with bs = 1."""
    B, Hq, L, D = q.shape
    nblk = (L + bs - 1) // bs
    full = L // bs
    out = torch.zeros(B, Hq // grp, nblk, D, dtype=q.dtype, device=q.device)
    if full:
        out[:, :, :full] = pool(q[:, :, bs - 1:full * bs:bs], 1, "mean_grp_then_tok", grp=grp)
    return out


def select_quest_lasttok(q, k, bs, topk, sink=True, engine="auto"):
    """SelectLastTok (src/qwen_blocksparse.py:244-264): the Quest score of each
    query block's last token (mean over its GQA group) against the per-block
    key min/max, then ``_finish``. Returns idx (B, Hkv, nblk, kk) int32."""
    Hkv = k.shape[1]
    grp = q.shape[1] // Hkv
    qlast = _pool_last_token(q, bs, grp)
    kmin, kmax = pool(k, bs, "minmax")
    return select(qlast, kmax, kmin, score="quest", convention="sorted_sink", topk=topk, sink=sink, engine=engine)


def select_learned(q, k, Wq, Wk, bs, topk, sink=True, scale=None, minmax=False, engine="auto"):
    """SelectLearned / SelectLearnedMinMax (src/qwen_blocksparse.py:168-213):
    block-pooled q (group mean, then token mean) and k (token mean, or the
    per-block [kmin, kmax]) projected through Wq / Wk (torch matmuls, as the
    reference), then the top-k of scale * sq.sk^T with ``_finish``. A positive
    scale does not change the order; the selection streams rnd(sq.sk) (exact,
    rounded to the operand dtype) and never forms the nblk x nblk matrix.
    Returns idx (B, Hkv, nblk, kk) int32."""
    Hkv = k.shape[1]
    grp = q.shape[1] // Hkv
    scale = float(Wq.shape[1] ** -0.5) if scale is None else float(scale)
    qpool = pool(q, bs, "mean_grp_then_tok", grp=grp)
    if minmax:
        kmin, kmax = pool(k, bs, "minmax")
        kfeat = torch.cat([kmin, kmax], dim=-1)
    else:
        kfeat = pool(k, bs, "mean_tok_then_grp", grp=1)
    sq = qpool.to(Wq.dtype) @ Wq
    sk = kfeat.to(Wk.dtype) @ Wk
    if scale < 0:
        sk = -sk  # rnd(-x) = -rnd(x): the order of scale * s is the order of -s
    elif scale == 0:
        sq = torch.zeros_like(sq)  # every score is 0
    return select(sq.contiguous(), sk.contiguous(), score="dot", convention="sorted_sink", topk=topk, sink=sink,
                  engine=engine)



def select_qmax(a, b1, b2, tok, *, topk, convention="sorted_sink", sink=True, cand=None, engine="auto"):
    """Row-block max Quest selection (``fbsa_select_qmax``).

    a: (B,H,La,D) query vectors, block i = vectors [i*tok, (i+1)*tok) (vectors
    at or past La count as zero); b1 = kmax, b2 = kmin (B,H,nblk,D). score(i,j)
    = max over block i's vectors of rnd(rnd(relu(a).b1_j) + rnd(min(a,0).b2_j))
    over j <= i, or over row i's entries of ``cand`` (B,H,nblk,M) int32.
    convention 'sorted_sink' (``_finish``, src/qwen_blocksparse.py:87-99) or
    'sorted_topk' (the bare ascending top-k set: SelectTwoStage's candidate
    stage, src/qwen_blocksparse.py:289-290). engine "auto" brackets 16-bit scores
    on MFMA and computes exactly only what the top-k needs; "fp64" computes
    every score in float64 -- identical results. Returns int32 (B,H,nblk,kk).
    """
    _require_cuda(a, b1, b2)
    if a.dim() != 4 or b1.dim() != 4 or b1.shape != b2.shape or a.shape[:2] != b1.shape[:2] \
            or a.shape[3] != b1.shape[3]:
        raise ValueError("fbsa.select_qmax: a (B,H,La,D), b1/b2 (B,H,nblk,D) expected")
    if a.dtype != b1.dtype or b2.dtype != a.dtype:
        raise ValueError("fbsa.select_qmax: operands must share a dtype")
    B, H, La, D = a.shape
    nblk = b1.shape[2]
    a, b1, b2 = a.contiguous(), b1.contiguous(), b2.contiguous()
    d = _lib.QmaxDesc()
    d.dtype = _dtype_code(a)
    d.convention = {"sorted_sink": _lib.SEL_SORTED_SINK, "sorted_topk": _lib.SEL_SORTED_TOPK}[convention]
    d.sink = 1 if (sink and convention == "sorted_sink") else 0
    d.flags = _lib.QMAX_EXACT if engine == "fp64" else 0
    k_eff = min(topk, nblk)
    kk = k_eff + 1 + d.sink if convention == "sorted_sink" else k_eff
    d.B, d.H, d.nblk, d.D, d.tok, d.la, d.topk, d.kk = B, H, nblk, D, tok, La, topk, kk
    if cand is not None:
        _require_cuda(cand)
        if cand.dim() != 4 or cand.shape[:3] != (B, H, nblk) or cand.dtype != torch.int32:
            raise ValueError(f"fbsa.select_qmax: cand must be int32 {(B, H, nblk)} + (M,)")
        cand = cand.contiguous()
        d.ncand = cand.shape[3]
    sel = torch.empty(B, H, nblk, kk, dtype=torch.int32, device=a.device)
    lib = _lib.load()
    nbytes = lib.fbsa_select_qmax_workspace_bytes(d)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
    _lib.check(lib.fbsa_select_qmax(d, _ptr(a), _ptr(b1), _ptr(b2), _ptr(cand), _ptr(sel), _ptr(ws), nbytes,
                                    _stream()), "fbsa_select_qmax")
    return sel


def select_quest_qmax(q, k, bs, topk, sink=True, engine="auto"):
    """SelectMaxQMax (src/qwen_blocksparse.py:216-241): the Quest score maxed
    over each query block's tokens (each token first averaged over its GQA
    group, rounded) against the per-block key min/max, then ``_finish``. The
    reference loops over query blocks; here one kernel scores every block.
    Returns idx (B, Hkv, nblk, kk) int32."""
    Hkv = k.shape[1]
    grp = q.shape[1] // Hkv
    qg = pool(q, 1, "mean_grp_then_tok", grp=grp)
    kmin, kmax = pool(k, bs, "minmax")
    return select_qmax(qg, kmax, kmin, bs, topk=topk, sink=sink, engine=engine)


def select_two_stage(q, k, bs, topk, sink=True, over=4, engine="auto"):
    """SelectTwoStage (src/qwen_blocksparse.py:267-299): candidates = the top
    M = min(over*topk, nblk) blocks by the block-mean Quest score (the
    SelectMax score), then the token-max Quest score over the candidates
    only, then ``_finish``. Returns idx (B, Hkv, nblk, kk) int32."""
    Hkv = k.shape[1]
    grp = q.shape[1] // Hkv
    qg = pool(q, 1, "mean_grp_then_tok", grp=grp)
    qpool = pool(qg, bs, "mean_tok_then_grp", grp=1)
    kmin, kmax = pool(k, bs, "minmax")
    nblk = kmax.shape[2]
    m = min(over * topk, nblk)
    cand = select_qmax(qpool, kmax, kmin, 1, topk=m, convention="sorted_topk", engine=engine)
    return select_qmax(qg, kmax, kmin, bs, topk=topk, sink=sink, cand=cand, engine=engine)
