"""Drop-in for the reference's ``qwen_blocksparse`` module (GQA block-sparse core), on gfx950.

Same surface as ``src/qwen_blocksparse.py``:

* ``blocksparse_forward(q, k, v, *, selector, topk, bs, causal=True,
  scale=None, q_chunk=4)`` (``:29-84``): post-RoPE q (B, Hq, L, d), k/v
  (B, Hkv, L, d); the selector picks key blocks per KV head
  (``.select(q, k) -> (B, Hkv, nblk, kk)``), shared by its query-head group;
  a key is attended iff its position <= the query position, < L, and its
  block is the first occurrence in the row (``:67-72``). With
  ``selector=None`` and ``topk >= nblk`` every block is selected and
  ``causal`` picks causal or full attention (the dense fast path, ``:37-41``).
  ``q_chunk`` is accepted and ignored: the fused kernel never materialises
  the gathered keys, so there is nothing to chunk. The extra keyword
  ``out_gate`` (B, Hq, L, d) applies ``o * sigmoid(out_gate)`` in the
  kernel's epilogue (the Qwen output gate, ``src/patch_qwen.py:55``).
* ``SelectMax`` (``:102-121``): Quest min/max upper-bound selector on the
  pooling and streaming top-k kernels; ``SelectLastTok`` (``:244-264``, the
  same score from each block's last token); ``SelectMaxQMax`` /
  ``SelectTwoStage`` (``:216-241``, ``:267-299``, the score maxed over each
  block's tokens, over all blocks or over block-mean candidates, on the
  row-block max kernel); ``SelectLearned`` /
  ``SelectLearnedMinMax`` (``:168-213``, pooled features through Wq / Wk, the
  projections in torch as in the reference); ``SelectAll`` (``:155-165``).
* ``block_mass`` -- the true block mass ``SelectOracle`` selects from (the
  ``capture_mass`` loop of ``src/eval_qwen_ppl.py:84-95``) on a fused kernel.
* ``_pad_blocks`` and ``_finish`` (``:20-26``, ``:87-99``) and the
  dense-score selectors ``SelectOracle`` / ``SelectRandom`` (``:124-152``),
  kept for callers that build their own score matrix.

Everything runs on the GPU; there is no CPU path.
"""
import torch
import torch.nn.functional as F

from fbsa_amd import ops, selection
from fbsa_amd.autograd import block_sparse_attention


def _pad_blocks(x, bs):
    """Zero-pad the token axis (-2) to a multiple of bs: (x, nblk, pad)."""
    L = x.shape[-2]
    nblk = (L + bs - 1) // bs
    pad = nblk * bs - L
    if pad:
        x = F.pad(x, (0, 0, 0, pad))
    return x, nblk, pad


def blocksparse_forward(q, k, v, *, selector, topk, bs, causal=True, scale=None, q_chunk=4, out_gate=None):
    B, Hq, L, d = q.shape
    Hkv = k.shape[1]
    if Hq % Hkv:
        raise ValueError(f"Hq={Hq} must be a multiple of Hkv={Hkv}")
    scale = d ** -0.5 if scale is None else scale
    nblk = (L + bs - 1) // bs
    if selector is None and topk >= nblk:
        # dense fast path: every block, causal or full, with no block list
        # (the kernels enumerate the blocks themselves; any length)
        sel = ops.DenseSelection(B, nblk)
        mask = ops.MASK_TOKEN_CAUSAL if causal else ops.MASK_NONE
    else:
        idx = selector.select(q, k)
        mask = ops.MASK_TOKEN_CAUSAL
        if tuple(idx.shape[:3]) != (B, Hkv, nblk):
            raise ValueError(f"selector returned {tuple(idx.shape)}, expected ({B}, {Hkv}, {nblk}, kk)")
        sel = idx.to(torch.int32).contiguous()
    qp, _, pad = _pad_blocks(q, bs)
    kp, _, _ = _pad_blocks(k, bs)
    vp, _, _ = _pad_blocks(v, bs)
    og = _pad_blocks(out_gate, bs)[0] if out_gate is not None else None
    out = block_sparse_attention(qp, kp, vp, sel, mask=mask, scale=scale, out_gate=og, l_valid=L)
    return out[..., :L, :] if pad else out


def block_mass(q, k, bs, scale=None):
    """True block attention mass (B, Hkv, nblk, nblk) for ``SelectOracle``: the
    dense causal softmax probability of each query block summed per key block,
    averaged over the block's rows and over each KV head's query heads (the
    ``capture_mass`` loop of src/eval_qwen_ppl.py:84-95, fused on the GPU: no
    L x L matrix, no per-block Python loop). q (B, Hq, L, d) post-RoPE, k
    (B, Hkv, L, d), L a multiple of bs; scale as passed to the attention."""
    B, Hq, L, d = q.shape
    Hkv = k.shape[1]
    m = ops.block_mass(q, k, bs, scale)
    return m.view(B, Hkv, Hq // Hkv, L // bs, L // bs).mean(2)


def _finish(score, topk, sink, B, Hkv, nblk, dev):
    """Causal top-k over a dense (B, Hkv, nblk, nblk) score, non-finite picks
    -> own block, + own (+ sink 0), sorted ascending (``:87-99``)."""
    ar = torch.arange(nblk, device=dev)
    score = score.masked_fill(ar.view(1, 1, nblk, 1) < ar.view(1, 1, 1, nblk), float("-inf"))
    kk = min(topk, nblk)
    topv, topi = score.topk(kk, dim=-1)
    own = ar.view(1, 1, nblk, 1).expand(B, Hkv, nblk, 1)
    topi = torch.where(torch.isfinite(topv), topi, own.expand_as(topi))
    parts = [topi, own]
    if sink:
        parts.append(torch.zeros(B, Hkv, nblk, 1, dtype=torch.long, device=dev))
    return torch.cat(parts, dim=-1).sort(dim=-1).values


class SelectMax:
    """Training-free Quest selector: score(i, j) = relu(qpool_i) . kmax_j +
    min(qpool_i, 0) . kmin_j, qpool the GQA-group-then-token mean, kmin/kmax
    the per-block element-wise extremes; top-k causal + own (+ sink), sorted.
    Pooling and the streaming top-k run on the GPU kernels; the nblk x nblk
    score matrix is never formed."""

    def __init__(self, topk, bs, sink=True):
        self.topk, self.bs, self.sink = topk, bs, sink

    @torch.no_grad()
    def select(self, q, k):
        return selection.select_quest(q, k, self.bs, self.topk, sink=self.sink).long()


class SelectLastTok:
    """SelectMax scored by each query block's last token (its GQA-group mean)
    instead of the block mean (``src/qwen_blocksparse.py:244-264``); pooling and
    the streaming top-k run on the GPU kernels."""

    def __init__(self, topk, bs, sink=True):
        self.topk, self.bs, self.sink = topk, bs, sink

    @torch.no_grad()
    def select(self, q, k):
        return selection.select_quest_lasttok(q, k, self.bs, self.topk, sink=self.sink).long()


class SelectMaxQMax:
    """SelectMax with the Quest score maxed over the query block's tokens
    instead of scored on their mean: score(i, j) = max_t relu(q_t) . kmax_j +
    min(q_t, 0) . kmin_j, q_t the GQA-group mean of token t
    (``src/qwen_blocksparse.py:216-241``). One kernel scores every query block
    (brackets on the matrix cores, exact float64 where the top-k needs it)
    instead of the reference's loop over blocks."""

    def __init__(self, topk, bs, sink=True):
        self.topk, self.bs, self.sink = topk, bs, sink

    @torch.no_grad()
    def select(self, q, k):
        return selection.select_quest_qmax(q, k, self.bs, self.topk, sink=self.sink).long()


class SelectTwoStage:
    """Two-stage Quest selection (``src/qwen_blocksparse.py:267-299``): the
    block-mean score picks over * topk candidates, the token-max score
    re-ranks them, then top-k causal + own (+ sink), sorted."""

    def __init__(self, topk, bs, sink=True, over=4):
        self.topk, self.bs, self.sink, self.over = topk, bs, sink, over

    @torch.no_grad()
    def select(self, q, k):
        return selection.select_two_stage(q, k, self.bs, self.topk, sink=self.sink, over=self.over).long()


class SelectLearned:
    """Learned selector: block-pooled q / k projected through Wq / Wk (d, sel_dim),
    top-k of scale * sq.sk^T (``src/qwen_blocksparse.py:168-187``)."""

    def __init__(self, Wq, Wk, topk, bs, sink=True, scale=None):
        self.Wq, self.Wk = Wq, Wk
        self.topk, self.bs, self.sink = topk, bs, sink
        self.scale = float(Wq.shape[1] ** -0.5) if scale is None else float(scale)

    @torch.no_grad()
    def select(self, q, k):
        return selection.select_learned(q, k, self.Wq, self.Wk, self.bs, self.topk, sink=self.sink,
                                        scale=self.scale).long()


class SelectLearnedMinMax(SelectLearned):
    """SelectLearned with the per-block key [kmin, kmax] (2d features) through Wk
    (2d, sel_dim) instead of the key mean (``src/qwen_blocksparse.py:190-213``)."""

    @torch.no_grad()
    def select(self, q, k):
        return selection.select_learned(q, k, self.Wq, self.Wk, self.bs, self.topk, sink=self.sink,
                                        scale=self.scale, minmax=True).long()


class SelectAll:
    """Every block for every query block (masked causally by the attention rule)."""

    def __init__(self, bs):
        self.bs = bs

    @torch.no_grad()
    def select(self, q, k):
        B, _, L, _ = q.shape
        nblk = (L + self.bs - 1) // self.bs
        return torch.arange(nblk, device=q.device).view(1, 1, 1, nblk).expand(B, k.shape[1], nblk, nblk).contiguous()


class SelectOracle:
    """Top-k key blocks by a supplied per-block attention mass (B, Hkv, nblk, nblk)."""

    def __init__(self, topk, bs, sink=True, mass=None):
        self.topk, self.bs, self.sink, self.mass = topk, bs, sink, mass

    @torch.no_grad()
    def select_from_mass(self, mass):
        B, Hkv, nblk, _ = mass.shape
        return _finish(mass.clone(), self.topk, self.sink, B, Hkv, nblk, mass.device)

    @torch.no_grad()
    def select(self, q, k):
        if self.mass is None:
            raise ValueError("SelectOracle needs a per-layer mass")
        return self.select_from_mass(self.mass)


class SelectRandom:
    """Random causal blocks (lower-bound baseline), seeded per call."""

    def __init__(self, topk, bs, sink=True, seed=0):
        self.topk, self.bs, self.sink, self.seed = topk, bs, sink, seed

    @torch.no_grad()
    def select(self, q, k):
        B, _, L, _ = q.shape
        Hkv = k.shape[1]
        nblk = (L + self.bs - 1) // self.bs
        g = torch.Generator(device=q.device).manual_seed(self.seed)
        score = torch.rand(B, Hkv, nblk, nblk, generator=g, device=q.device)
        return _finish(score, self.topk, self.sink, B, Hkv, nblk, q.device)
