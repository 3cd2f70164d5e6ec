"""Drop-in for the reference's ``ssa_model`` attention modules, on gfx950 kernels.

``BlockSparseSSA`` keeps the reference module's constructor, attributes,
state-dict names and training hooks (``src/ssa_model.py:93-201``):

* ctor ``(d, h, block=64, topk=8, sel_dim=32, gate=False, causal=False,
  use_triton=False)``; parameters ``qkv``, ``o``, ``sel_q.{0,2}``,
  ``sel_k.{0,2}`` (2-layer GELU MLP selectors, ``:34-35``);
* ``_scores(x, B, nblk, Bs)`` -> raw (B, nblk, nblk) = max(sq . sk_mean,
  sq . sk_max) (``:113-119``), still available for callers that want the
  dense matrix (``src/bench_crossover.py:43``);
* ``last_block_logits`` (the last query block's raw row), ``last_hit`` (with
  ``needle_pos``), ``distill`` / ``distill_logits`` / ``distill_target``
  (``:138-149``; for 16-bit models with block 64/128 and head dim 64/128/256
  the dense per-block mass comes from the fused block-mass kernel instead of an
  (B, H, L, L) probability matrix).

The forward never forms the nblk x nblk score matrix: the block-pooled
selector features go to the streaming top-k kernel (own block first, then
the top-k content blocks by descending score, diagonal and -- when causal --
future blocks excluded, ``:151-165``), which also returns each chosen
block's score for the log-sigmoid gate (``:189-191``). Attention runs on the
fused block-sparse kernel for both values of ``use_triton``; they differ only
in what the reference's two paths differ in: the gather path
(``use_triton=False``) back-propagates into the gate bias and thus into the
selector MLPs, the fused op (``use_triton=True``) returns no gate gradient
(``src/triton_kernel.py:254``).

``DenseAttention`` and ``TinyTransformer`` are the reference's dense baseline
and toy wrapper (``:38-54``, ``:516-562``), so callers importing them keep
working. The centroid/LSH selectors are not part of this build.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from fbsa_amd import ops, selection
from fbsa_amd.autograd import block_sparse_attention


def _mlp_sel(d, sel_dim):
    return nn.Sequential(nn.Linear(d, sel_dim), nn.GELU(), nn.Linear(sel_dim, sel_dim))


class DenseAttention(nn.Module):
    """Exact softmax attention over all keys (the dense baseline)."""

    def __init__(self, d, h, causal=False):
        super().__init__()
        self.h, self.dh = h, d // h
        self.causal = causal
        self.qkv = nn.Linear(d, 3 * d)
        self.o = nn.Linear(d, d)

    def forward(self, x, needle_pos=None):
        B, L, D = x.shape
        q, k, v = (t.view(B, L, self.h, self.dh).transpose(1, 2) for t in self.qkv(x).chunk(3, -1))
        out = F.scaled_dot_product_attention(q, k, v, is_causal=self.causal)
        return self.o(out.transpose(1, 2).reshape(B, L, D))


class BlockSparseSSA(nn.Module):
    """Content-dependent block-sparse attention: own block + top-k blocks by
    pooled selector scores, exact softmax over the selected blocks."""

    def __init__(self, d, h, block=64, topk=8, sel_dim=32, gate=False, causal=False, use_triton=False):
        super().__init__()
        self.h, self.dh = h, d // h
        self.block, self.topk = block, topk
        self.qkv = nn.Linear(d, 3 * d)
        self.o = nn.Linear(d, d)
        self.sel_q = _mlp_sel(d, sel_dim)
        self.sel_k = _mlp_sel(d, sel_dim)
        self.sel_dim = sel_dim
        self.gate = gate
        self.causal = causal
        self.use_triton = use_triton
        self.distill = False
        self.last_hit = None
        self.last_block_logits = None
        self.distill_logits = None
        self.distill_target = None

    def _pooled(self, x, B, nblk, Bs):
        """Block-pooled selector features (B, nblk, sel_dim): mean of sel_q(x);
        mean and max of sel_k(x) (``src/ssa_model.py:114-117``)."""
        sq = self.sel_q(x).view(B, nblk, Bs, self.sel_dim).mean(2)
        skv = self.sel_k(x).view(B, nblk, Bs, self.sel_dim)
        return sq, skv.mean(2), skv.max(2).values

    def _scores(self, x, B, nblk, Bs):
        sq, sk_mean, sk_max = self._pooled(x, B, nblk, Bs)
        return torch.maximum(sq @ sk_mean.transpose(-1, -2), sq @ sk_max.transpose(-1, -2))

    def _select(self, sq, sk_mean, sk_max):
        """Convention-A selection on the streaming top-k kernel: (sel, chosen scores), (B, 1, nblk, kk)."""
        return selection.select(sq.detach().unsqueeze(1).contiguous(), sk_mean.detach().unsqueeze(1).contiguous(),
                                sk_max.detach().unsqueeze(1).contiguous(), score="max2", convention="own_first",
                                topk=self.topk, causal=self.causal, need_scores=True)

    def forward(self, x, needle_pos=None):
        B, L, D = x.shape
        Bs = self.block
        pad = (Bs - L % Bs) % Bs
        if pad:
            x = F.pad(x, (0, 0, 0, pad))
        Lp = L + pad
        nblk = Lp // Bs
        H, dh = self.h, self.dh
        dev = x.device

        q, k, v = (t.view(B, Lp, H, dh).transpose(1, 2) for t in self.qkv(x).chunk(3, -1))
        sq, sk_mean, sk_max = self._pooled(x, B, nblk, Bs)
        last = sq[:, nblk - 1:nblk]
        self.last_block_logits = torch.maximum(last @ sk_mean.transpose(-1, -2),
                                               last @ sk_max.transpose(-1, -2))[:, 0]

        if self.distill:
            scale = dh ** -0.5
            if q.dtype in (torch.bfloat16, torch.float16) and Bs in (64, 128) and dh in (64, 128, 256):
                # the dense causal per-block mass on the fused kernel: no (B, H, Lp, Lp)
                # matrix; scores rounded as the 16-bit matmul and scale multiply round
                # them, fp32 softmax (the autocast case; without autocast torch's
                # softmax output is additionally rounded to q's dtype)
                mass = ops.block_mass(q.detach(), k.detach(), Bs, scale)
                if not torch.is_autocast_enabled():
                    mass = mass.to(q.dtype)
            else:
                att = (q @ k.transpose(-1, -2)) * scale
                future_tok = torch.triu(torch.ones(Lp, Lp, dtype=torch.bool, device=dev), 1)
                att = att.masked_fill(future_tok, float("-inf")).softmax(-1)
                mass = att.view(B, H, nblk, Bs, nblk, Bs).sum(-1).mean(3)
            self.distill_target = mass.mean(1).detach()
            ar = torch.arange(nblk, device=dev)
            raw = torch.maximum(sq @ sk_mean.transpose(-1, -2), sq @ sk_max.transpose(-1, -2))
            self.distill_logits = raw.masked_fill((ar.view(nblk, 1) < ar.view(1, nblk)).unsqueeze(0), -1e9)

        kk_c = min(self.topk, nblk - 1)
        if kk_c > selection.MAX_TOPK and kk_c == nblk - 1:
            # every block is selected: own block first, the rest in index order
            # (the attention and the gate are invariant to slot order)
            ar = torch.arange(nblk, device=dev)
            others = ar.view(1, nblk).expand(nblk, nblk)[ar.view(nblk, 1) != ar.view(1, nblk)].view(nblk, nblk - 1)
            sel = torch.cat([ar.view(nblk, 1), others], 1).to(torch.int32).view(1, 1, nblk, nblk)
            sel = sel.expand(B, 1, nblk, nblk).contiguous()
            raw = torch.maximum(sq @ sk_mean.transpose(-1, -2), sq @ sk_max.transpose(-1, -2)).detach()
            sel_score = torch.gather(raw, -1, sel[:, 0].long()).float().unsqueeze(1)
        else:
            # own block + top-k content blocks, streamed (no nblk x nblk matrix)
            sel, sel_score = self._select(sq, sk_mean, sk_max)
        gate_bias = None
        if self.gate:
            raw_sel = sel_score[:, 0].to(sq.dtype)
            if torch.is_grad_enabled() and sq.requires_grad:
                # same values, with the gradient of max(sq . sk_mean[j], sq . sk_max[j])
                idx = sel[:, 0].long()
                gm = torch.gather(sk_mean.unsqueeze(1).expand(B, nblk, nblk, self.sel_dim), 2,
                                  idx.unsqueeze(-1).expand(B, nblk, idx.shape[-1], self.sel_dim))
                gx = torch.gather(sk_max.unsqueeze(1).expand(B, nblk, nblk, self.sel_dim), 2,
                                  idx.unsqueeze(-1).expand(B, nblk, idx.shape[-1], self.sel_dim))
                diff = torch.maximum((sq.unsqueeze(2) * gm).sum(-1), (sq.unsqueeze(2) * gx).sum(-1))
                raw_sel = raw_sel + (diff - diff.detach())
            gate_bias = F.logsigmoid(raw_sel).unsqueeze(1)

        mask = ops.MASK_SLOT_CAUSAL if self.causal else ops.MASK_NONE
        out = block_sparse_attention(q, k, v, sel, mask=mask, gate=gate_bias, gate_grad=not self.use_triton)
        out = out.transpose(1, 2).reshape(B, Lp, D)[:, :L]

        if needle_pos is not None:
            chosen_last = sel[:, 0, nblk - 1, :].long()
            self.last_hit = (chosen_last == (needle_pos // Bs).unsqueeze(-1)).any(-1).float().mean().item()
        return self.o(out)


class _NotInThisBuild(nn.Module):
    def __init__(self, *a, **kw):
        raise NotImplementedError(f"{type(self).__name__}: the centroid/LSH selectors are not part of this "
                                  "build (only block-pair selection + fused block-sparse attention)")


class CentroidSSA(_NotInThisBuild):
    pass


class LSHBucketSSA(_NotInThisBuild):
    pass


def _make_attn(d, h, attn, kw):
    if attn == "dense":
        return DenseAttention(d, h, causal=kw.get("causal", False))
    if attn == "centroid":
        return CentroidSSA(d, h, **kw)
    if attn == "lsh":
        return LSHBucketSSA(d, h, **kw)
    return BlockSparseSSA(d, h, **kw)


class TinyTransformer(nn.Module):
    """Pre-LN toy transformer reading out the last position (MQAR), as
    ``src/ssa_model.py:526-562``."""

    def __init__(self, vocab, n_val, d=128, h=4, layers=2, max_len=4096, attn="dense", **kw):
        super().__init__()
        self.emb = nn.Embedding(vocab, d)
        self.pos = nn.Parameter(torch.randn(1, max_len, d) * 0.02)
        self.blocks = nn.ModuleList(nn.ModuleDict({
            "ln1": nn.LayerNorm(d), "attn": _make_attn(d, h, attn, kw),
            "ln2": nn.LayerNorm(d),
            "mlp": nn.Sequential(nn.Linear(d, 4 * d), nn.GELU(), nn.Linear(4 * d, d)),
        }) for _ in range(layers))
        self.head = nn.Linear(d, n_val)

    def forward(self, toks, needle_pos=None):
        x = self.emb(toks) + self.pos[:, :toks.size(1)]
        for b in self.blocks:
            x = x + b["attn"](b["ln1"](x), needle_pos=needle_pos)
            x = x + b["mlp"](b["ln2"](x))
        return self.head(x[:, -1])

    def set_dense_select(self, flag):
        for b in self.blocks:
            if hasattr(b["attn"], "dense_select"):
                b["attn"].dense_select = flag

    def selection_hit(self):
        hs = [b["attn"].last_hit for b in self.blocks if getattr(b["attn"], "last_hit", None) is not None]
        return sum(hs) / len(hs) if hs else None

    def route_logits(self):
        return [b["attn"].last_block_logits for b in self.blocks
                if getattr(b["attn"], "last_block_logits", None) is not None]

    def centroid_align(self):
        return []
