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
working. ``CentroidSSA`` and ``LSHBucketSSA`` (``:204-513``) keep their
constructors, parameters and hooks; their routing is small torch work on the
device and their attention runs on the same fused kernel.
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


def _bucket_members(home, n_buckets, cap):
    """Fixed-capacity buckets: home (B, n) bucket id per block -> (B, n_buckets,
    cap) member block ids in ascending block order, -1 for an unused place;
    a block after the first cap members of its bucket is left out."""
    B, n = home.shape
    dev = home.device
    before = (F.one_hot(home, n_buckets).cumsum(1) - 1).gather(2, home.unsqueeze(-1)).squeeze(-1)
    keep = before < cap
    members = torch.full((B, n_buckets, cap), -1, dtype=torch.long, device=dev)
    rows = torch.arange(B, device=dev).view(B, 1).expand(B, n)
    ids = torch.arange(n, device=dev).view(1, n).expand(B, n)
    members[rows[keep], home[keep], before[keep]] = ids[keep]
    return members


def _attend_slots(q, k, v, sel_all, gate_val, gate_on, mask, dtype):
    """Fused attention over per-row slots sel_all (B, nblk, kk) int64 where -1
    marks an empty slot: empty slots get a -inf gate (removed from the
    softmax), others 0 or, with gate_on, logsigmoid(gate_val) rounded to the
    model dtype, as the reference's additive mask (differentiable)."""
    valid = sel_all >= 0
    add = torch.zeros(sel_all.shape, device=q.device, dtype=dtype).masked_fill(~valid, float("-inf"))
    if gate_on:
        add = add + F.logsigmoid(gate_val).masked_fill(~valid, 0.0).to(dtype)
    sel = sel_all.clamp(min=0).to(torch.int32).unsqueeze(1)
    return block_sparse_attention(q, k, v, sel.contiguous(), mask=mask, gate=add.unsqueeze(1), gate_grad=True)


class CentroidSSA(nn.Module):
    """Centroid-routed block selection (``src/ssa_model.py:204-336``): each key
    block joins the bucket of its nearest of n_centroids learned centroids
    (first cap members per bucket, in block order), each query block reads the
    buckets of its top-cpq centroids plus its own block, optionally re-ranked
    to refine_topk candidates by the block-mean main q.k; attention is not
    causal. Routing costs O(nblk * C) torch work on the device (no nblk x nblk
    tensor); the attention over the routed blocks runs on the fused kernel,
    with empty slots removed by a -inf gate and, with gate=True, the
    logsigmoid of the query's logit for the key block's centroid added per
    slot (trainable through the kernel's gate gradient)."""

    def __init__(self, d, h, block=64, topk=8, sel_dim=32, n_centroids=16, cpq=2, cap=4, gate=False,
                 refine_topk=None):
        super().__init__()
        self.h, self.dh = h, d // h
        self.block, self.topk = block, topk
        self.cpq, self.cap = cpq, cap
        self.qkv = nn.Linear(d, 3 * d)
        self.o = nn.Linear(d, d)
        self.sel_q = _mlp_sel(d, sel_dim)
        self.sel_k = _mlp_sel(d, sel_dim)
        self.sel_dim = sel_dim
        self.cent = nn.Parameter(torch.randn(n_centroids, sel_dim) * (sel_dim ** -0.5))
        self.refine_topk = refine_topk
        self.gate = gate
        self.last_hit = None
        self.last_block_logits = None
        self.align_q = None
        self.align_k = None

    def forward(self, x, needle_pos=None):
        B, L, D = x.shape
        Bs = self.block
        pad = (Bs - L % Bs) % Bs
        if pad:
            x = F.pad(x, (0, 0, 0, pad))
        Lp = L + pad
        nblk = Lp // Bs
        H, dh = self.h, self.dh
        C = self.cent.shape[0]
        cpq, cap = min(self.cpq, C), min(self.cap, nblk)
        dev = x.device

        q, k, v = (t.view(B, Lp, H, dh).transpose(1, 2) for t in self.qkv(x).chunk(3, -1))
        sq = self.sel_q(x).view(B, nblk, Bs, self.sel_dim).mean(2)
        kf = self.sel_k(x).view(B, nblk, Bs, self.sel_dim)
        sk = torch.maximum(kf.mean(2), kf.max(2).values)
        qc, kc = sq @ self.cent.t(), sk @ self.cent.t()                # (B, nblk, C)
        home = kc.argmax(-1)                                           # centroid of each key block
        routes = qc.topk(cpq, dim=-1).indices                          # query block -> centroids
        self.last_block_logits = qc[:, nblk - 1, :].gather(1, home)

        members = _bucket_members(home, C, cap)                        # (B, C, cap)
        cand = members.gather(1, routes.reshape(B, nblk * cpq, 1).expand(B, nblk * cpq, cap))
        cand = cand.view(B, nblk, cpq * cap)
        own = torch.arange(nblk, device=dev).view(1, nblk, 1)
        cand = cand.masked_fill(cand == own, -1)                       # the own block has slot 0
        if self.refine_topk is not None and self.refine_topk < cpq * cap:
            qm = q.reshape(B, H, nblk, Bs, dh).mean(3).mean(1)
            km = k.reshape(B, H, nblk, Bs, dh).mean(3).mean(1)
            kcand = km[torch.arange(B, device=dev).view(B, 1, 1), cand.clamp(min=0)]
            sc = (qm.unsqueeze(2) * kcand).sum(-1).masked_fill(cand < 0, float("-inf"))
            cand = cand.gather(-1, sc.topk(min(self.refine_topk, cpq * cap), dim=-1).indices)
        sel_all = torch.cat([own.expand(B, nblk, 1), cand], dim=-1)    # (B, nblk, kk), -1 = empty
        gval = None
        if self.gate:
            cen = home.gather(1, sel_all.clamp(min=0).reshape(B, -1)).view(sel_all.shape)
            gval = qc.gather(2, cen)
        out = _attend_slots(q, k, v, sel_all, gval, self.gate, ops.MASK_NONE, q.dtype)
        out = out.transpose(1, 2).reshape(B, Lp, D)[:, :L]

        if needle_pos is not None:
            chosen_last = sel_all[:, nblk - 1, :]
            self.last_hit = (chosen_last == (needle_pos // Bs).unsqueeze(-1)).any(-1).float().mean().item()
            self.align_q = qc[:, nblk - 1, :]
            self.align_k_all = kc
        return self.o(out)


class LSHBucketSSA(nn.Module):
    """LSH-bucketed block selection with a full-fidelity re-score
    (``src/ssa_model.py:339-513``). Selector features are L2-normalised; each
    round hashes every block to the argmax of its projection on fixed (or, with
    learn_hash, trained) random planes R; a query block's candidates are the
    first cap members of its bucket in every round (duplicates dropped), scored
    by scale * cos(sq, sk), own block and (causal) future blocks excluded, and
    the top-k kept after the own block. With dense_select the top-k runs over
    all pairs instead, on the streaming selection kernel (no nblk x nblk
    matrix), and learn_hash adds the soft-collision InfoNCE hash loss of
    ``:406-424`` (``last_hash_loss``). Attention runs on the fused kernel:
    own-block causal when causal, empty or -inf picks removed by a -inf gate,
    gate=True adds logsigmoid of the chosen scores."""

    def __init__(self, d, h, block=32, topk=4, sel_dim=32, n_rounds=4, n_buckets=8, cap=8, gate=False,
                 causal=False, scale=None, learn_hash=False, hash_tau=1.0, hash_detach_reps=False):
        super().__init__()
        self.h, self.dh = h, d // h
        self.block, self.topk = block, topk
        self.qkv = nn.Linear(d, 3 * d)
        self.o = nn.Linear(d, d)
        self.sel_q = _mlp_sel(d, sel_dim)
        self.sel_k = _mlp_sel(d, sel_dim)
        self.sel_dim = sel_dim
        self.scale = float(sel_dim ** 0.5) if scale is None else float(scale)
        self.n_rounds, self.n_buckets, self.cap = n_rounds, n_buckets, cap
        self.gate, self.causal = gate, causal
        self.dense_select = False
        self.learn_hash, self.hash_tau = learn_hash, hash_tau
        self.hash_detach_reps = hash_detach_reps
        R0 = torch.randn(sel_dim, n_rounds, n_buckets)
        if learn_hash:
            self.R = nn.Parameter(R0)
        else:
            self.register_buffer("R", R0)
        self.last_hit = None
        self.last_block_logits = None
        self.last_hash_loss = None

    def _hash_loss(self, sq, sk, sel_content, cont_valid):
        """Soft-collision InfoNCE pulling dense-selected key blocks into their
        query block's buckets (train only, O(nblk^2) like dense selection)."""
        B, nblk, _ = sq.shape
        dev = sq.device
        sq_h = sq.detach() if self.hash_detach_reps else sq
        sk_h = sk.detach() if self.hash_detach_reps else sk
        pq = F.softmax(torch.einsum("bns,src->bnrc", sq_h, self.R) / self.hash_tau, -1)
        pk = F.softmax(torch.einsum("bns,src->bnrc", sk_h, self.R) / self.hash_tau, -1)
        coll = torch.einsum("birc,bjrc->bij", pq, pk)                  # expected collisions
        ar = torch.arange(nblk, device=dev)
        cmask = (ar.view(1, nblk) < ar.view(nblk, 1)) if self.causal else (ar.view(1, nblk) != ar.view(nblk, 1))
        cmask = cmask.unsqueeze(0).expand(B, nblk, nblk)
        pos = torch.zeros(B, nblk, nblk, device=dev).scatter_(2, sel_content, cont_valid.float())
        pos = (pos > 0.5) & cmask
        logit = coll.masked_fill(~cmask, float("-inf"))
        num = torch.logsumexp(logit.masked_fill(~pos, float("-inf")), -1)
        den = torch.logsumexp(logit, -1)
        has = pos.any(-1)
        return (den - num)[has].mean() if has.any() else None

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
        NR, NB, cap = self.n_rounds, self.n_buckets, min(self.cap, nblk)

        q, k, v = (t.view(B, Lp, H, dh).transpose(1, 2) for t in self.qkv(x).chunk(3, -1))
        sq = F.normalize(self.sel_q(x).view(B, nblk, Bs, self.sel_dim).mean(2), dim=-1)
        kf = self.sel_k(x).view(B, nblk, Bs, self.sel_dim)
        sk = F.normalize(torch.maximum(kf.mean(2), kf.max(2).values), dim=-1)
        ar = torch.arange(nblk, device=dev)
        self.last_block_logits = self.scale * torch.bmm(sk, sq[:, nblk - 1:nblk].transpose(-1, -2)).squeeze(-1)
        kk_c = min(self.topk, max(1, nblk - 1))

        if self.dense_select:
            if nblk > 1 and kk_c <= selection.MAX_TOPK:
                sel4, _ = selection.select(sq.detach().unsqueeze(1).contiguous(), sk.detach().unsqueeze(1).contiguous(),
                                           score="dot", convention="own_first", topk=kk_c, causal=self.causal,
                                           need_scores=True)
                sel_content = sel4[:, 0, :, 1:].long()
                cont_valid = sel_content != ar.view(1, nblk, 1)         # fills repeat the own block
                if self.causal:
                    cont_valid &= sel_content < ar.view(1, nblk, 1)
            else:
                raw = (sq @ sk.transpose(-1, -2)).masked_fill(ar.view(1, nblk, 1) == ar.view(1, 1, nblk), float("-inf"))
                if self.causal:
                    raw = raw.masked_fill(ar.view(1, 1, nblk) > ar.view(1, nblk, 1), float("-inf"))
                topv, sel_content = raw.topk(kk_c, dim=-1)
                cont_valid = torch.isfinite(topv)
            if self.learn_hash and self.training:
                self.last_hash_loss = self._hash_loss(sq, sk, sel_content, cont_valid)
        else:
            kbkt = torch.einsum("bns,src->bnrc", sk, self.R).argmax(-1)  # (B, nblk, NR)
            qbkt = torch.einsum("bns,src->bnrc", sq, self.R).argmax(-1)
            cand = torch.cat([_bucket_members(kbkt[..., r], NB, cap).gather(
                1, qbkt[..., r].unsqueeze(-1).expand(B, nblk, cap)) for r in range(NR)], dim=-1)  # (B, nblk, P)
            P = cand.shape[-1]
            cc = cand.clamp(min=0)
            # a repeat of an earlier place is dropped; as in the reference the
            # comparison is on clamped ids, so an empty place (-1 -> 0) also
            # drops a later block 0 of the same list
            dup = (cc.unsqueeze(-1) == cc.unsqueeze(-2)) & torch.tril(
                torch.ones(P, P, dtype=torch.bool, device=dev), -1)
            ok = (cand >= 0) & ~dup.any(-1) & (cand != ar.view(1, nblk, 1))
            if self.causal:
                ok &= cand < ar.view(1, nblk, 1)
            sc = (sq.unsqueeze(2) * sk[torch.arange(B, device=dev).view(B, 1, 1), cc]).sum(-1)
            sc = (self.scale * sc).masked_fill(~ok, float("-inf"))
            topv, topi = sc.topk(min(kk_c, P), dim=-1)
            sel_content = cc.gather(-1, topi)
            cont_valid = torch.isfinite(topv)

        sel_all = torch.cat([ar.view(1, nblk, 1).expand(B, nblk, 1),
                             sel_content.masked_fill(~cont_valid, -1)], dim=-1)
        gval = None
        if self.gate:
            # scale * cos(sq_i, sk_j) of each slot, differentiable into the selector
            skj = sk[torch.arange(B, device=dev).view(B, 1, 1), sel_all.clamp(min=0)]
            gval = self.scale * (sq.unsqueeze(2) * skj).sum(-1)
        mask = ops.MASK_SLOT_CAUSAL if self.causal else ops.MASK_NONE
        out = _attend_slots(q, k, v, sel_all, gval, self.gate, mask, q.dtype)
        out = out.transpose(1, 2).reshape(B, Lp, D)[:, :L]

        if needle_pos is not None:
            chosen_last = sel_all[:, nblk - 1, :]
            self.last_hit = (chosen_last == (needle_pos // Bs).unsqueeze(-1)).any(-1).float().mean().item()
        return self.o(out)


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
        """(align_q, align_k_all) of every layer that stashed them: the last
        query block's centroid logits (B, C) and all key blocks' (B, nblk, C),
        set by CentroidSSA when needle_pos is given (``src/ssa_model.py:560-562``);
        train.py builds its centroid InfoNCE routing loss from these pairs."""
        return [(b["attn"].align_q, b["attn"].align_k_all) for b in self.blocks
                if getattr(b["attn"], "align_q", None) is not None]
