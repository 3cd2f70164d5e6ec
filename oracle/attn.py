"""Attention oracle: gather block-sparse attention in float64 (test infrastructure only).

Layouts follow the reference: q (B,Hq,N,D), k/v (B,Hkv,N,D) with Hq a multiple
of Hkv, N = nblk*bs. sel (B,Hs,nblk,kk) int with Hs = 1 (one selection shared
by every head: ``src/ssa_model.py:65``, ``src/triton_kernel.py:51``) or Hs = Hkv
(per KV head, shared by its query-head group: ``src/qwen_blocksparse.py:60-78``).
gate (B,Hs,nblk,kk) is an additive bias on every key of a slot, added after the
softmax scale (``src/triton_kernel.py:62-64``; ``src/ssa_model.py:71-74``).

Mask rules (``mask``):

* ``"none"``        -- every key of every slot at a position < L_valid
                       (non-causal BlockSparseSSA and ``bsattn(causal=False)``;
                       duplicates count twice; L_valid < N only for the padded
                       non-causal dense path, ``src/qwen_blocksparse.py:37-41``).
* ``"slot_causal"`` -- slot 0: key row u <= query row t (triu on the own
                       block); slot s>0: whole slot valid iff sel < i.
                       ``src/triton_kernel.py:57-61``; ``src/ssa_model.py:167-183``.
* ``"token_causal"``-- key position sel*bs+u <= query position i*bs+t, key
                       position < L_valid, and the slot is the first
                       occurrence of its block index in the row.
                       ``src/qwen_blocksparse.py:67-72``.

Softmax and products are float64; outputs are float64 (callers round).
"""
import numpy as np

MASKS = ("none", "slot_causal", "token_causal")


def _valid(sel_rows, rows, bs, mask, L_valid):
    """Validity (R, bs_q, kk, bs_k) for query-block rows ``rows`` with
    selections sel_rows (R, kk)."""
    R, kk = sel_rows.shape
    t = np.arange(bs)
    if mask == "none":
        keypos = sel_rows[:, :, None] * bs + t[None, None, :]      # (R, kk, bs)
        return np.broadcast_to((keypos < L_valid)[:, None, :, :], (R, bs, kk, bs)).copy()
    if mask == "slot_causal":
        v = np.ones((R, bs, kk, bs), dtype=bool)
        v[:, :, 0, :] = t[None, None, :] <= t[None, :, None]      # u <= t on slot 0
        if kk > 1:
            blk_ok = sel_rows[:, 1:] < rows[:, None]              # (R, kk-1)
            v[:, :, 1:, :] &= blk_ok[:, None, :, None]
        return v
    if mask == "token_causal":
        keypos = sel_rows[:, :, None] * bs + t[None, None, :]      # (R, kk, bs)
        qpos = rows[:, None] * bs + t[None, :]                     # (R, bs)
        v = keypos[:, None, :, :] <= qpos[:, :, None, None]
        v &= (keypos < L_valid)[:, None, :, :]
        earlier = np.tril(np.ones((kk, kk), dtype=bool), -1)       # s' < s
        dup = ((sel_rows[:, :, None] == sel_rows[:, None, :]) & earlier[None]).any(-1)
        v &= ~dup[:, None, :, None]
        return v
    raise ValueError(mask)


def _chunks(nrows, bs, kk, D, budget=1 << 23):
    per_row = bs * kk * max(bs, D)
    step = max(1, budget // max(1, per_row))
    for r0 in range(0, nrows, step):
        yield r0, min(nrows, r0 + step)


def _head_maps(Hq, Hkv, Hs):
    grp = Hq // Hkv
    if Hs not in (1, Hkv):
        raise ValueError("sel heads must be 1 or Hkv")
    return grp, (lambda hk: 0 if Hs == 1 else hk)


def _sigmoid(x):
    return 0.5 * (1.0 + np.tanh(0.5 * x))


def fwd(q, k, v, sel, mask, scale=None, gate=None, L_valid=None, out_gate=None, rows=None):
    """Forward. Returns (o (B,Hq,R*bs,D), lse (B,Hq,R*bs)) for the query-block
    rows ``rows`` (all by default). o is the un-gated attention times
    sigmoid(out_gate) when out_gate (B,Hq,N,D) is given (``src/patch_qwen.py:55``);
    lse is the natural-log normaliser of the un-gated softmax. A query row with
    no valid key returns o = 0 and lse = -inf."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    sel = np.asarray(sel, dtype=np.int64)
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    _, Hs, nblk, kk = sel.shape
    bs = N // nblk
    assert nblk * bs == N
    grp, hsel = _head_maps(Hq, Hkv, Hs)
    scale = D ** -0.5 if scale is None else scale
    L_valid = N if L_valid is None else L_valid
    rows = np.arange(nblk) if rows is None else np.asarray(rows)
    R = len(rows)
    o = np.zeros((B, Hq, R * bs, D))
    lse = np.full((B, Hq, R * bs), -np.inf)
    for b in range(B):
        for hq in range(Hq):
            hk = hq // grp
            hs = hsel(hk)
            kb = k[b, hk].reshape(nblk, bs, D)
            vb = v[b, hk].reshape(nblk, bs, D)
            qb = q[b, hq].reshape(nblk, bs, D)
            for r0, r1 in _chunks(R, bs, kk, D):
                rr = rows[r0:r1]
                s_rows = sel[b, hs, rr]                          # (r, kk)
                kg, vg = kb[s_rows], vb[s_rows]                  # (r, kk, bs, D)
                lg = np.einsum("rtd,rsud->rtsu", qb[rr], kg) * scale
                if gate is not None:
                    lg = lg + np.asarray(gate, dtype=np.float64)[b, hs, rr][:, None, :, None]
                ok = _valid(s_rows, rr, bs, mask, L_valid)
                lg = np.where(ok, lg, -np.inf)
                m = lg.max(axis=(2, 3))
                m_safe = np.where(np.isfinite(m), m, 0.0)
                p = np.exp(lg - m_safe[:, :, None, None])
                lsum = p.sum(axis=(2, 3))
                out = np.einsum("rtsu,rsud->rtd", p, vg)
                out = np.where(lsum[..., None] > 0, out / np.where(lsum > 0, lsum, 1.0)[..., None], 0.0)
                o[b, hq, r0 * bs:r1 * bs] = out.reshape(-1, D)
                lse[b, hq, r0 * bs:r1 * bs] = np.where(lsum > 0, m_safe + np.log(np.where(lsum > 0, lsum, 1.0)), -np.inf).reshape(-1)
    if out_gate is not None:
        og = np.asarray(out_gate, dtype=np.float64)
        og_rows = og.reshape(B, Hq, nblk, bs, D)[:, :, rows].reshape(B, Hq, R * bs, D)
        o = o * _sigmoid(og_rows)
    return o, lse


def bwd(q, k, v, sel, do, mask, scale=None, gate=None, L_valid=None, out_gate=None, rows=None):
    """Backward of ``fwd`` by explicit softmax calculus (float64).

    Returns dq, dk, dv (shapes of q, k, v), dgate (B,Hs,nblk,kk) and dout_gate
    (B,Hq,N,D or None). dK/dV of a key block sum over every (query block, slot)
    that selected it and over the GQA group (scatter-add, duplicates included),
    which is what the reference's atomics compute (``src/triton_kernel.py:178-179``).
    dgate sums the score gradient over the slot's keys, the block's queries and
    the heads sharing the selection (the gradient the gather path gives the
    gate, ``src/ssa_model.py:72-74``; the fused reference op returns None).

    ``rows`` restricts the computation to the contributions of those query
    blocks (dq and dgate of other rows stay 0; dk/dv hold only those rows'
    contributions -- complete for a key block when ``rows`` covers every row
    that selected it)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(do, dtype=np.float64)
    sel = np.asarray(sel, dtype=np.int64)
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    _, Hs, nblk, kk = sel.shape
    bs = N // nblk
    grp, hsel = _head_maps(Hq, Hkv, Hs)
    scale = D ** -0.5 if scale is None else scale
    L_valid = N if L_valid is None else L_valid
    rows = np.arange(nblk) if rows is None else np.asarray(rows, dtype=np.int64)
    o_r, lse_r = fwd(q, k, v, sel, mask, scale, gate, L_valid, None, rows=rows)   # (B,Hq,R*bs,*)
    R = len(rows)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    dgate = np.zeros(sel.shape)
    dog = None
    do_r = do.reshape(B, Hq, nblk, bs, D)[:, :, rows]                              # (B,Hq,R,bs,D)
    if out_gate is not None:
        og_r = np.asarray(out_gate, dtype=np.float64).reshape(B, Hq, nblk, bs, D)[:, :, rows]
        sg = _sigmoid(og_r)
        dog = np.zeros_like(q)
        dog.reshape(B, Hq, nblk, bs, D)[:, :, rows] = do_r * o_r.reshape(B, Hq, R, bs, D) * sg * (1.0 - sg)
        do_r = do_r * sg
    for b in range(B):
        for hq in range(Hq):
            hk = hq // grp
            hs = hsel(hk)
            kb = k[b, hk].reshape(nblk, bs, D)
            vb = v[b, hk].reshape(nblk, bs, D)
            qb = q[b, hq].reshape(nblk, bs, D)
            dqb = dq[b, hq].reshape(nblk, bs, D)
            dkb = dk[b, hk].reshape(nblk, bs, D)
            dvb = dv[b, hk].reshape(nblk, bs, D)
            ob = o_r[b, hq].reshape(R, bs, D)
            lseb = lse_r[b, hq].reshape(R, bs)
            for r0, r1 in _chunks(R, bs, kk, D):
                rr = rows[r0:r1]
                s_rows = sel[b, hs, rr]
                kg, vg = kb[s_rows], vb[s_rows]
                lg = np.einsum("rtd,rsud->rtsu", qb[rr], kg) * scale
                if gate is not None:
                    lg = lg + np.asarray(gate, dtype=np.float64)[b, hs, rr][:, None, :, None]
                ok = _valid(s_rows, rr, bs, mask, L_valid)
                ls = lseb[r0:r1]
                ls_safe = np.where(np.isfinite(ls), ls, 0.0)
                p = np.where(ok, np.exp(np.where(ok, lg, 0.0) - ls_safe[:, :, None, None]), 0.0)
                p = np.where(np.isfinite(ls)[:, :, None, None], p, 0.0)
                dor = do_r[b, hq, r0:r1]
                Dr = (dor * ob[r0:r1]).sum(-1)                                   # (r, t)
                dp = np.einsum("rtd,rsud->rtsu", dor, vg)
                ds = p * (dp - Dr[:, :, None, None])
                dqb[rr] += scale * np.einsum("rtsu,rsud->rtd", ds, kg)
                np.add.at(dkb, s_rows.reshape(-1),
                          (scale * np.einsum("rtsu,rtd->rsud", ds, qb[rr])).reshape(-1, bs, D))
                np.add.at(dvb, s_rows.reshape(-1),
                          np.einsum("rtsu,rtd->rsud", p, dor).reshape(-1, bs, D))
                dgate[b, hs, rr] += ds.sum(axis=(1, 3))
    return dq, dk, dv, dgate, dog


def fwd_bruteforce(q, k, v, sel, mask, scale=None, gate=None, L_valid=None):
    """Per-token loop over explicitly enumerated valid keys (tiny shapes only).
    Independent of ``fwd``'s vectorised masks: it re-derives validity from the
    reference's per-slot rules token by token."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    sel = np.asarray(sel, dtype=np.int64)
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    _, Hs, nblk, kk = sel.shape
    bs = N // nblk
    grp = Hq // Hkv
    scale = D ** -0.5 if scale is None else scale
    L_valid = N if L_valid is None else L_valid
    o = np.zeros_like(q)
    for b in range(B):
        for hq in range(Hq):
            hk = hq // grp
            hs = 0 if Hs == 1 else hk
            for pos in range(N):
                i, t = divmod(pos, bs)
                logits, vals = [], []
                row = [int(x) for x in sel[b, hs, i]]
                for s, j in enumerate(row):
                    for u in range(bs):
                        kpos = j * bs + u
                        if mask == "slot_causal":
                            ok = (u <= t) if s == 0 else (j < i)
                        elif mask == "token_causal":
                            ok = kpos <= pos and kpos < L_valid and j not in row[:s]
                        else:
                            ok = kpos < L_valid
                        if not ok:
                            continue
                        g = 0.0 if gate is None else float(gate[b, hs, i, s])
                        logits.append(scale * float(q[b, hq, pos] @ k[b, hk, kpos]) + g)
                        vals.append(v[b, hk, kpos])
                if not logits:
                    continue
                lg = np.array(logits)
                w = np.exp(lg - lg.max())
                o[b, hq, pos] = (w[:, None] * np.array(vals)).sum(0) / w.sum()
    return o


def dense(q, k, v, causal, scale=None, L_valid=None):
    """Textbook softmax attention over all keys (GQA by head groups); the
    all-blocks closed form (``scripts/run_all.sh:7-21``,
    ``src/test_qwen_blocksparse.py:10-34``)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    grp = Hq // Hkv
    scale = D ** -0.5 if scale is None else scale
    L_valid = N if L_valid is None else L_valid
    kr = np.repeat(k, grp, axis=1)
    vr = np.repeat(v, grp, axis=1)
    lg = np.einsum("bhtd,bhud->bhtu", q, kr) * scale
    t = np.arange(N)
    ok = np.ones((N, N), dtype=bool)
    if causal:
        ok &= t[None, :] <= t[:, None]
    ok &= t[None, :] < L_valid
    lg = np.where(ok, lg, -np.inf)
    m = lg.max(-1, keepdims=True)
    p = np.exp(lg - m)
    return np.einsum("bhtu,bhud->bhtd", p, vr) / p.sum(-1, keepdims=True)


def block_mass(q, k, bs, scale, dtype):
    """Dense causal per-block attention mass (``capture_mass``,
    ``src/eval_qwen_ppl.py:65-108``): for each query block i and key block j,
    the mean over block i's query rows t of the softmax probability summed over
    block j's keys s <= t, averaged over each KV head's query-head group.
    Scores are rounded as torch's 16-bit matmul and scale multiply round them
    (rnd(rnd(q.k) * scale) in ``dtype``; exact products, float64 sums), the
    softmax is float64. q (B,Hq,L,D), k (B,Hkv,L,D), L = nblk*bs.
    Returns (B, Hkv, nblk, nblk) float64, zero above the diagonal."""
    from .numerics import round_to
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    B, Hq, L, D = q.shape
    Hkv = k.shape[1]
    grp = Hq // Hkv
    nblk = L // bs
    out = np.zeros((B, Hq, nblk, nblk))
    kpos = np.arange(L)
    for h in range(Hq):
        kh = k[:, h // grp]
        for i in range(nblk):
            qi = q[:, h, i * bs:(i + 1) * bs]                       # (B, bs, D)
            s = round_to(round_to(np.einsum("btd,bsd->bts", qi, kh), dtype) * scale, dtype)
            qpos = i * bs + np.arange(bs)
            s = np.where(kpos[None, None, :] > qpos[None, :, None], -np.inf, s)
            s = s - s.max(-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(-1, keepdims=True)
            out[:, h, i] = p.reshape(B, bs, nblk, bs).sum(-1).mean(1)
    return out.reshape(B, Hkv, grp, nblk, nblk).mean(2)

