"""Float32 torch restatement of the gather attention, forward and backward,
for full-size GPU checks (test infrastructure only).

The float64 oracle (``oracle/attn.py``) is exact but takes seconds per query
block at the configuration-4 shape, so full-size comparisons (every output
row, dK/dV of the sink block that every row reads) use this fp32 version on
the device instead. It is the reference's gather path
(``src/ssa_model.py:57-90``, ``src/qwen_blocksparse.py:57-84``): the selected
K/V blocks are gathered per query block, scores masked by the same three rules
as the oracle, softmax, P.V, optional sigmoid output gate
(``src/patch_qwen.py:55``); gradients come from torch autograd, chunk by
chunk. ``tests/test_torchref.py`` pins it against the oracle on the CPU.
"""
import torch

MASK_NAMES = ("none", "slot_causal", "token_causal")


def _valid(srow, rows, bs, mask, l_valid):
    """(B, Hs, R, bs_q, kk, bs_k) validity of selections srow (B, Hs, R, kk)."""
    dev = srow.device
    t = torch.arange(bs, device=dev)
    B, Hs, R, kk = srow.shape
    if mask == "none":
        keypos = srow[..., None] * bs + t                                  # (B,Hs,R,kk,bs)
        return (keypos < l_valid)[:, :, :, None].expand(B, Hs, R, bs, kk, bs)
    if mask == "slot_causal":
        v = torch.ones(B, Hs, R, bs, kk, bs, dtype=torch.bool, device=dev)
        v[..., 0, :] = t.view(1, bs) <= t.view(bs, 1)
        if kk > 1:
            v[..., 1:, :] &= (srow[..., 1:] < rows.view(1, 1, R, 1))[:, :, :, None, :, None]
        return v
    if mask == "token_causal":
        keypos = srow[..., None] * bs + t                                  # (B,Hs,R,kk,bs)
        qpos = rows.view(R, 1) * bs + t                                    # (R, bs)
        v = keypos[:, :, :, None] <= qpos.view(1, 1, R, bs, 1, 1)
        v &= (keypos < l_valid)[:, :, :, None]
        earlier = torch.tril(torch.ones(kk, kk, dtype=torch.bool, device=dev), -1)
        dup = ((srow[..., :, None] == srow[..., None, :]) & earlier).any(-1)  # (B,Hs,R,kk)
        return v & ~dup[:, :, :, None, :, None]
    raise ValueError(mask)


def attention(q, k, v, sel, mask, scale=None, gate=None, out_gate=None, l_valid=None, do=None, chunk=16):
    """q (B,Hq,N,D), k/v (B,Hkv,N,D), sel (B,Hs,nblk,kk) with Hs in {1, Hkv},
    gate (B,Hs,nblk,kk) additive per slot, out_gate (B,Hq,N,D). Computes in
    fp32 on q's device. Returns (o, lse) or, with do, (o, lse, dq, dk, dv,
    dout_gate), all fp32. Rows without a valid key give o = 0, lse = -inf."""
    B, Hq, N, D = q.shape
    Hkv = k.shape[1]
    _, Hs, nblk, kk = sel.shape
    bs = N // nblk
    grp = Hq // Hkv
    dev = q.device
    scale = D ** -0.5 if scale is None else scale
    l_valid = N if l_valid is None else l_valid
    sel = sel.to(dev).long()
    kf = k.float().detach().requires_grad_(do is not None)
    vf = v.float().detach().requires_grad_(do is not None)
    o = torch.empty(B, Hq, N, D, device=dev)
    lse = torch.empty(B, Hq, N, device=dev)
    dq = torch.zeros(B, Hq, N, D, device=dev) if do is not None else None
    dog = torch.zeros(B, Hq, N, D, device=dev) if (do is not None and out_gate is not None) else None
    bidx = torch.arange(B, device=dev).view(B, 1, 1, 1)
    hidx = torch.arange(Hkv, device=dev).view(1, Hkv, 1, 1)
    for r0 in range(0, nblk, chunk):
        r1 = min(nblk, r0 + chunk)
        R = r1 - r0
        rows = torch.arange(r0, r1, device=dev)
        tok = slice(r0 * bs, r1 * bs)
        s = sel[:, :, r0:r1].expand(B, Hkv, R, kk)                         # per KV head
        qc = q[:, :, tok].float().reshape(B, Hkv, grp, R, bs, D).detach().requires_grad_(do is not None)
        with torch.set_grad_enabled(do is not None):
            kg = kf.view(B, Hkv, nblk, bs, D)[bidx, hidx, s].reshape(B, Hkv, 1, R, kk * bs, D)
            vg = vf.view(B, Hkv, nblk, bs, D)[bidx, hidx, s].reshape(B, Hkv, 1, R, kk * bs, D)
            lg = torch.matmul(qc, kg.transpose(-1, -2).contiguous()) * scale   # (B,Hkv,grp,R,bs,kk*bs)
            if gate is not None:
                gs = gate.to(dev).float()[:, :, r0:r1].expand(B, Hkv, R, kk)
                lg = lg + gs.repeat_interleave(bs, -1).view(B, Hkv, 1, R, 1, kk * bs)
            ok = _valid(sel[:, :, r0:r1], rows, bs, mask, l_valid).expand(B, Hkv, R, bs, kk, bs)
            ok = ok.reshape(B, Hkv, 1, R, bs, kk * bs)
            lg = lg.masked_fill(~ok, float("-inf"))
            ls = torch.logsumexp(lg, -1)                                   # (B,Hkv,grp,R,bs)
            fin = torch.isfinite(ls)
            p = torch.exp(lg - torch.where(fin, ls, torch.zeros_like(ls)).unsqueeze(-1))
            p = torch.where(fin.unsqueeze(-1), p, torch.zeros_like(p))
            oc = torch.matmul(p, vg)                                       # (B,Hkv,grp,R,bs,D)
            oc = oc.reshape(B, Hq, R * bs, D)
            if out_gate is not None:
                ogc = out_gate[:, :, tok].float().detach().requires_grad_(do is not None)
                oc = oc * torch.sigmoid(ogc)
            o[:, :, tok] = oc.detach()
            lse[:, :, tok] = ls.reshape(B, Hq, R * bs).detach()
            if do is not None:
                (oc * do[:, :, tok].float()).sum().backward()
                dq[:, :, tok] = qc.grad.reshape(B, Hq, R * bs, D)
                if dog is not None:
                    dog[:, :, tok] = ogc.grad
    if do is None:
        return o, lse
    return o, lse, dq, kf.grad, vf.grad, dog
