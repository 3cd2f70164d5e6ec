"""The reference's fused-kernel arithmetic, restated on the CPU (test infrastructure only).

``oracle/attn.py`` is the exact (float64) gradient. This module instead follows
the rounding points of the reference's own Triton backward
(``src/triton_kernel.py:77-181``) on fp32 loads of the 16-bit inputs, so that
its error against the exact gradient can be printed beside the GPU build's:

* every ``tl.dot`` rounds its fp32 operands to TF32 (10 stored mantissa bits;
  Triton's default input precision for fp32 dots on NVIDIA GPUs) and
  accumulates in fp32 (``:126,146-147,168-176``);
* P = exp(S - m) / l and D = sum_j rowsum(P * dP) in fp32 (``:132-150``);
* dS = P (dP - D) scale in fp32 (``:170``);
* each (query block, slot) pair's dV and dK tiles are cast to the output
  dtype and added into the bf16 dK / dV tensors by ``tl.atomic_add``
  (``:172-179``): every addition rounds the running sum to bf16. The order of
  the atomics is not fixed on the GPU; this restatement adds in program order
  (query block, then slot), which changes the rounding pattern, not its size;
* dQ accumulates in fp32 over the slots and is stored in the output dtype.

GQA (several query heads per K/V head) is restated as one program per query
head adding into its K/V head, the same atomics (the reference kernel has one
K/V head per query head).

``exact=True`` turns every rounding off, which reduces the restatement to the
exact gradient (pinned against ``attn.bwd`` by ``tests/test_triton_arith.py``).
"""
import numpy as np

from .numerics import round_bf16, round_f32


def round_tf32(x):
    """fp32 -> TF32 (10 stored mantissa bits), round to nearest even; float64 out."""
    x32 = np.ascontiguousarray(np.asarray(x, dtype=np.float64).astype(np.float32))
    u = x32.view(np.uint32).astype(np.uint64)
    r = ((u + 0xFFF + ((u >> 13) & 1)) >> 13) << 13
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def bwd(q, k, v, sel, do, mask, gate=None, exact=False):
    """dq, dk, dv of the reference kernel's arithmetic.

    q, do (Hq, N, D); k, v (Hkv, N, D) as float64 arrays of bf16 values; sel
    (nblk, kk) one selection shared by the heads; mask "none" or "slot_causal"
    (``src/triton_kernel.py:56-61``); gate (nblk, kk) additive after the scale.
    Returns float64 arrays holding bf16 values (exact=False)."""
    q, k, v, do = (np.asarray(x, np.float64) for x in (q, k, v, do))
    sel = np.asarray(sel, np.int64)
    Hq, N, D = q.shape
    Hkv = k.shape[0]
    grp = Hq // Hkv
    nblk, kk = sel.shape
    bs = N // nblk
    scale = D ** -0.5 if exact else float(np.float32(D ** -0.5))  # the kernel's constexpr is fp32
    ident = lambda x: x  # noqa: E731
    tf = ident if exact else round_tf32
    f32 = ident if exact else round_f32
    b16 = ident if exact else round_bf16
    g = np.zeros((nblk, kk)) if gate is None else np.asarray(gate, np.float64)
    t = np.arange(bs)
    valid = np.ones((nblk, kk, bs, bs), bool)                      # [i, slot, query t, key u]
    if mask == "slot_causal":
        valid[:, 0] = t[:, None] >= t[None, :]
        valid[:, 1:] &= (sel[:, 1:] < np.arange(nblk)[:, None])[:, :, None, None]
    elif mask != "none":
        raise ValueError(mask)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for h in range(Hq):
        hk = h // grp
        qb = q[h].reshape(nblk, bs, D)
        dob = do[h].reshape(nblk, bs, D)
        kg = k[hk].reshape(nblk, bs, D)[sel]                        # (nblk, kk, bs, D)
        vg = v[hk].reshape(nblk, bs, D)[sel]
        s = f32(f32(np.einsum("itd,isud->istu", tf(qb), tf(kg))) * scale)
        x = np.where(valid, s + g[:, :, None, None], -np.inf)
        m = x.max(axis=(1, 3), keepdims=True)                       # over every key of the row
        p = np.exp(x - m)
        l_ = p.sum(axis=(1, 3), keepdims=True)
        p = f32(p / l_)
        dp = f32(np.einsum("itd,isud->istu", tf(dob), tf(vg)))
        dacc = f32((p * dp).sum(axis=(1, 3), keepdims=True))
        ds = f32(p * (dp - dacc) * scale)
        dq[h] = b16(np.einsum("istu,isud->itd", tf(ds), tf(kg))).reshape(N, D)
        dv_t = b16(np.einsum("istu,itd->isud", tf(p), tf(dob)))    # cast before the atomic
        dk_t = b16(np.einsum("istu,itd->isud", tf(ds), tf(qb)))
        dkh = dk[hk].reshape(nblk, bs, D)
        dvh = dv[hk].reshape(nblk, bs, D)
        for i in range(nblk):
            for sl in range(kk):
                j = sel[i, sl]
                dvh[j] = b16(dvh[j] + dv_t[i, sl])
                dkh[j] = b16(dkh[j] + dk_t[i, sl])
    return dq, dk, dv
