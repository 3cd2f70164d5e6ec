"""Autograd wrappers of the fused block-sparse attention (forward + atomics-free backward).

``BSAttnFunction`` / ``bsattn`` keep the reference op's contract
(``src/triton_kernel.py:237-259``): inputs (q, k, v, sel, gate_bias, causal),
sel (B, nblk, kk) shared by every head, slot 0 = own block, gate_bias
(B, nblk, kk) additive after the 1/sqrt(D) scale, and ``None`` as the gradient
of sel, gate_bias and causal.

``BlockSparseAttention`` is the general form used by the module and GQA
surfaces: any mask rule, scale, padding length, per-KV-head selection, an
optional sigmoid output gate, and a gradient for the gate bias (the gradient
the reference's gather path gives it, ``src/ssa_model.py:72-74``).
"""
import torch

from . import ops


class BlockSparseAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, sel, gate, out_gate, mask, scale, l_valid, gate_grad):
        o, lse = ops.attention_forward(q, k, v, sel, mask=mask, scale=scale, gate=gate, l_valid=l_valid,
                                       out_gate=out_gate, need_lse=True)
        ctx.dense = sel if isinstance(sel, ops.DenseSelection) else None
        ctx.save_for_backward(q, k, v, None if ctx.dense is not None else sel, gate, out_gate, o, lse)
        ctx.mask, ctx.scale, ctx.l_valid, ctx.gate_grad = mask, scale, l_valid, gate_grad
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, sel, gate, out_gate, o, lse = ctx.saved_tensors
        if ctx.dense is not None:
            sel = ctx.dense
        need_dg = gate is not None and ctx.gate_grad and ctx.needs_input_grad[4]
        dq, dk, dv, dgate, dog = ops.attention_backward(
            q, k, v, sel, o, lse, do, mask=ctx.mask, scale=ctx.scale, gate=gate, l_valid=ctx.l_valid,
            out_gate=out_gate, need_dgate=need_dg)
        if dgate is not None:
            dgate = dgate.to(gate.dtype)
        return dq, dk, dv, None, dgate, dog, None, None, None, None


def block_sparse_attention(q, k, v, sel, *, mask, scale=None, gate=None, out_gate=None, l_valid=None,
                           gate_grad=True):
    """Differentiable fused block-sparse attention; sel is (B, Hsel, nblk, kk)
    or an ``ops.DenseSelection`` (every block)."""
    return BlockSparseAttention.apply(q, k, v, sel, gate, out_gate, mask, scale, l_valid, gate_grad)


class BSAttnFunction(torch.autograd.Function):
    """Reference-compatible op: ``BSAttnFunction.apply(q, k, v, sel, gate_bias, causal)``."""

    @staticmethod
    def forward(ctx, q, k, v, sel, gate_bias, causal):
        mask = ops.MASK_SLOT_CAUSAL if causal else ops.MASK_NONE
        sel4 = sel.to(torch.int32).unsqueeze(1)
        gate4 = gate_bias.unsqueeze(1) if gate_bias is not None else None
        o, lse = ops.attention_forward(q, k, v, sel4, mask=mask, gate=gate4, need_lse=True)
        ctx.save_for_backward(q, k, v, sel4, gate4 if gate4 is not None else torch.empty(0, device=q.device),
                              o, lse)
        ctx.has_gate, ctx.mask = gate_bias is not None, mask
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, sel4, gate4, o, lse = ctx.saved_tensors
        dq, dk, dv, _, _ = ops.attention_backward(q, k, v, sel4, o, lse, do, mask=ctx.mask,
                                                  gate=gate4 if ctx.has_gate else None)
        return dq, dk, dv, None, None, None


def bsattn(q, k, v, sel, gate_bias=None, causal=False):
    """Autograd-aware block-sparse attention (``src/triton_kernel.py:257-259``)."""
    return BSAttnFunction.apply(q, k, v, sel, gate_bias, causal)
