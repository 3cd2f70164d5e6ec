"""Drop-in for the reference's ``triton_kernel`` module, on gfx950 HIP kernels.

Same names, arguments and conventions as ``src/triton_kernel.py``:

* ``bsattn_forward(q, k, v, sel, gate_bias=None, causal=False) -> o``
  (``src/triton_kernel.py:184-207``): q, k, v (B, H, L, dh); sel (B, nblk, kk)
  key-block ids shared by every head, slot 0 the query block's own block;
  gate_bias (B, nblk, kk) added to every score of a slot after the 1/sqrt(dh)
  scale; causal: slot 0 triangular (key row <= query row), slots > 0 valid
  only for blocks strictly before the query block (``:57-61``).
* ``bsattn_backward(q, k, v, sel, o, do, gate_bias=None, causal=False)
  -> (dQ, dK, dV)`` (``:210-234``), here without atomics (bitwise repeatable).
* ``BSAttnFunction`` / ``bsattn`` (``:237-259``): autograd op returning
  ``None`` for the gradient of sel, gate_bias and causal.

No Triton is involved: every call runs the library's HIP kernels on the
current stream. Tensors must be on the GPU.
"""
import torch

from fbsa_amd import ops
from fbsa_amd.autograd import BSAttnFunction, bsattn  # noqa: F401


def _shapes(q, sel):
    B, H, L, dh = q.shape
    nblk = sel.shape[1]
    if nblk == 0 or L % nblk:
        raise AssertionError(f"L={L} must be a multiple of nblk={nblk}")
    return B, H, L, dh, nblk


def bsattn_forward(q, k, v, sel, gate_bias=None, causal=False):
    _shapes(q, sel)
    mask = ops.MASK_SLOT_CAUSAL if causal else ops.MASK_NONE
    gate = gate_bias.unsqueeze(1) if gate_bias is not None else None
    return ops.attention_forward(q, k, v, sel.to(torch.int32).unsqueeze(1), mask=mask, gate=gate)


def bsattn_backward(q, k, v, sel, o, do, gate_bias=None, causal=False):
    """Gradients of ``bsattn_forward``. The softmax statistics are recomputed
    by a forward pass (the reference's first backward pass does the same)."""
    _shapes(q, sel)
    mask = ops.MASK_SLOT_CAUSAL if causal else ops.MASK_NONE
    gate = gate_bias.unsqueeze(1) if gate_bias is not None else None
    sel4 = sel.to(torch.int32).unsqueeze(1)
    _, lse = ops.attention_forward(q, k, v, sel4, mask=mask, gate=gate, need_lse=True)
    dq, dk, dv, _, _ = ops.attention_backward(q, k, v, sel4, o, lse, do, mask=mask, gate=gate)
    return dq, dk, dv
