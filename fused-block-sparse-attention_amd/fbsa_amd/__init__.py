"""fbsa_amd -- MI355X (gfx950) block-pair selection + fused block-sparse attention.

Host side of libfbsa.so. Reference-compatible surfaces live in the sibling
modules ``triton_kernel``, ``ssa_model`` and ``qwen_blocksparse`` of this
directory; this package holds the ctypes binding (``_lib``) and the device ops
(``ops``, ``selection``, ``autograd``).
"""
from . import _lib, ops  # noqa: F401
from .ops import attention_forward  # noqa: F401
