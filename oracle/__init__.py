"""CPU oracle for block-pair selection + fused block-sparse attention.

TEST INFRASTRUCTURE ONLY. This package restates, in numpy, the reference
algorithm of apoc/fused-block-sparse-attention for the hot path
(selection -> fused block-sparse forward -> backward). Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker (or the timed CPU baseline). The product
path (``fbsa_amd``) never imports it and has no CPU fallback.

Modules
-------
numerics : bf16 / fp32 rounding used to mirror torch's rounding points.
select   : pooling (mean / min / max), pooled scores, selection conventions
           A (own block first, ``src/ssa_model.py:151-165``) and
           B (``_finish``, ``src/qwen_blocksparse.py:87-99``), near-tie census.
attn     : gather attention forward/backward in float64 with the reference's
           three masking rules, plus dense closed forms.
triton_arith : the reference Triton backward's own rounding points (TF32
           dots, fp32 D, bf16 atomic sums; ``src/triton_kernel.py:77-181``),
           to print its error beside the build's.

Every function cites the reference file:line it restates. What pins each
function (golden vectors, closed forms, brute force) is listed in
``tests/test_oracle_*.py``.
"""
from . import numerics, select, attn, triton_arith  # noqa: F401
