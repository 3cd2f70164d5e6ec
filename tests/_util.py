"""Shared helpers for the parity tests (seeded inputs, dtype rounding, metrics)."""
import numpy as np
import torch

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def randn(gen, shape, dtype, scale=1.0, device="cpu"):
    """fp32 N(0,1) from a torch.Generator, scaled, cast to dtype."""
    x = torch.randn(*shape, generator=gen, dtype=torch.float32) * scale
    return x.to(TORCH_DT[dtype] if isinstance(dtype, str) else dtype).to(device)


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# north_star tolerances: fp32 1e-4 max-abs; bf16 2e-2 max-abs and 1e-2 relative L2.
# A 16-bit output carries its own storage rounding (half an ulp: <= 2^-8 |x|
# for bf16, 2^-11 |x| for fp16), which the max-abs bound adds elementwise:
# |got - ref| <= max_abs + OUT_ROUND * |ref|.
TOL = {"f32": dict(max_abs=1e-4, rel_l2=1e-5), "bf16": dict(max_abs=2e-2, rel_l2=1e-2),
       "f16": dict(max_abs=5e-3, rel_l2=3e-3)}
OUT_ROUND = {"f32": 0.0, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}


def assert_close(got, ref, dtype, what, scale=1.0):
    """Parity check against the float64 oracle; returns (excess max-abs, rel-L2)."""
    t = TOL[dtype]
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    excess = float(np.max(np.abs(got - ref) - OUT_ROUND[dtype] * np.abs(ref))) if got.size else 0.0
    rl = rel_l2(got, ref)
    assert excess <= t["max_abs"] * scale and rl <= t["rel_l2"] * max(scale, 1.0), \
        f"{what}: max_abs(beyond output rounding)={excess:.3e} rel_l2={rl:.3e} (tol {t}, scale {scale})"
    return excess, rl
