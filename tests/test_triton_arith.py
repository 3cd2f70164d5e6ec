"""CPU: the reference kernel's own arithmetic (oracle/triton_arith.py) against the exact gradient.

Pins the restatement (TF32 rounding; with every rounding off it is the exact
gradient of ``oracle/attn.bwd``) and records how far the reference's rounding
points -- TF32 dots, fp32 D, and dK / dV summed by bf16 atomic adds into bf16
tensors (``src/triton_kernel.py:132-150,168-179``) -- land from the exact
gradient on a key block read by a long list of query rows. The GPU build sums
such lists in fp32 and is checked against the absolute bf16 bar there
(``tests/test_gpu_bwd.py``)."""
import numpy as np
import torch

from oracle import attn as oattn, triton_arith as ta
from _util import randn, np64, OUT_ROUND, TOL


def test_round_tf32():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100000) * np.exp2(rng.integers(-20, 20, 100000))
    r = ta.round_tf32(x)
    u = r.astype(np.float32).view(np.uint32)
    assert not np.any(u & 0x1FFF)                                   # 10 stored mantissa bits
    x32 = x.astype(np.float32).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.abs(x32))) - 10)
    assert np.all(np.abs(r - x32) <= ulp / 2)                        # nearest
    ties = np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11, -(1 + 2 ** -11)])
    assert ta.round_tf32(ties).tolist() == [1.0, 1 + 2 ** -9, -1.0]  # ties to even


def _case(seed, H, Hkv, N, D, bs, kk, long_list):
    g = torch.Generator().manual_seed(seed)
    q, do = (np64(randn(g, (1, H, N, D), "bf16")) for _ in range(2))
    k, v = (np64(randn(g, (1, Hkv, N, D), "bf16")) for _ in range(2))
    nblk = N // bs
    if long_list:
        sel = np.zeros((nblk, kk), np.int64)                         # every content slot reads block 0
    else:
        sel = torch.randint(0, nblk, (nblk, kk), generator=g).numpy()
    sel[:, 0] = np.arange(nblk)
    return q, k, v, do, sel


def test_exact_mode_is_the_oracle_gradient():
    for mask, gated, hkv in (("none", False, 2), ("slot_causal", True, 2), ("none", True, 1)):
        q, k, v, do, sel = _case(1, 2, hkv, 256, 32, 16, 5, False)
        gate = np.log(np.random.default_rng(2).uniform(0.1, 1.0, sel.shape)) if gated else None
        got = ta.bwd(q[0], k[0], v[0], sel, do[0], mask, gate=gate, exact=True)
        ref = oattn.bwd(q, k, v, sel[None, None], do, mask, gate=None if gate is None else gate[None, None])
        for a, b in zip(got, ref[:3]):
            assert np.max(np.abs(a - b[0])) < 1e-9


def test_reference_arithmetic_on_a_long_list():
    # B1 H2 N1024 D64 bs16, kk 9, mask none: block 0 is read by every content
    # slot of every row (8 * 64 + 1 = 513 entries per head). The reference's
    # bf16 atomics round the running dK / dV sums to bf16 after every addition
    q, k, v, do, sel = _case(8, 2, 2, 1024, 64, 16, 9, True)
    got = ta.bwd(q[0], k[0], v[0], sel, do[0], "none")
    ref = oattn.bwd(q, k, v, sel[None, None], do, "none")
    errs = {}
    for n, a, b in zip(("dq", "dk", "dv"), got, ref[:3]):
        b = b[0]
        errs[n] = float(np.max(np.abs(a - b) - OUT_ROUND["bf16"] * np.abs(b)))
        print(f"  reference arithmetic {n}: max_abs(beyond output rounding)={errs[n]:.3e} "
              f"max|ref|={float(np.max(np.abs(b))):.2f}", flush=True)
    # dq sums in fp32 and meets the bar; the atomically summed dk / dv of the
    # long list miss it by far
    assert errs["dq"] <= TOL["bf16"]["max_abs"]
    assert errs["dk"] > 10 * TOL["bf16"]["max_abs"] and errs["dv"] > 10 * TOL["bf16"]["max_abs"]
