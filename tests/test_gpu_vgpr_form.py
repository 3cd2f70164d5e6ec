"""GPU: the backward built with MFMA results in VGPRs (libfbsa.so, hipcc
-mllvm -amdgpu-mfma-vgpr-form) against the same sources built with the
default AGPR accumulators (libfbsa_bwdagpr.so): the register class of the
accumulators does not change the arithmetic, so every gradient must be
bit-identical. Guards against a hazard the option could introduce between an
MFMA and the inline-asm LDS reads that follow it."""
import os

import numpy as np
import pytest
import torch

from _util import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
MC = {"slot_causal": 1, "token_causal": 2}


def _libs():
    from fbsa_amd import _lib
    path = os.path.join(os.path.dirname(_lib.LIB_PATH), "libfbsa_bwdagpr.so")
    return _lib, _lib.open_library(path)


def _both(run):
    lib, alt = _libs()
    a = run()
    prev = lib.use(alt)
    try:
        b = run()
    finally:
        lib.use(prev)
    torch.cuda.synchronize()
    return a, b


def _same(name, a, b):
    for n, x, y in zip(("dq", "dk", "dv", "dgate", "dout_gate"), a, b):
        if x is None:
            assert y is None
            continue
        eq = torch.equal(x, y)
        print(f"[vgpr-form] {name} {n}: bit-identical={eq}", flush=True)
        assert eq, f"{name} {n} differs between the VGPR and AGPR backward builds"


def _case(q, k, v, sel, do, mask, scale=None, gate=None, out_gate=None, need_dgate=False):
    from fbsa_amd import ops
    o, lse = ops.attention_forward(q, k, v, sel, mask=MC[mask], scale=scale, gate=gate, out_gate=out_gate,
                                   need_lse=True)
    return _both(lambda: ops.attention_backward(q, k, v, sel, o, lse, do, mask=MC[mask], scale=scale, gate=gate,
                                                out_gate=out_gate, need_dgate=need_dgate))


def test_config4_shape():
    import qwen_blocksparse as qb
    from bench import rope_partial
    B, Hq, Hkv, N, D, bs, topk = 1, 16, 2, 65536, 256, 128, 32
    g = torch.Generator(device=DEV).manual_seed(11)
    rn = lambda *s: torch.randn(*s, generator=g, device=DEV).to(torch.bfloat16)  # noqa: E731
    q, k = rope_partial(rn(B, Hq, N, D)), rope_partial(rn(B, Hkv, N, D))
    v, og, do = rn(B, Hkv, N, D), rn(B, Hq, N, D), rn(B, Hq, N, D)
    idx = qb.SelectMax(topk=topk, bs=bs, sink=True).select(q, k).to(torch.int32).contiguous()
    a, b = _case(q, k, v, idx, do, "token_causal", scale=D ** -0.5, out_gate=og)
    _same("config 4", a, b)


def test_d256_fp32_sink_segments():
    g = torch.Generator().manual_seed(7)
    B, Hq, Hkv, nblk, D, bs, kr = 1, 16, 2, 300, 256, 128, 8
    N = nblk * bs
    q, do, og = (randn(g, (B, Hq, N, D), "f32", device=DEV) for _ in range(3))
    k, v = (randn(g, (B, Hkv, N, D), "f32", device=DEV) for _ in range(2))
    i = torch.arange(nblk).view(1, 1, nblk, 1)
    past = (torch.rand(B, Hkv, nblk, kr, generator=g) * (i + 1)).long()
    idx = torch.cat([past, i.expand(B, Hkv, nblk, 1), torch.zeros(B, Hkv, nblk, 1, dtype=torch.long)], -1)
    idx = idx.sort(-1).values.to(torch.int32).to(DEV)
    a, b = _case(q, k, v, idx, do, "token_causal", scale=D ** -0.5, out_gate=og)
    _same("d256 fp32 sink", a, b)


@pytest.mark.parametrize("bs", [32, 64])
def test_d64_bf16_gate_and_output_gate(bs):
    from oracle import select as osel
    from _util import np64
    g = torch.Generator().manual_seed(12)
    B, H, N, D, topk = 4, 8, 2048, 64, 8
    q, k, v, do, og = (randn(g, (B, H, N, D), "bf16") for _ in range(5))
    sel, _ = osel.select_mean_pooled(np64(q), np64(k), bs, topk, True, "bf16")
    gate = torch.nn.functional.logsigmoid(torch.randn(B, 1, N // bs, topk + 1, generator=g))
    t = lambda x: torch.as_tensor(x).to(DEV)  # noqa: E731
    a, b = _case(t(q), t(k), t(v), t(np.asarray(sel)[:, None]).to(torch.int32), t(do), "slot_causal",
                 gate=t(gate), out_gate=t(og), need_dgate=True)
    _same(f"d64 bf16 bs{bs}", a, b)
