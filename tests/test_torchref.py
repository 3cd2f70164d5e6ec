"""Pins the fp32 torch gather-attention restatement (``tests/_torchref.py``)
against the float64 oracle on the CPU, under all three mask rules, GQA with a
per-KV-head selection, duplicates, a slot gate, the output gate and a padded
length, forward and backward."""
import numpy as np
import pytest
import torch

from oracle import attn as oattn
import _torchref


def _np(t):
    return None if t is None else t.detach().double().numpy()


@pytest.mark.parametrize("mask", ["none", "slot_causal", "token_causal"])
@pytest.mark.parametrize("gqa", [False, True])
def test_torchref_matches_oracle(mask, gqa):
    g = torch.Generator().manual_seed(11)
    B, Hq, N, D, bs, kk = 2, 4, 256, 32, 32, 5
    Hkv, Hs = (2, 2) if gqa else (Hq, 1)
    nblk = N // bs
    q, do, og = (torch.randn(B, Hq, N, D, generator=g) for _ in range(3))
    k, v = (torch.randn(B, Hkv, N, D, generator=g) for _ in range(2))
    own = torch.arange(nblk).view(1, 1, nblk, 1).expand(B, Hs, nblk, 1)
    sel = torch.cat([own, torch.randint(0, nblk, (B, Hs, nblk, kk - 1), generator=g)], -1)
    sel[..., 2] = sel[..., 1]                                   # a duplicate in every row
    if mask == "token_causal":
        sel = sel.sort(-1).values
    gate = torch.nn.functional.logsigmoid(torch.randn(B, Hs, nblk, kk, generator=g))
    lv = N - 19 if mask != "slot_causal" else None
    ref = oattn.bwd(_np(q), _np(k), _np(v), sel.numpy(), _np(do), mask, scale=0.3, gate=gate.numpy(),
                    L_valid=lv, out_gate=_np(og))
    ro, rl = oattn.fwd(_np(q), _np(k), _np(v), sel.numpy(), mask, scale=0.3, gate=gate.numpy(), L_valid=lv,
                       out_gate=_np(og))
    o, lse, dq, dk, dv, dog = _torchref.attention(q, k, v, sel, mask, scale=0.3, gate=gate, out_gate=og,
                                                  l_valid=lv, do=do, chunk=3)
    fin = np.isfinite(rl)
    assert np.array_equal(np.isfinite(_np(lse)), fin)
    np.testing.assert_allclose(_np(lse)[fin], rl[fin], atol=2e-5, rtol=0)
    for name, got, want in (("o", o, ro), ("dq", dq, ref[0]), ("dk", dk, ref[1]), ("dv", dv, ref[2]),
                            ("dout_gate", dog, ref[4])):
        np.testing.assert_allclose(_np(got), want, atol=2e-5, rtol=0, err_msg=name)
