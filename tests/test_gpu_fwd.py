"""GPU parity: fused forward (libfbsa.so) vs the float64 CPU oracle."""
import numpy as np
import pytest
import torch

from oracle import attn as oattn, select as osel
from _util import randn, np64, assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(q, k, v, sel, mask, dtype, gate=None, l_valid=None, out_gate=None, scale=None):
    from fbsa_amd import ops
    print(f"[fwd] q{tuple(q.shape)} k{tuple(k.shape)} sel{tuple(sel.shape)} {dtype} mask={mask}", flush=True)
    mcode = {"none": 0, "slot_causal": 1, "token_causal": 2}[mask]
    o, lse = ops.attention_forward(q.to(DEV), k.to(DEV), v.to(DEV), torch.as_tensor(sel).to(DEV),
                                   mask=mcode, scale=scale,
                                   gate=None if gate is None else torch.as_tensor(gate).to(DEV),
                                   l_valid=l_valid,
                                   out_gate=None if out_gate is None else out_gate.to(DEV), need_lse=True)
    torch.cuda.synchronize()
    ro, rl = oattn.fwd(np64(q), np64(k), np64(v), np.asarray(sel), mask, scale=scale,
                       gate=None if gate is None else np.asarray(gate, np.float64), L_valid=l_valid,
                       out_gate=None if out_gate is None else np64(out_gate))
    return np64(o), ro, lse.cpu().numpy().astype(np.float64), rl


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_config1_shape_mean_pooled_selection(dtype):
    # config 1: B1 H4 N4096 D64 bs64 causal top-8 by mean-pooled q.k (convention A)
    g = torch.Generator().manual_seed(0)
    B, H, N, D, bs = 1, 4, 4096, 64, 64
    q, k, v = (randn(g, (B, H, N, D), dtype) for _ in range(3))
    sel, _ = osel.select_mean_pooled(np64(q), np64(k), bs, 8, True, dtype)
    o, ro, lse, rl = _run(q, k, v, sel[:, None], "slot_causal", dtype)
    assert_close(o, ro, dtype, "o")
    fin = np.isfinite(rl)
    assert np.array_equal(fin, np.isfinite(lse))
    # the row normalisers are fp32 sums of the unrounded exponentials in every dtype
    lerr = float(np.max(np.abs(lse[fin] - rl[fin])))
    print(f"  lse ({dtype}): max_abs={lerr:.2e}", flush=True)
    assert lerr < 1e-4


def test_config2_shape_gate_bias():
    # config 2 forward: B32 H8 N1024 D64 bs32 causal top-4, gate = logsigmoid(N(0,1))
    g = torch.Generator().manual_seed(0)
    B, H, N, D, bs, topk = 32, 8, 1024, 64, 32, 4
    q, k, v = (randn(g, (B, H, N, D), "bf16") for _ in range(3))
    sel, _ = osel.select_mean_pooled(np64(q), np64(k), bs, topk, True, "bf16")
    gate = torch.nn.functional.logsigmoid(torch.randn(B, N // bs, topk + 1, generator=g)).numpy()
    o, ro, _, _ = _run(q, k, v, sel[:, None], "slot_causal", "bf16", gate=gate[:, None])
    assert_close(o, ro, "bf16", "o")


@pytest.mark.parametrize("bs,D", [(16, 64), (32, 32), (64, 128), (128, 64), (128, 256), (64, 256), (16, 32)])
def test_block_and_head_sizes_random_sel_noncausal(bs, D):
    # make_sel-style selection (own + random with replacement, future blocks allowed), no mask
    g = torch.Generator().manual_seed(1)
    B, H, nblk, kk = 1, 2, 12, 5
    N = nblk * bs
    q, k, v = (randn(g, (B, H, N, D), "bf16") for _ in range(3))
    rnd = torch.randint(0, nblk, (B, nblk, kk - 1), generator=g)
    sel = torch.cat([torch.arange(nblk).view(1, nblk, 1), rnd], -1).numpy()
    gate = torch.nn.functional.logsigmoid(torch.randn(B, nblk, kk, generator=g)).numpy()
    o, ro, _, _ = _run(q, k, v, sel[:, None], "none", "bf16", gate=gate[:, None])
    assert_close(o, ro, "bf16", "o")
    o, ro, _, _ = _run(q, k, v, sel[:, None], "slot_causal", "bf16")
    assert_close(o, ro, "bf16", "o causal")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_gqa_token_causal_quest_padding_outgate(dtype):
    g = torch.Generator().manual_seed(2)
    B, Hq, Hkv, N, D, bs, topk = 1, 8, 2, 1024, 128, 128, 3
    q = randn(g, (B, Hq, N, D), dtype)
    k, v = (randn(g, (B, Hkv, N, D), dtype) for _ in range(2))
    og = randn(g, (B, Hq, N, D), dtype)
    idx, _ = osel.select_quest(np64(q), np64(k), bs, topk, True, dtype)
    o, ro, _, _ = _run(q, k, v, idx, "token_causal", dtype, l_valid=N - 77, out_gate=og, scale=0.0625)
    assert_close(o[..., :N - 77, :], ro[..., :N - 77, :], dtype, "o")


def test_strided_qwen_layout_out_gate():
    # q/k/v as transposed views of (B, L, H, D) and the out gate as a (B, L, Hq*D) view
    g = torch.Generator().manual_seed(3)
    B, Hq, Hkv, N, D, bs = 1, 4, 2, 512, 64, 64
    qs = randn(g, (B, N, Hq, D), "bf16")
    ks = randn(g, (B, N, Hkv, D), "bf16")
    vs = randn(g, (B, N, Hkv, D), "bf16")
    gs = randn(g, (B, N, Hq * D), "bf16")
    q, k, v = qs.transpose(1, 2), ks.transpose(1, 2), vs.transpose(1, 2)
    og = gs.view(B, N, Hq, D).transpose(1, 2)
    nblk = N // bs
    sel = np.broadcast_to(np.arange(nblk), (B, Hkv, nblk, nblk)).copy()     # SelectAll
    o, ro, _, _ = _run(q, k, v, sel, "token_causal", "bf16", out_gate=og)
    assert_close(o, ro, "bf16", "o")
    dense = oattn.dense(np64(q), np64(k), np64(v), True) / (1 + np.exp(-np64(og)))
    assert_close(o, dense, "bf16", "o vs dense")


def test_selection_out_of_range_is_skipped():
    # out-of-range block ids are dropped by the kernel's plan (never gathered)
    g = torch.Generator().manual_seed(4)
    B, H, N, D, bs = 1, 1, 256, 64, 64
    q, k, v = (randn(g, (B, H, N, D), "bf16") for _ in range(3))
    from fbsa_amd import ops
    sel = np.array([[[0, 9], [1, -3], [2, 1], [3, 99]]])
    o = ops.attention_forward(q.to(DEV), k.to(DEV), v.to(DEV), torch.as_tensor(sel[:, None]).to(DEV), mask=1)
    ok_sel = np.array([[[0, 0], [1, 1], [2, 1], [3, 3]]])   # invalid content slots masked
    ro, _ = oattn.fwd(np64(q), np64(k), np64(v), ok_sel[:, None], "slot_causal")
    assert_close(np64(o), ro, "bf16", "o")
