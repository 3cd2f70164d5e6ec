"""GPU: selection budgets of thousands of blocks at bs 128 / d 256, forward and backward.

The reference takes any budget: its kernel loops over KK slots
(``src/triton_kernel.py:50,110,133,154``) and ``SelectMax`` keeps the top
``topk`` of every row (``src/qwen_blocksparse.py:87-121``). Here
``SelectMax(topk=3000)`` over 3072 key blocks of 128 tokens (GQA 2:1, d 256,
token-causal, own + sink): the forward's and dQ's per-workgroup slot tables
hold 3002 slots, and the backward's transposed lists are walked in segments.
Checked against the float64 oracle on sampled query blocks (O, dQ) and on
the last key block, which only the last query block reads (dK, dV)."""
import numpy as np
import pytest
import torch

from oracle import attn as oattn
from _util import np64, assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_select_max_topk3000_bs128_d256():
    import qwen_blocksparse as qb
    from fbsa_amd import ops
    B, Hq, Hkv, D, bs, nblk, topk = 1, 2, 1, 256, 128, 3072, 3000
    N = nblk * bs
    g = torch.Generator(device=DEV).manual_seed(30)
    rn = lambda *s: torch.randn(*s, generator=g, device=DEV).to(torch.bfloat16)  # noqa: E731
    q, k, v, do = rn(B, Hq, N, D), rn(B, Hkv, N, D), rn(B, Hkv, N, D), rn(B, Hq, N, D)
    idx = qb.SelectMax(topk=topk, bs=bs, sink=True).select(q, k)
    assert idx.shape == (B, Hkv, nblk, topk + 2)
    sc = D ** -0.5
    idx32 = idx.to(torch.int32).contiguous()
    print(f"[long-lists] kk={idx.shape[-1]} forward", flush=True)
    o, lse = ops.attention_forward(q, k, v, idx32, mask=ops.MASK_TOKEN_CAUSAL, scale=sc, need_lse=True)
    print("[long-lists] backward", flush=True)
    dq, dk, dv = ops.attention_backward(q, k, v, idx32, o, lse, do, mask=ops.MASK_TOKEN_CAUSAL, scale=sc)[:3]
    torch.cuda.synchronize()
    rows = [1500, nblk - 1]
    blk = lambda x, bl: np.concatenate([x[:, :, b * bs:(b + 1) * bs] for b in bl], 2)  # noqa: E731
    sel = idx.cpu().numpy()
    print("[long-lists] oracle forward", flush=True)
    ro, _ = oattn.fwd(np64(q), np64(k), np64(v), sel, "token_causal", scale=sc, rows=rows)
    ex, rl = assert_close(blk(np64(o), rows), ro, "bf16", "o")
    print(f"[long-lists] o (oracle, blocks {rows}): max_abs={ex:.3e} rel_l2={rl:.3e}", flush=True)
    print("[long-lists] oracle backward", flush=True)
    r = oattn.bwd(np64(q), np64(k), np64(v), sel, np64(do), "token_causal", scale=sc, rows=[nblk - 1])
    for name, got, ref, bl in (("dq", dq, r[0], [nblk - 1]), ("dk", dk, r[1], [nblk - 1]),
                               ("dv", dv, r[2], [nblk - 1])):
        ex, rl = assert_close(blk(np64(got), bl), blk(ref, bl), "bf16", name)
        print(f"[long-lists] {name} (oracle, block {bl[0]}): max_abs={ex:.3e} rel_l2={rl:.3e}", flush=True)
