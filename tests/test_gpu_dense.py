"""GPU parity of the dense fast path (FBSA_FLAG_DENSE, ``ops.DenseSelection``):
every key block, causal or full, with no block list -- the reference's
``selector=None, topk >= nblk`` path of ``blocksparse_forward``
(``src/qwen_blocksparse.py:37-41``), which calls SDPA there.

* Small shapes: bit-identical to the same attention through an explicit
  all-blocks list (``arange`` per row), and within tolerance of the float64
  oracle's dense attention.
* A sequence past the former list limit (8448 blocks of 16 tokens): forward
  and backward through ``qwen_blocksparse.blocksparse_forward`` against a
  chunked fp32 causal attention in torch (autograd), and its first rows against
  the oracle (causal rows depend only on the prefix)."""
import numpy as np
import pytest
import torch

from oracle import attn as oattn
from _util import randn, np64, assert_close, TOL, OUT_ROUND

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print("[dense]", *a, flush=True)


@pytest.mark.parametrize("dtype,mask", [("bf16", "token_causal"), ("bf16", "none"), ("f32", "token_causal"),
                                        ("f32", "none")])
def test_dense_equals_explicit_all_blocks(dtype, mask):
    from fbsa_amd import ops
    g = torch.Generator().manual_seed(21)
    B, Hq, Hkv, N, D, bs = 2, 4, 2, 1024, 64, 32
    nblk = N // bs
    lv = N - 45
    q, do, og = (randn(g, (B, Hq, N, D), dtype).to(DEV) for _ in range(3))
    k, v = (randn(g, (B, Hkv, N, D), dtype).to(DEV) for _ in range(2))
    m = ops.MASK_TOKEN_CAUSAL if mask == "token_causal" else ops.MASK_NONE
    dense = ops.DenseSelection(B, nblk)
    idx = torch.arange(nblk, dtype=torch.int32, device=DEV).view(1, 1, 1, nblk).expand(B, Hkv, nblk, nblk).contiguous()
    _say(dtype, mask, "dense vs explicit list")
    o1, l1 = ops.attention_forward(q, k, v, dense, mask=m, l_valid=lv, out_gate=og, need_lse=True)
    o2, l2 = ops.attention_forward(q, k, v, idx, mask=m, l_valid=lv, out_gate=og, need_lse=True)
    g1 = ops.attention_backward(q, k, v, dense, o1, l1, do, mask=m, l_valid=lv, out_gate=og)
    g2 = ops.attention_backward(q, k, v, idx, o2, l2, do, mask=m, l_valid=lv, out_gate=og)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    for name, a, b in zip(("dq", "dk", "dv", "dgate", "dout_gate"), g1, g2):
        if a is None:
            continue
        if dtype == "f32" and mask == "none" and name in ("dk", "dv"):
            # fp32 lists this long are walked in segments (fp32 partials summed
            # in order) through the explicit list, in one pass through the dense one
            assert_close(np64(a), np64(b), "f32", name)
        else:
            assert torch.equal(a, b), name
    # the oracle's dense attention (src/qwen_blocksparse.py:37-41 is SDPA)
    ro, _ = oattn.fwd(np64(q), np64(k), np64(v), idx.cpu().numpy(), mask, L_valid=lv, out_gate=np64(og))
    rows = torch.arange(N) < lv
    assert_close(np64(o1)[:, :, rows.numpy()], ro[:, :, rows.numpy()], dtype, "o vs oracle")


def _chunked_causal_reference(q, k, v, do, scale, chunk=2048):
    """fp32 causal attention over every key (GQA by head repeat), chunk by chunk
    of query rows, with autograd for dq, dk, dv."""
    B, Hq, N, D = q.shape
    grp = Hq // k.shape[1]
    kf = k.float().repeat_interleave(grp, 1).detach().requires_grad_(True)
    vf = v.float().repeat_interleave(grp, 1).detach().requires_grad_(True)
    o = torch.empty(B, Hq, N, D, device=q.device)
    dq = torch.empty(B, Hq, N, D, device=q.device)
    for r0 in range(0, N, chunk):
        r1 = min(N, r0 + chunk)
        qc = q[:, :, r0:r1].float().detach().requires_grad_(True)
        s = torch.matmul(qc, kf[:, :, :r1].transpose(-1, -2).contiguous()) * scale
        t = torch.arange(r0, r1, device=q.device).view(-1, 1)
        u = torch.arange(r1, device=q.device).view(1, -1)
        s = s.masked_fill(u > t, float("-inf"))
        oc = torch.matmul(torch.softmax(s, -1), vf[:, :, :r1])
        o[:, :, r0:r1] = oc.detach()
        (oc * do[:, :, r0:r1].float()).sum().backward()
        dq[:, :, r0:r1] = qc.grad
    dk = kf.grad.view(B, k.shape[1], grp, N, D).sum(2)
    dv = vf.grad.view(B, k.shape[1], grp, N, D).sum(2)
    return o, dq, dk, dv


def test_dense_long_sequence_forward_backward():
    import qwen_blocksparse as qb
    B, Hq, Hkv, D, bs = 1, 2, 1, 64, 16
    nblk = 8448                                  # past the 8192 blocks an explicit list allowed
    N = nblk * bs
    g = torch.Generator(device=DEV).manual_seed(22)
    rn = lambda *s: torch.randn(*s, generator=g, device=DEV).to(torch.bfloat16)  # noqa: E731
    q, k, v = (rn(B, Hq, N, D) * 0.5, rn(B, Hkv, N, D) * 0.5, rn(B, Hkv, N, D))
    do = rn(B, Hq, N, D)
    qd, kd, vd = (x.detach().requires_grad_(True) for x in (q, k, v))
    _say(f"blocksparse_forward dense, N={N} nblk={nblk}")
    o = qb.blocksparse_forward(qd, kd, vd, selector=None, topk=nblk, bs=bs, causal=True)
    o.backward(do)
    ro, rdq, rdk, rdv = _chunked_causal_reference(q, k, v, do, D ** -0.5)
    torch.cuda.synchronize()
    for name, got, ref in (("o", o, ro), ("dq", qd.grad, rdq), ("dk", kd.grad, rdk), ("dv", vd.grad, rdv)):
        t = TOL["bf16"]
        got, ref = got.detach().double(), ref.double()
        excess = float(((got - ref).abs() - OUT_ROUND["bf16"] * ref.abs()).max())
        rl = float((got - ref).norm() / ref.norm())
        _say(f"{name}: max_abs={excess:.3e} rel_l2={rl:.3e}")
        assert excess <= t["max_abs"] and rl <= t["rel_l2"], name
    # causal rows depend only on the prefix: the first 256 tokens against the oracle
    P = 256
    rp = oattn.dense(np64(q[:, :, :P]), np64(k[:, :, :P]), np64(v[:, :, :P]), True)
    ro_np = rp[0] if isinstance(rp, tuple) else rp
    assert_close(np64(o[:, :, :P]), ro_np, "bf16", "o prefix vs oracle")


def test_dense_fp32_long_lists_walked_in_segments():
    # fp32, MASK_NONE, 2048 blocks of 16: every key block's implicit list holds
    # all 2048 query blocks (x 2 query heads), so its fp32 dK/dV sums 65,536
    # query rows; the dense lists are walked in segments like explicit ones
    # (closed-form offsets), and the result meets the absolute fp32 bar against
    # fp32 attention in torch (autograd)
    from fbsa_amd import ops
    B, Hq, Hkv, D, bs, nblk = 1, 2, 1, 32, 16, 2048
    N = nblk * bs
    g = torch.Generator(device=DEV).manual_seed(23)
    rn = lambda *s: torch.randn(*s, generator=g, device=DEV)  # noqa: E731
    q, k, v, do = rn(B, Hq, N, D), rn(B, Hkv, N, D), rn(B, Hkv, N, D), rn(B, Hq, N, D)
    dense = ops.DenseSelection(B, nblk)
    o, lse = ops.attention_forward(q, k, v, dense, mask=ops.MASK_NONE, need_lse=True)
    dq, dk, dv = ops.attention_backward(q, k, v, dense, o, lse, do, mask=ops.MASK_NONE)[:3]
    # torch fp32 reference: full (non-causal) attention, query chunks, GQA by repeat
    kf = k.repeat_interleave(2, 1).detach().requires_grad_(True)
    vf = v.repeat_interleave(2, 1).detach().requires_grad_(True)
    ro = torch.empty_like(q)
    rdq = torch.empty_like(q)
    for r0 in range(0, N, 4096):
        qc = q[:, :, r0:r0 + 4096].detach().requires_grad_(True)
        oc = torch.matmul(torch.softmax(torch.matmul(qc, kf.transpose(-1, -2).contiguous()) * D ** -0.5, -1), vf)
        ro[:, :, r0:r0 + 4096] = oc.detach()
        (oc * do[:, :, r0:r0 + 4096]).sum().backward()
        rdq[:, :, r0:r0 + 4096] = qc.grad
    rdk = kf.grad.view(B, Hkv, 2, N, D).sum(2)
    rdv = vf.grad.view(B, Hkv, 2, N, D).sum(2)
    torch.cuda.synchronize()
    for name, got, ref in (("o", o, ro), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        err = float((got.double() - ref.double()).abs().max())
        rl = float((got.double() - ref.double()).norm() / ref.double().norm())
        _say(f"fp32 dense segments {name}: max_abs={err:.3e} rel_l2={rl:.3e} max|ref|={float(ref.abs().max()):.3g}")
        assert err <= TOL["f32"]["max_abs"] and rl <= TOL["f32"]["rel_l2"], name
