"""GPU regression: tile base addresses whose low 32-bit word has bit 31 set.

The direct-to-LDS copies take a wave-uniform 64-bit tile base in SGPRs; its
low word, read back from a VGPR as a signed 32-bit value, must be
zero-extended when the two halves are joined, or every base with bit 31 of
the low word set points elsewhere (the one GPU memory fault seen in this
work). Here q, k, v and dO are placed in one device buffer at addresses whose
low word has bit 31 set (a 4 GiB window's upper half) and, separately, at
addresses whose low word has it clear; the forward and backward must give
bit-identical results for the same data."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
GIB = 1 << 30


@pytest.fixture(scope="module")
def windows():
    # 8 GiB: holds a whole 4 GiB-aligned window whatever the base address
    buf = torch.empty(8 * GIB, dtype=torch.uint8, device=DEV)
    base = buf.data_ptr()
    lo = ((base >> 32) + 1) << 32                 # low word 0x00000000: bit 31 clear
    hi = lo + (1 << 31)                            # low word 0x80000000: bit 31 set
    assert lo >= base and hi + GIB <= base + 8 * GIB
    return buf, lo - base, hi - base


def _place(buf, off, tensors):
    """Copies of `tensors` laid out back to back from byte offset `off`."""
    out = []
    for t in tensors:
        n = t.numel() * t.element_size()
        v = buf[off:off + n].view(t.dtype).view(t.shape)
        v.copy_(t)
        out.append(v)
        off += (n + 4095) // 4096 * 4096
    return out


def _run(q, k, v, do, sel, mask, scale):
    from fbsa_amd import ops
    o, lse = ops.attention_forward(q, k, v, sel, mask=mask, scale=scale, need_lse=True)
    dq, dk, dv = ops.attention_backward(q, k, v, sel, o, lse, do, mask=mask, scale=scale)[:3]
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("case", ["bs64_d64_slot_causal", "bs128_d256_gqa_token_causal", "bs64_d128_slot_causal"])
def test_bit31_tile_bases(windows, case):
    from fbsa_amd import ops
    buf, off_lo, off_hi = windows
    g = torch.Generator(device=DEV).manual_seed(31)
    rn = lambda *s: torch.randn(*s, generator=g, device=DEV).to(torch.bfloat16)  # noqa: E731
    if case.startswith("bs128"):
        B, Hq, Hkv, N, D, bs, kk, mask = 1, 8, 1, 8192, 256, 128, 6, ops.MASK_TOKEN_CAUSAL
    else:
        B, Hq, Hkv, N, D, bs, kk, mask = 1, 4, 4, 16384, (64 if "d64" in case else 128), 64, 9, ops.MASK_SLOT_CAUSAL
    nblk = N // bs
    q, k, v, do = rn(B, Hq, N, D), rn(B, Hkv, N, D), rn(B, Hkv, N, D), rn(B, Hq, N, D)
    i = torch.arange(nblk, device=DEV).view(1, 1, nblk, 1)
    past = (torch.rand(B, 1 if mask == ops.MASK_SLOT_CAUSAL else Hkv, nblk, kk - 1, generator=g, device=DEV)
            * i).long()
    sel = torch.cat([i.expand(past.shape[0], past.shape[1], nblk, 1), past], -1).to(torch.int32)
    sc = D ** -0.5
    ref = _run(*_place(buf, off_lo, (q, k, v, do)), sel, mask, sc)
    got = _run(*_place(buf, off_hi, (q, k, v, do)), sel, mask, sc)
    print(f"[high-address] {case}: q at {hex(_place(buf, off_hi, (q,))[0].data_ptr())}", flush=True)
    for n, a, b in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        assert torch.equal(a, b), f"{case}: {n} differs between bit-31-set and bit-31-clear addresses"
