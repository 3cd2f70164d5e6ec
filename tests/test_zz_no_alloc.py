"""fbsa_select_noalloc: the selection entry point that allocates nothing (its
MFMA workspace is the library's static device scratch). Called through the C
ABI and compared bit for bit with fbsa_select given a caller workspace, on two
calls in a row, the second with a smaller input; oversized selections are
rejected on the host before any launch."""
import ctypes

import pytest
import torch

from fbsa_amd import _lib

DEV = "cuda"


def _desc(B, H, nblk, D, topk, score):
    d = _lib.SelectDesc()
    d.dtype = _lib.BF16
    d.score = {"dot": _lib.SCORE_DOT, "max2": _lib.SCORE_MAX2}[score]
    d.convention = _lib.SEL_OWN_FIRST
    d.causal, d.sink, d.flags = 1, 0, 0
    d.B, d.H, d.nblk, d.D, d.topk = B, H, nblk, D, topk
    d.kk = 1 + min(topk, nblk - 1)
    return d


def test_noalloc_rejects_selections_beyond_the_scratch():
    # B*H*nblk*K partial-list entries far past 32 MiB: refused before any device work
    lib = _lib.load()
    d = _desc(64, 8, 65536, 64, 16, "dot")
    assert lib.fbsa_select_workspace_bytes(d) > _lib.SELECT_SCRATCH_BYTES
    dummy = ctypes.c_void_p(1 << 20)        # never dereferenced: the size check fails first
    st = lib.fbsa_select_noalloc(d, dummy, dummy, None, dummy, None, None)
    assert st == _lib.EWORKSPACE
    assert b"static scratch" in lib.fbsa_last_error()


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point():
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    # configuration 3's pooled shape, then a smaller ragged one (chunked rows, max-of-two scores)
    for B, H, nblk, D, topk, score in ((1, 1, 4096, 64, 16, "dot"), (2, 1, 700, 32, 8, "max2")):
        print(f"[noalloc] B{B} H{H} nblk{nblk} D{D} top-{topk} {score}", flush=True)
        g = torch.Generator(device=DEV).manual_seed(nblk)
        a, b1, b2 = (torch.randn(B, H, nblk, D, generator=g, device=DEV).to(torch.bfloat16) for _ in range(3))
        if score == "dot":
            b2 = None
        d = _desc(B, H, nblk, D, topk, score)
        need = lib.fbsa_select_workspace_bytes(d)
        assert 0 < need <= _lib.SELECT_SCRATCH_BYTES
        kk = d.kk
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        sel_ref = torch.empty(B, H, nblk, kk, dtype=torch.int32, device=DEV)
        sc_ref = torch.empty(B, H, nblk, kk, dtype=torch.float32, device=DEV)
        _lib.check(lib.fbsa_select(d, p(a), p(b1), p(b2), p(sel_ref), p(sc_ref), p(ws), need, stream), "fbsa_select")
        sel = torch.full((B, H, nblk, kk), -7, dtype=torch.int32, device=DEV)
        sc = torch.full((B, H, nblk, kk), float("nan"), dtype=torch.float32, device=DEV)
        _lib.check(lib.fbsa_select_noalloc(d, p(a), p(b1), p(b2), p(sel), p(sc), stream), "fbsa_select_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(sel, sel_ref)
        assert torch.equal(sc.view(torch.int32), sc_ref.view(torch.int32))
