"""GPU: the backward captured in a HIP graph (torch.cuda.graph) and replayed.

Outside capture fbsa_bwd runs its index stage on a second stream beside dQ;
under capture it runs the stages in order on the caller's stream. Every
replay, with eager work in between, must give the eager result bit for bit."""
import pytest
import torch

from _util import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_backward_graph_replays_match_eager(dt):
    from fbsa_amd import ops
    g = torch.Generator().manual_seed(43)
    B, Hq, Hkv, nblk, bs, D, kk = 1, 4, 2, 48, 64, 64, 9
    L = nblk * bs
    q, do = (randn(g, (B, Hq, L, D), dt, device=DEV) for _ in range(2))
    k, v = (randn(g, (B, Hkv, L, D), dt, device=DEV) for _ in range(2))
    i = torch.arange(nblk).view(1, 1, nblk, 1)
    past = (torch.rand(B, Hkv, nblk, kk - 1, generator=g) * (i + 1)).long()
    sel = torch.cat([i.expand(B, Hkv, nblk, 1), past], -1).to(torch.int32).to(DEV)
    mask, sc = ops.MASK_TOKEN_CAUSAL, D ** -0.5
    o, lse = ops.attention_forward(q, k, v, sel, mask=mask, scale=sc, need_lse=True)
    run = lambda: ops.attention_backward(q, k, v, sel, o, lse, do, mask=mask, scale=sc)[:3]  # noqa: E731
    eager = [t.clone() for t in run()]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print(f"[bwd-graph] {dt}: capture", flush=True)
    with torch.cuda.graph(graph):
        out = run()
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for n, a, b in zip(("dq", "dk", "dv"), out, eager):
            assert torch.equal(a, b), f"{dt} replay {r}: {n} differs from the eager backward"
        print(f"[bwd-graph] {dt}: replay {r} matches", flush=True)
        again = run()  # eager work between the replays
        torch.cuda.synchronize()
        for a, b in zip(again, eager):
            assert torch.equal(a, b)
