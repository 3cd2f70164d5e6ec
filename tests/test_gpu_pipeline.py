"""GPU: row-range selection / forward and the two-stream select+forward step.

Row ranges must reproduce the full call's rows bit for bit (same kernels, same
rows), and the pipelined step must equal the sequential step exactly; the
sequential step itself is pinned against the oracle in test_gpu_select.py and
test_gpu_fwd.py."""
import numpy as np
import pytest
import torch

from _util import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print("[pipeline]", *a, flush=True)


@pytest.mark.parametrize("engine", ["auto", "fp64"])
@pytest.mark.parametrize("causal", [True, False])
def test_select_rows_match_full(engine, causal):
    from fbsa_amd import selection
    g = torch.Generator().manual_seed(11)
    B, H, nblk, D, topk = 2, 2, 700, 64, 16
    a, b = (randn(g, (B, H, nblk, D), "bf16").to(DEV) for _ in range(2))
    _say("select rows", engine, causal)
    full, fsc = selection.select(a, b, topk=topk, causal=causal, need_scores=True, engine=engine)
    part = torch.full_like(full, -7)
    for r0, r1 in ((0, 64), (64, 200), (200, 256), (256, 700)):
        selection.select(a, b, topk=topk, causal=causal, engine=engine, rows=(r0, r1), out=part)
    assert torch.equal(part, full)
    # a range leaves the other rows alone
    only = torch.full_like(full, -7)
    selection.select(a, b, topk=topk, causal=causal, engine=engine, rows=(128, 320), out=only)
    assert torch.equal(only[:, :, 128:320], full[:, :, 128:320])
    assert (only[:, :, :128] == -7).all() and (only[:, :, 320:] == -7).all()


def test_fwd_rows_match_full():
    from fbsa_amd import ops
    g = torch.Generator().manual_seed(12)
    B, H, N, D, bs, kk = 1, 4, 64 * 96, 64, 64, 9
    q, k, v = (randn(g, (B, H, N, D), "bf16").to(DEV) for _ in range(3))
    nblk = N // bs
    sel = torch.randint(0, nblk, (B, 1, nblk, kk), generator=g).to(torch.int32)
    sel[..., 0] = torch.arange(nblk, dtype=torch.int32)
    sel = sel.to(DEV)
    _say("fwd rows")
    o, lse = ops.attention_forward(q, k, v, sel, mask=ops.MASK_SLOT_CAUSAL, need_lse=True)
    prep = ops.prepare_forward(q, k, v, sel, mask=ops.MASK_SLOT_CAUSAL, need_lse=True)
    for r in ((0, 10), (10, 64), (64, 96)):
        ops.launch_forward(prep, r)
    o2, lse2 = ops.finish_forward(prep, True)
    assert torch.equal(o2, o) and torch.equal(lse2, lse)


@pytest.mark.parametrize("N,splits", [(64 * 1000, 4), (64 * 300, 3), (64 * 64, 2)])
def test_pipelined_step_equals_sequential(N, splits):
    from fbsa_amd import ops, pipeline, selection
    g = torch.Generator().manual_seed(13)
    B, H, D, bs, topk = 1, 4, 64, 64, 16
    q, k, v = ((randn(g, (B, H, N, D), "bf16") * 0.125).to(torch.bfloat16).to(DEV) for _ in range(3))
    _say("pipelined step", N, splits)
    sel = selection.select_mean_pooled(q, k, bs, topk, True)
    o, lse = ops.attention_forward(q, k, v, sel[:, None], mask=ops.MASK_SLOT_CAUSAL, need_lse=True)
    psel, po, plse = pipeline.select_and_attend(q, k, v, bs, topk, need_lse=True, splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(psel, sel)
    assert torch.equal(po, o) and torch.equal(plse, lse)
    # repeated calls (stream reuse) stay identical
    psel2, po2 = pipeline.select_and_attend(q, k, v, bs, topk, splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(psel2, sel) and torch.equal(po2, o)



@pytest.mark.parametrize("engine,need_lse", [("auto", True), ("fp64", False)])
def test_graph_step_replays_match_eager(engine, need_lse):
    # the captured step, replayed several times with eager work and
    # synchronisations in between, equals the eager step every time, also
    # after the inputs change in place
    from fbsa_amd import ops, pipeline, selection
    g = torch.Generator().manual_seed(12)
    B, H, L, D, bs, topk = 1, 4, 16384, 64, 64, 16
    q, k, v = (randn(g, (B, H, L, D), "bf16", scale=0.125).to(DEV) for _ in range(3))

    def eager():
        sel = selection.select_mean_pooled(q, k, bs, topk, causal=True, engine=engine)
        out = ops.attention_forward(q, k, v, sel[:, None], mask=ops.MASK_SLOT_CAUSAL, need_lse=need_lse)
        return (sel,) + (tuple(out) if need_lse else (out,))

    _say("graph step", engine, need_lse)
    step = pipeline.GraphStep(q, k, v, bs, topk, need_lse=need_lse, engine=engine)
    for rep in range(4):
        if rep == 2:  # new inputs, same buffers
            q.copy_(randn(g, (B, H, L, D), "bf16", scale=0.125).to(DEV))
            v.mul_(-1)
        got = [t.clone() for t in step.replay()]
        torch.cuda.synchronize()
        ref = eager()
        x = torch.randn(1000, device=DEV).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(x)
        for a, b in zip(got, ref):
            assert torch.equal(a, b), f"replay {rep}"
