"""Selection and forward of one step, overlapped on two streams.

The step of the synthetic configurations (and of ``BlockSparseSSA`` without
the gate) is: pool q and k per block, pick each query block's own block plus
its top-k content blocks (convention A, ``src/ssa_model.py:151-165``), then
the fused block-sparse forward. The forward of query block i reads only row i
of the selection, and with a causal selection row i reads only the pooled
rows <= i. So the rows are cut into ``splits`` ranges: the selection of range
r runs on the caller's stream while the forward of range r - 1 runs on a
second stream. The selection kernels are latency bound and move little data
while the forward is bound by its K/V gather, so the two overlap well; the
results are identical to the sequential step (same kernels, same rows).
"""
import torch

from . import ops, selection

_side = {}


def _side_stream(device):
    s = _side.get(device)
    if s is None:
        s = _side[device] = torch.cuda.Stream(device=device)  # default priority
    return s


def _row_splits(nblk, splits):
    """Row boundaries on 64-row multiples (the MFMA selection's row blocks).
    Causal selection work grows with the row, so the cuts are taken at equal
    shares of the forward (rows), not of the selection."""
    cuts = [0]
    for r in range(1, splits):
        c = (nblk * r // splits) // 64 * 64
        if c > cuts[-1]:
            cuts.append(c)
    if cuts[-1] != nblk:
        cuts.append(nblk)
    return list(zip(cuts[:-1], cuts[1:]))


def select_and_attend(q, k, v, bs, topk, *, causal=True, scale=None, need_lse=False, splits=4, engine="auto"):
    """Mean-pooled top-k selection (convention A) + fused forward, pipelined.

    q, k, v (B, H, L, D), L a multiple of bs. Returns (sel (B, nblk, kk) int32,
    o (B, H, L, D)) or (sel, o, lse) with need_lse. Same values as
    ``selection.select_mean_pooled`` followed by ``ops.attention_forward``.
    """
    B, H, L, D = q.shape
    nblk = L // bs
    qp = selection.pool(q, bs, "mean_tok_then_grp", grp=H)
    kp = selection.pool(k, bs, "mean_tok_then_grp", grp=k.shape[1])
    kk = selection.budget("own_first", topk, nblk)
    sel = torch.empty(B, 1, nblk, kk, dtype=torch.int32, device=q.device)
    mask = ops.MASK_SLOT_CAUSAL if causal else ops.MASK_NONE
    prep = ops.prepare_forward(q, k, v, sel, mask=mask, scale=scale, need_lse=need_lse)
    nbytes = selection.select_workspace_bytes(qp, topk=topk) if engine == "auto" else 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
    cur = torch.cuda.current_stream(q.device)
    side = _side_stream(q.device)
    side.wait_stream(cur)  # q, k, v, outputs and earlier work of the caller
    for r0, r1 in _row_splits(nblk, splits if causal else 1):
        selection.select(qp, kp, score="dot", convention="own_first", topk=topk, causal=causal, engine=engine,
                         rows=(r0, r1), out=sel, workspace=ws)
        ready = torch.cuda.Event()
        ready.record(cur)
        side.wait_event(ready)
        with torch.cuda.stream(side):
            ops.launch_forward(prep, (r0, r1))
    cur.wait_stream(side)
    out = ops.finish_forward(prep, need_lse)
    if need_lse:
        return sel[:, 0], out[0], out[1]
    return sel[:, 0], out


class GraphStep:
    """The sequential select + forward step recorded once as a HIP graph and
    replayed, for loops that repeat the step on fixed buffers (serving,
    benchmarks): pool q and k, the top-k selection and the fused forward go
    out as one graph launch instead of one host launch each.

    The step runs eagerly ``warmup`` times on a side stream (first-use setup
    such as kernel attributes happens there), then is captured with its
    workspaces in a graph-private memory pool. ``replay()`` re-runs it on the
    same q, k, v tensors (update them in place between replays) and returns
    the same output tensors (sel (B, nblk, kk) int32, o[, lse]), overwritten.
    None of the step's launches is a memset, so every replay is
    self-contained. Same values as ``selection.select_mean_pooled`` followed
    by ``ops.attention_forward``.
    """

    def __init__(self, q, k, v, bs, topk, *, causal=True, scale=None, need_lse=False, engine="auto", warmup=2):
        mask = ops.MASK_SLOT_CAUSAL if causal else ops.MASK_NONE

        def run():
            sel = selection.select_mean_pooled(q, k, bs, topk, causal=causal, engine=engine)
            out = ops.attention_forward(q, k, v, sel[:, None], mask=mask, scale=scale, need_lse=need_lse)
            return (sel,) + (tuple(out) if need_lse else (out,))

        side = torch.cuda.Stream(device=q.device)  # default priority
        side.wait_stream(torch.cuda.current_stream(q.device))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                run()
        torch.cuda.current_stream(q.device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.outputs = run()

    def replay(self):
        self.graph.replay()
        return self.outputs
