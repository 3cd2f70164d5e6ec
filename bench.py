"""Benchmark: block-pair selection + fused block-sparse forward on one MI355X.

Workload (the north-star shape): bf16, B=1, H=8,
D=64, N=262144, block 64 (nblk=4096), causal, top-16 content blocks by
mean-pooled q.k scores (kk=17), q,k,v ~ N(0,1)/sqrt(D). One step = pool q,
pool k, streaming top-k selection, fused forward, all on device-resident
inputs, one after the other on one
stream. ``--overlap`` times ``fbsa_amd.pipeline.select_and_attend`` instead,
which overlaps the selection of later query blocks with the forward of
earlier ones on a second stream (identical results; slower on MI355X at this
shape, the two kernels contend for the CUs).

Prints ONE JSON line. ``value`` is tokens/s of the select+fwd step
(BASELINE's headline); ``bwd`` times the backward of the same attention
(row statistics, transposed index, dQ, dK/dV) with its own MFMA roofline (skip it with
--no-bwd); ``roofline`` is the fused forward kernel (MFMA-bound: 4*B*H*nblk*kk*bs^2*D
FLOP per launch, the reference's own formula, src/bench_crossover.py:105)
timed with HIP events on the launch stream in separate, unoverlapped
launches; ``cpu_baseline`` times the reference's PyTorch gather path on the
host cores (same dtype) on a bounded sample of query blocks and scales it to
the whole workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "fused-block-sparse-attention_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--N", type=int, default=262144)
    p.add_argument("--H", type=int, default=8)
    p.add_argument("--D", type=int, default=64)
    p.add_argument("--bs", type=int, default=64)
    p.add_argument("--topk", type=int, default=16)
    p.add_argument("--bwd", action="store_true", default=True,
                   help="also time the backward (the default; its own fields and roofline)")
    p.add_argument("--no-bwd", dest="bwd", action="store_false", help="skip the backward")
    p.add_argument("--graph", action="store_true",
                   help="time the step as one replayed HIP graph (fbsa_amd.pipeline.GraphStep)")
    p.add_argument("--overlap", action="store_true",
                   help="time the two-stream step (selection overlapped with the forward)")
    p.add_argument("--splits", type=int, default=4, help="row ranges of the overlapped step")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    p.add_argument("--min-warmup-s", type=float, default=0.5,
                   help="continue the untimed warm-up until this much GPU time has run (clock settling)")
    p.add_argument("--cpu-rows", type=int, default=4096, help="query blocks in the CPU sample (4096 = all at config 3)")
    p.add_argument("--qwen", choices=["max", "qmax", "twostage", "lasttok"], default=None,
                   help="time configuration 4 instead (GQA Qwen shape) with this qwen_blocksparse selector")
    p.add_argument("--sweep", action="store_true",
                   help="selection-vs-read crossover sweep (src/bench_crossover.py): one JSON line per "
                        "(block, L) point, then the fitted scaling exponents")
    p.add_argument("--sweep-lengths", default="262144,1048576,4194304,16777216")
    p.add_argument("--sweep-blocks", default="32,64,128")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a plain 1 GiB device-to-device copy 3 times (HBM counter calibration)")
    return p.parse_args()


def warm_up(step, n_min, seconds):
    """Untimed warm-up: at least n_min steps, continued until `seconds` of GPU
    work have run (the clock takes some tens of milliseconds of sustained load to
    settle: the first launches of a cold GPU run up to a third slower). Returns
    the steps run."""
    import torch
    t0, n = time.perf_counter(), 0
    while n < n_min or time.perf_counter() - t0 < seconds:
        step()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def roofline_record(flops, alg_bytes, t_ms, kernel, traffic=None, traffic_note=None):
    """Roofline of one kernel from its algorithmic work: the bound is whichever of
    the MFMA time (flops / 2.5 PFLOP/s) and the HBM time (compulsory bytes / 8 TB/s)
    is larger, and `achieved` / `frac` are measured against that bound."""
    t_mfma = flops / (PEAK_BF16_TFLOPS * 1e12)
    t_hbm = alg_bytes / (PEAK_HBM_GBS * 1e9)
    t = t_ms * 1e-3
    if t_mfma >= t_hbm:
        rec = {"bound": "mfma", "achieved": flops / t / 1e12, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s"}
    else:
        rec = {"bound": "hbm", "achieved": alg_bytes / t / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    rec["frac"] = rec["achieved"] / rec["peak"]
    rec.update({"traffic": traffic, "traffic_source": traffic_note, "kernel": kernel, "flop_per_launch": flops,
                "algorithmic_bytes_per_launch": alg_bytes, "t_mfma_us": t_mfma * 1e6, "t_hbm_us": t_hbm * 1e6})
    return rec


def calibrate_copy():
    """A plain copy of known size: 1 GiB read + 1 GiB written per launch. Its
    FETCH_SIZE / WRITE_SIZE readings give the counter-to-byte factor."""
    import torch
    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": 1 << 30, "launches": 3}), flush=True)


KERNEL_SOURCES = {
    # kernel -> the sources its code is built from (a traffic figure measured on
    # other sources is stale and not reported)
    "fwd_kernel": ["csrc/fbsa_fwd.hip", "csrc/fbsa_common.h", "csrc/fbsa_tiles.h"],
    "dq_kernel": ["csrc/fbsa_bwd.hip", "csrc/fbsa_common.h", "csrc/fbsa_tiles.h"],
    "dkdv_kernel": ["csrc/fbsa_bwd.hip", "csrc/fbsa_common.h", "csrc/fbsa_tiles.h"],
}


def source_sha(kernel):
    """sha256 (16 hex digits) over the kernel's source files."""
    import hashlib
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES[kernel]:
        with open(os.path.join(PKG, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def traffic_from_profiles(kernel, workload):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE,
    copy-kernel calibrated) and recorded in profiles/traffic.json together with
    the sha of the kernel's sources and the commit it was measured at. Returns
    (bytes, note): bytes is None when absent or measured on other sources."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)[workload][kernel]
    except (OSError, KeyError, ValueError):
        return None, "not measured"
    if rec.get("source_sha") != source_sha(kernel):
        return None, f"stale: measured at {rec.get('commit', '?')} on other kernel sources"
    return rec["bytes_per_launch"], f"rocprofv3 FETCH_SIZE+WRITE_SIZE at {rec.get('commit', '?')}, same sources"


def cpu_baseline(q, k, v, bs, topk, rows_wanted):
    """The reference's PyTorch path on the host cores, in the same dtype: block
    pooling (mean over tokens, then heads, src/ssa_model.py:287-288), scores
    qpool kpool^T and convention A (own block + top-k strictly past blocks,
    src/ssa_model.py:151-165), then the gather path: selected K/V blocks
    gathered per query block, additive mask (slot 0 causal triu, slots > 0
    valid iff block < i) and SDPA (src/ssa_model.py:57-90, 167-183). Pooling
    runs over the whole sequence; scores, top-k and attention over a bounded
    sample of `rows_wanted` query blocks spread over the sequence (chunks of 64),
    scaled to all blocks. Threads: torch's intra-op pool (the box sets
    OMP_NUM_THREADS to its CPU share)."""
    import torch
    import torch.nn.functional as F

    nthreads = torch.get_num_threads()
    affinity = len(os.sched_getaffinity(0))
    qc, kc, vc = (t.detach().cpu() for t in (q, k, v))
    B, H, N, D = qc.shape
    nblk = N // bs
    rows = torch.linspace(0, nblk - 1, rows_wanted).round().long().unique()
    NEG = torch.finfo(torch.float32).min
    t0 = time.perf_counter()
    qpool = qc.view(B, H, nblk, bs, D).mean(3).mean(1)  # (B, nblk, D)
    kpool = kc.view(B, H, nblk, bs, D).mean(3).mean(1)
    t_pool = time.perf_counter() - t0

    t_sel = t_fwd = 0.0
    kb = kc.view(B, H, nblk, bs, D)
    vb = vc.view(B, H, nblk, bs, D)
    qb = qc.view(B, H, nblk, bs, D)
    kk_c = min(topk, nblk - 1)
    ar = torch.arange(nblk)
    tri = torch.zeros(bs, (kk_c + 1) * bs)
    tri[:, :bs] = torch.triu(torch.full((bs, bs), NEG), 1)
    for c0 in range(0, len(rows), 64):
        r = rows[c0:c0 + 64]
        t0 = time.perf_counter()
        raw = torch.matmul(qpool[:, r], kpool.transpose(1, 2))  # (B, R, nblk)
        content = raw.masked_fill(ar.view(1, 1, nblk) >= r.view(1, -1, 1), float("-inf"))
        sel = torch.cat([r.view(1, -1, 1).expand(B, -1, 1), content.topk(kk_c, dim=-1).indices], dim=-1)
        t_sel += time.perf_counter() - t0
        t0 = time.perf_counter()
        R, kk = sel.shape[1], sel.shape[2]
        bi = torch.arange(B).view(B, 1, 1, 1)
        hi = torch.arange(H).view(1, H, 1, 1)
        si = sel.view(B, 1, R, kk)
        ks = kb[bi, hi, si].reshape(B, H, R, kk * bs, D)
        vs = vb[bi, hi, si].reshape(B, H, R, kk * bs, D)
        valid = torch.ones(B, R, kk, dtype=torch.bool)
        valid[..., 1:] = sel[..., 1:] < r.view(1, -1, 1)
        blk = torch.zeros(B, R, kk).masked_fill_(~valid, NEG).repeat_interleave(bs, dim=-1).unsqueeze(2)
        mask = (blk + tri).unsqueeze(1).to(qc.dtype)  # (B, 1, R, bs, kk*bs)
        F.scaled_dot_product_attention(qb[:, :, r], ks, vs, attn_mask=mask)
        t_fwd += time.perf_counter() - t0
    scale = nblk / len(rows)
    total = t_pool + (t_sel + t_fwd) * scale
    return {
        "value": B * N / total, "unit": "tokens/s", "cores": nthreads, "kind": "port",
        "cpus_in_affinity_mask": affinity,
        "sample": (f"torch {str(qc.dtype).replace('torch.', '')} on {nthreads} host threads (torch's intra-op "
                   f"pool; {affinity} CPUs in the process affinity mask), the reference's "
                   f"gather path: full q/k pooling ({t_pool:.2f} s) + scores, top-k and gather attention for "
                   f"{len(rows)} of {nblk} query blocks x {H} heads ({t_sel + t_fwd:.2f} s), scaled "
                   f"x{scale:.1f} to all blocks; est. {total:.1f} s per step"),
    }


def cpu_baseline_bwd(q, k, v, do, bs, topk, rows_wanted):
    """The reference's backward on the host cores, in the same dtype: torch
    autograd through the gather path of `cpu_baseline` (gathered K/V blocks,
    additive mask, SDPA; src/ssa_model.py:57-90, 167-183), i.e. dQ for the
    sampled query blocks and dK/dV scattered back into full-size K/V gradients.
    One forward + backward over a bounded sample of `rows_wanted` query blocks
    spread over the sequence; the backward alone is timed and scaled to all
    blocks (the selection is not timed here)."""
    import torch
    import torch.nn.functional as F

    nthreads = torch.get_num_threads()
    qc, kc, vc, dc = (t.detach().cpu() for t in (q, k, v, do))
    B, H, N, D = qc.shape
    nblk = N // bs
    rows = torch.linspace(0, nblk - 1, rows_wanted).round().long().unique()
    NEG = torch.finfo(torch.float32).min
    qpool = qc.view(B, H, nblk, bs, D).mean(3).mean(1)
    kpool = kc.view(B, H, nblk, bs, D).mean(3).mean(1)
    ar = torch.arange(nblk)
    kk_c = min(topk, nblk - 1)
    raw = torch.matmul(qpool[:, rows], kpool.transpose(1, 2))
    content = raw.masked_fill(ar.view(1, 1, nblk) >= rows.view(1, -1, 1), float("-inf"))
    sel = torch.cat([rows.view(1, -1, 1).expand(B, -1, 1), content.topk(kk_c, dim=-1).indices], dim=-1)
    R, kk = sel.shape[1], sel.shape[2]
    kb = kc.view(B, H, nblk, bs, D).detach().requires_grad_(True)
    vb = vc.view(B, H, nblk, bs, D).detach().requires_grad_(True)
    qs = qc.view(B, H, nblk, bs, D)[:, :, rows].detach().requires_grad_(True)
    bi = torch.arange(B).view(B, 1, 1, 1)
    hi = torch.arange(H).view(1, H, 1, 1)
    si = sel.view(B, 1, R, kk)
    ks = kb[bi, hi, si].reshape(B, H, R, kk * bs, D)
    vs = vb[bi, hi, si].reshape(B, H, R, kk * bs, D)
    tri = torch.zeros(bs, kk * bs)
    tri[:, :bs] = torch.triu(torch.full((bs, bs), NEG), 1)
    valid = torch.ones(B, R, kk, dtype=torch.bool)
    valid[..., 1:] = sel[..., 1:] < rows.view(1, -1, 1)
    blk = torch.zeros(B, R, kk).masked_fill_(~valid, NEG).repeat_interleave(bs, dim=-1).unsqueeze(2)
    mask = (blk + tri).unsqueeze(1).to(qc.dtype)
    o = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask)
    g = dc.view(B, H, nblk, bs, D)[:, :, rows]
    t0 = time.perf_counter()
    o.backward(g)
    t_bwd = time.perf_counter() - t0
    scale = nblk / len(rows)
    total = t_bwd * scale
    return {
        "value": B * N / total, "unit": "tokens/s", "cores": nthreads, "kind": "port",
        "sample": (f"torch {str(qc.dtype).replace('torch.', '')} autograd on {nthreads} host threads through "
                   f"the reference's gather path (dQ, and dK/dV scattered into full-size gradients) for "
                   f"{len(rows)} of {nblk} query blocks x {H} heads ({t_bwd:.2f} s), scaled x{scale:.1f} to all "
                   f"blocks; est. {total:.1f} s per backward"),
    }


def rope_partial(x, dims=64, theta=1e7):
    """rotate_half rotary embedding on the first `dims` channels at positions
    0..N-1 (Qwen's partial RoPE, applied by the caller before attention)."""
    import torch
    N = x.shape[2]
    half = dims // 2
    inv = 1.0 / theta ** (torch.arange(0, dims, 2, device=x.device, dtype=torch.float32) / dims)
    ang = torch.arange(N, device=x.device, dtype=torch.float32)[:, None] * inv[None]
    cos, sin = torch.cat([ang.cos()] * 2, -1), torch.cat([ang.sin()] * 2, -1)
    xr = x[..., :dims].float()
    rot = torch.cat([-xr[..., half:], xr[..., :half]], -1)
    return torch.cat([(xr * cos + rot * sin).to(x.dtype), x[..., dims:]], -1)


def qwen_main(a):
    """Configuration 4: B1 N65536 Hq16 Hkv2 D256, block
    128 (nblk 512), post-RoPE q/k, convention B top-32 + own + sink per KV
    head, output gate sigmoid(g). One step = selector.select(q, k) and the
    fused GQA forward with the gate epilogue (qwen_blocksparse drop-ins)."""
    import torch
    import qwen_blocksparse as qb

    dev = "cuda:0"
    torch.cuda.set_device(0)
    B, Hq, Hkv, N, D, bs, topk = 1, 16, 2, 65536, 256, 128, 32
    nblk = N // bs
    g = torch.Generator(device=dev).manual_seed(0)
    q = rope_partial((torch.randn(B, Hq, N, D, generator=g, device=dev)).to(torch.bfloat16))
    k = rope_partial((torch.randn(B, Hkv, N, D, generator=g, device=dev)).to(torch.bfloat16))
    v = torch.randn(B, Hkv, N, D, generator=g, device=dev).to(torch.bfloat16)
    og = torch.randn(B, Hq, N, D, generator=g, device=dev).to(torch.bfloat16)
    S = {"max": qb.SelectMax, "qmax": qb.SelectMaxQMax, "twostage": qb.SelectTwoStage,
         "lasttok": qb.SelectLastTok}[a.qwen](topk=topk, bs=bs, sink=True)
    stream = torch.cuda.current_stream()
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    def step():
        return qb.blocksparse_forward(q, k, v, selector=S, topk=topk, bs=bs, out_gate=og)

    n_warm = warm_up(step, a.warmup, a.min_warmup_s)
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / a.steps
    # per-stage times: the selector alone, then the forward on its indices
    sel_ev, fwd_ev = [], []
    for it in range(a.warmup + a.steps):
        e0, e1, e2 = ev(), ev(), ev()
        e0.record(stream)
        idx = S.select(q, k)
        e1.record(stream)
        qb.blocksparse_forward(q, k, v, selector=_Fixed(idx), topk=topk, bs=bs, out_gate=og)
        e2.record(stream)
        if it >= a.warmup:
            sel_ev.append((e0, e1))
            fwd_ev.append((e1, e2))
    torch.cuda.synchronize()
    t_sel = sum(x.elapsed_time(y) for x, y in sel_ev) / a.steps
    t_fwd = sum(x.elapsed_time(y) for x, y in fwd_ev) / a.steps
    kk = topk + 2
    flops = 4.0 * B * Hq * nblk * kk * bs * bs * D
    # HBM counters were taken on the SelectMax indices (other selectors pick other blocks)
    traffic_b, traffic_note = (traffic_from_profiles("fwd_kernel", f"cfg4_N{N}_Hq{Hq}_Hkv{Hkv}_D{D}_bs{bs}_top{topk}_sink")
                               if a.qwen == "max" else (None, "measured for SelectMax only"))
    out = {
        "metric": f"select+fwd tokens/s at {N // 1000}k tokens, 1 GPU (bf16, GQA Hq{Hq} Hkv{Hkv} D{D} bs{bs} "
                  f"top-{topk} +own +sink, {type(S).__name__})",
        "value": B * N / (ms_step * 1e-3), "unit": "tokens/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "warmup_steps_run": n_warm, "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (q,k,v,g ~ N(0,1), RoPE on q/k dims 0..63, theta 1e7, seed 0, device generator)",
        "config": {"workload": f"BASELINE configs[3]: qwen_blocksparse.{type(S).__name__} + blocksparse_forward "
                               "with the output gate", "B": B, "Hq": Hq, "Hkv": Hkv, "N": N, "D": D, "block": bs,
                   "nblk": nblk, "topk": topk, "kk": kk},
        "ms_select": t_sel, "ms_fwd": t_fwd,
        # L2-miss bytes (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated) per launch over its time:
        # they count every request the L2s send out, Infinity Cache hits included
        "fwd_l2miss_GBps": (traffic_b / (t_fwd * 1e-3) / 1e9) if traffic_b else None,
        "roofline": roofline_record(flops, 2 * B * Hq * N * D * 2 + 2 * B * Hkv * N * D * 2 + B * Hq * N * D * 2,
                                    t_fwd, "fbsa::fwd_kernel<bf16,128,256>", traffic_b, traffic_note),
        "cpu_baseline": None,
    }
    if a.bwd:
        # the backward of the same attention on the selector's indices (dO ~ N(0,1)):
        # prep, transposed index, dQ and dK/dV, timed with HIP events on the stream
        from fbsa_amd import ops
        idx = S.select(q, k).to(torch.int32).contiguous()
        do = torch.randn(B, Hq, N, D, generator=g, device=dev).to(torch.bfloat16)
        sc = D ** -0.5
        o, lse = ops.attention_forward(q, k, v, idx, mask=ops.MASK_TOKEN_CAUSAL, scale=sc, out_gate=og,
                                       need_lse=True)
        bwd_ev = []
        for it in range(a.warmup + a.steps):
            e0, e1 = ev(), ev()
            e0.record(stream)
            ops.attention_backward(q, k, v, idx, o, lse, do, mask=ops.MASK_TOKEN_CAUSAL, scale=sc, out_gate=og)
            e1.record(stream)
            if it >= a.warmup:
                bwd_ev.append((e0, e1))
        torch.cuda.synchronize()
        t_bwd = sum(x.elapsed_time(y) for x, y in bwd_ev) / a.steps
        out["ms_bwd"] = t_bwd
        out["bwd_TFLOPs"] = 2.5 * flops / (t_bwd * 1e-3) / 1e12
    print(json.dumps(out), flush=True)


class _Fixed:
    """Selector returning precomputed indices (separates the stage timings)."""

    def __init__(self, idx):
        self.idx = idx

    def select(self, q, k):
        return self.idx


def crossover_sweep(a):
    """Selection and attention read timed separately over context lengths and
    block sizes, as src/bench_crossover.py:97-153 does: D_model 512, H 8,
    dh 64, top-8 (kk 9), sel_dim 32, causal, bf16, B 1. Selection is the
    BlockSparseSSA module's own stage (MLP selector features pooled per block,
    then the max-of-two-products convention-A top-k on the streaming kernel;
    no nblk x nblk matrix); the read is the fused forward on a fabricated
    causal selection (own block + 8 uniform random blocks, future ones masked)
    with a log-sigmoid gate bias, as make_sel / bsattn_forward there. Times
    are wall clock around synchronised iterations (warm-up 2 / iterations 5
    up to 1M tokens, 1 / 3 beyond), peak memory from torch's allocator."""
    import math
    import torch
    import torch.nn.functional as F
    from fbsa_amd import ops
    from ssa_model import BlockSparseSSA

    dev = "cuda:0"
    torch.cuda.set_device(0)
    Dm, H, topk, sel_dim, B = 512, 8, 8, 32, 1
    dh = Dm // H
    kk = topk + 1
    lengths = [int(x) for x in a.sweep_lengths.split(",")]
    blocks = [int(x) for x in a.sweep_blocks.split(",")]
    g = torch.Generator(device=dev).manual_seed(0)

    def timed(fn, iters, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / iters * 1e3, torch.cuda.max_memory_allocated() / 1e9

    pts = []
    for bs in blocks:
        for L in lengths:
            nblk = L // bs
            iters, warmup = (5, 2) if L <= 1048576 else (3, 1)
            model = BlockSparseSSA(Dm, H, block=bs, topk=topk, sel_dim=sel_dim, causal=True,
                                   use_triton=True).to(dev).to(torch.bfloat16).eval()
            x = torch.randn(B, L, Dm, generator=g, device=dev, dtype=torch.bfloat16)

            def select():
                sq, sk_mean, sk_max = model._pooled(x, B, nblk, bs)
                return model._select(sq, sk_mean, sk_max)

            with torch.no_grad():
                sel_ms, sel_gb = timed(select, iters, warmup)
            del x, model
            torch.cuda.empty_cache()
            q, k, v = (torch.randn(B, H, L, dh, generator=g, device=dev, dtype=torch.bfloat16) for _ in range(3))
            own = torch.arange(nblk, device=dev).view(1, nblk, 1)
            rnd = torch.randint(0, nblk, (B, nblk, kk - 1), generator=g, device=dev)
            sel = torch.cat([own.expand(B, nblk, 1), rnd], -1).to(torch.int32)[:, None]
            gate = F.logsigmoid(torch.randn(B, 1, nblk, kk, generator=g, device=dev))
            with torch.no_grad():
                attn_ms, attn_gb = timed(lambda: ops.attention_forward(q, k, v, sel, mask=ops.MASK_SLOT_CAUSAL,
                                                                       gate=gate), iters, warmup)
            del q, k, v, sel, gate
            torch.cuda.empty_cache()
            pt = {"sweep": "crossover", "block": bs, "L": L, "nblk": nblk, "sel_ms": sel_ms, "attn_ms": attn_ms,
                  "sel_GB": sel_gb, "attn_GB": attn_gb,
                  # the reference's analytical FLOPs (src/bench_crossover.py:104-105)
                  "sel_pflop": 2 * 2 * B * nblk * nblk * sel_dim / 1e15,
                  "attn_pflop": 2 * 2 * B * H * L * kk * bs * dh / 1e15}
            pts.append(pt)
            print(json.dumps(pt), flush=True)

    def slope(xs, ys):
        lx, ly = [math.log(x) for x in xs], [math.log(y) for y in ys]
        mx, my = sum(lx) / len(lx), sum(ly) / len(ly)
        return sum((u - mx) * (w - my) for u, w in zip(lx, ly)) / sum((u - mx) ** 2 for u in lx)

    fit = {}
    for bs in blocks:
        ps = [p for p in pts if p["block"] == bs]
        if len(ps) >= 2:
            fit[str(bs)] = {"sel_exponent": slope([p["L"] for p in ps], [p["sel_ms"] for p in ps]),
                            "attn_exponent": slope([p["L"] for p in ps], [p["attn_ms"] for p in ps])}
    print(json.dumps({"sweep": "crossover_fit", "loglog_slope_vs_L": fit}), flush=True)


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {a.gpus}); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    if a.calibrate_copy:
        calibrate_copy()
        return
    if a.sweep:
        crossover_sweep(a)
        return
    if a.qwen:
        qwen_main(a)
        return
    import torch
    from fbsa_amd import ops, pipeline, selection

    dev = "cuda:0"
    torch.cuda.set_device(0)
    B, H, N, D, bs, topk = 1, a.H, a.N, a.D, a.bs, a.topk
    nblk = N // bs
    kk = 1 + min(topk, nblk - 1)
    g = torch.Generator(device=dev).manual_seed(0)
    sc = D ** -0.5
    q, k, v = ((torch.randn(B, H, N, D, generator=g, device=dev) * sc).to(torch.bfloat16) for _ in range(3))
    do = torch.randn(B, H, N, D, generator=g, device=dev).to(torch.bfloat16) if a.bwd else None

    stream = torch.cuda.current_stream()
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    fwd_ms, sel_ms = [], []

    def seq_step(timed):
        # events only in the per-stage pass: three timing events per step cost
        # about 40 us of GPU time, which the whole-step timing must not include
        if timed:
            e0, e1, e2 = ev(), ev(), ev()
            e0.record(stream)
        sel = selection.select_mean_pooled(q, k, bs, topk, causal=True)
        if timed:
            e1.record(stream)
        o, lse = ops.attention_forward(q, k, v, sel[:, None], mask=ops.MASK_SLOT_CAUSAL, need_lse=True)
        if timed:
            e2.record(stream)
            sel_ms.append((e0, e1))
            fwd_ms.append((e1, e2))
        return sel, o, lse

    graph = pipeline.GraphStep(q, k, v, bs, topk, need_lse=True) if a.graph else None

    def step():
        if graph is not None:
            return graph.replay()
        if not a.overlap:
            return seq_step(False)
        return pipeline.select_and_attend(q, k, v, bs, topk, need_lse=True, splits=a.splits)

    n_warm = warm_up(step, a.warmup, a.min_warmup_s)
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / a.steps
    # unoverlapped launches for the per-stage times and the forward's roofline
    for _ in range(a.warmup):
        seq_step(False)
    for _ in range(a.steps):
        seq_step(True)
    torch.cuda.synchronize()
    t_sel = sum(x.elapsed_time(y) for x, y in sel_ms) / a.steps
    t_fwd = sum(x.elapsed_time(y) for x, y in fwd_ms) / a.steps

    flops = 4.0 * B * H * nblk * kk * bs * bs * D
    wl = f"cfg3_N{N}_H{H}_D{D}_bs{bs}_top{topk}"
    gathered = B * H * nblk * kk * 2 * bs * D * 2
    shape = (H, D, bs, topk)
    cfg_name = ("BASELINE configs[2]" if (N, shape) == (262144, (8, 64, 64, 16))
                else "BASELINE configs[4] (selection-scaling stress)" if (N, shape) == (4194304, (8, 64, 64, 16))
                else "custom shape")
    traffic_b, traffic_note = traffic_from_profiles("fwd_kernel", wl)
    out = {
        "metric": (f"select+fwd tokens/s at {N // 1000}k tokens, 1 GPU (bf16, H{H} D{D} bs{bs} top-{topk}, causal)"),
        "value": B * N / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "warmup_steps_run": n_warm,
        "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (q,k,v ~ N(0,1)/sqrt(D), seed 0, device generator)",
        "config": {"workload": f"{cfg_name}: block-pair selection (mean-pooled q.k, top-{topk}, "
                               "own-first) + fused block-sparse forward, causal",
                   "B": B, "H": H, "N": N, "D": D, "block": bs, "nblk": nblk, "topk": topk, "kk": kk,
                   "step": (f"selection overlapped with the forward ({a.splits} row ranges, 2 streams)" if a.overlap
                            else "pool, select, forward in sequence, replayed as one HIP graph" if a.graph
                            else "pool, select, forward in sequence on one stream")},
        "ms_select": t_sel, "ms_fwd": t_fwd,
        "fwd_gather_GBps_effective": gathered / (t_fwd * 1e-3) / 1e9,
        # bytes the L2s exchange with the fabric per forward launch (rocprofv3 FETCH_SIZE +
        # WRITE_SIZE, copy-calibrated: L2 misses, Infinity Cache hits included) over the
        # launch time, against the 8 TB/s HBM peak
        "fwd_l2miss_GBps": (traffic_b / (t_fwd * 1e-3) / 1e9) if traffic_b else None,
        "fwd_l2miss_frac_of_hbm_peak": (traffic_b / (t_fwd * 1e-3) / 1e9 / PEAK_HBM_GBS) if traffic_b else None,
        # the selection's algorithmic bytes (q and k read once by the pooling) over its time
        "select_hbm_GBps_algorithmic": (2 * B * H * N * D * 2) / (t_sel * 1e-3) / 1e9,
        # compulsory bytes: q, k, v read and o written once (+ the selection list)
        "roofline": roofline_record(flops, 4 * B * H * N * D * 2 + B * nblk * kk * 4, t_fwd,
                                    f"fbsa::fwd_kernel<bf16,{bs},{D}>", traffic_b, traffic_note),
        "strict_roofline_select_fwd_us": None,
    }
    # strict roofline of the whole select+fwd step: selection reads q,k once (HBM), forward FLOPs (MFMA)
    t_star = (2 * B * H * N * D * 2) / (PEAK_HBM_GBS * 1e9) + flops / (PEAK_BF16_TFLOPS * 1e12)
    out["strict_roofline_select_fwd_us"] = t_star * 1e6
    out["frac_of_strict_roofline"] = t_star / (ms_step * 1e-3)

    if a.bwd:
        from fbsa_amd import autograd  # noqa: F401
        bwd_ev = []
        sel, o, lse = seq_step(False)
        for it in range(a.warmup + a.steps):
            e0, e1 = ev(), ev()
            e0.record(stream)
            ops.attention_backward(q, k, v, sel[:, None], o, lse, do, mask=ops.MASK_SLOT_CAUSAL)
            e1.record(stream)
            if it >= a.warmup:
                bwd_ev.append((e0, e1))
        torch.cuda.synchronize()
        t_bwd = sum(x.elapsed_time(y) for x, y in bwd_ev) / a.steps
        # algorithmic backward work: 5 tile products per (query block, slot) against
        # the forward's 2 (S, dP, dV, dQ, dK) = 2.5x the forward's FLOPs; this build
        # recomputes S and dP in both the dQ and the dK/dV kernel (3.5x)
        bflops = 2.5 * flops
        out["ms_bwd"] = t_bwd
        out["bwd"] = {"ms": t_bwd, "tokens_per_s": B * N / (t_bwd * 1e-3),
                      # compulsory bytes: q, k, v, o, dO read, dq, dk, dv written once
                      "roofline": dict(roofline_record(bflops, 8 * B * H * N * D * 2, t_bwd, "backward (all stages)"),
                                       implementation_flop_per_launch=3.5 * flops,
                                       t_star_us=max(bflops / (PEAK_BF16_TFLOPS * 1e12),
                                                     8 * B * H * N * D * 2 / (PEAK_HBM_GBS * 1e9)) * 1e6),
                      "stages": ("row statistics (formed in dQ for bf16 without an output gate, else a prep pass), "
                                 "transposed index (stable radix sort; beside dQ on a second stream), dQ, dK/dV")}
        out["ms_select_fwd_bwd"] = ms_step + t_bwd
        out["train_step_tokens_per_s"] = B * N / ((ms_step + t_bwd) * 1e-3)

    if not a.no_cpu:
        out["cpu_baseline"] = cpu_baseline(q, k, v, bs, topk, a.cpu_rows)
        if a.bwd:
            out["bwd"]["cpu_baseline"] = cpu_baseline_bwd(q, k, v, do, bs, topk, max(1, a.cpu_rows // 16))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
