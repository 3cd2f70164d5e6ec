"""GPU: the library called from several host threads at once.

Each thread runs forward + backward on its own stream (bf16: the backward's
index stage goes to the library's second stream of that thread; fp16: the
staged backward), while the other thread does the same. Every result must
equal, bit for bit, the same problem run alone on the default stream."""
import threading

import pytest
import torch

from _util import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _problem(seed, dt):
    g = torch.Generator().manual_seed(seed)
    B, Hq, Hkv, nblk, bs, D, kk = 1, 4, 2, 64, 64, 64, 9
    L = nblk * bs
    q, do = (randn(g, (B, Hq, L, D), dt, device=DEV) for _ in range(2))
    k, v = (randn(g, (B, Hkv, L, D), dt, device=DEV) for _ in range(2))
    i = torch.arange(nblk).view(1, 1, nblk, 1)
    past = (torch.rand(B, Hkv, nblk, kk - 1, generator=g) * (i + 1)).long()
    sel = torch.cat([i.expand(B, Hkv, nblk, 1), past], -1).to(torch.int32).to(DEV)
    return q, k, v, sel, do


def _run(p):
    from fbsa_amd import ops
    q, k, v, sel, do = p
    mask, sc = ops.MASK_TOKEN_CAUSAL, q.shape[-1] ** -0.5
    o, lse = ops.attention_forward(q, k, v, sel, mask=mask, scale=sc, need_lse=True)
    dq, dk, dv = ops.attention_backward(q, k, v, sel, o, lse, do, mask=mask, scale=sc)[:3]
    return [o, lse, dq, dk, dv]


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_two_host_threads_match_sequential(dt):
    probs = [_problem(50 + t, dt) for t in range(2)]
    ref = [[x.clone() for x in _run(p)] for p in probs]
    torch.cuda.synchronize()
    got = [None, None]
    errs = []

    def worker(t):
        try:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.default_stream())
            with torch.cuda.stream(s):
                outs = None
                for _ in range(3):
                    outs = _run(probs[t])
            s.synchronize()
            got[t] = outs
        except Exception as e:  # reported by the main thread
            errs.append(repr(e))

    print(f"[threads] {dt}: two host threads", flush=True)
    th = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for x in th:
        x.start()
    for x in th:
        x.join(timeout=120)
    assert not any(x.is_alive() for x in th), "a worker thread did not finish"
    assert not errs, errs
    torch.cuda.synchronize()
    for t in range(2):
        for n, a, b in zip(("o", "lse", "dq", "dk", "dv"), got[t], ref[t]):
            assert torch.equal(a, b), f"{dt} thread {t}: {n} differs from the sequential run"
    print(f"[threads] {dt}: both threads match", flush=True)
