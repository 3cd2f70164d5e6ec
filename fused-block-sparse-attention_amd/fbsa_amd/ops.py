"""Device ops over the C ABI: block-sparse attention forward/backward, pooling, selection.

All tensors live on the GPU; launches go on torch's current stream. Outputs
are allocated with torch. Arguments are checked by the library before launch
(ValueError on a bad shape/layout); there is no CPU path.
"""
import torch

from . import _lib

MASK_NONE, MASK_SLOT_CAUSAL, MASK_TOKEN_CAUSAL = _lib.MASK_NONE, _lib.MASK_SLOT_CAUSAL, _lib.MASK_TOKEN_CAUSAL
SUPPORTED_D = (32, 64, 128, 256)
SUPPORTED_BS = (16, 32, 64, 128)
_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


class DenseSelection:
    """Every key block selected, slot s holding block s (FBSA_FLAG_DENSE): the
    implicit (B, 1, nblk, nblk) list of dense attention, never stored. With
    MASK_TOKEN_CAUSAL query block i reads blocks 0..i, with MASK_NONE all; the
    dense fast path of ``blocksparse_forward`` (src/qwen_blocksparse.py:37-41)."""

    def __init__(self, B, nblk):
        self.shape = (B, 1, nblk, nblk)

    def dim(self):
        return 4


def _dtype_code(t):
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"fbsa: unsupported dtype {t.dtype}") from None


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("fbsa: tensors must be on the GPU (no CPU path)")


def _kernel_ready(x, min_align=16):
    """Unit stride on D, row starts and base 16-byte aligned (the kernels load
    rows with 16-byte vector / direct-to-LDS loads); copy otherwise."""
    es = x.element_size()
    ok = x.stride(-1) == 1 and x.data_ptr() % min_align == 0 and all(
        (s * es) % 16 == 0 for s in x.stride()[:-1])
    return x if ok else x.contiguous()


def padded_head_dim(D):
    for d in SUPPORTED_D:
        if D <= d:
            return d
    raise ValueError(f"fbsa: head dim {D} > 256 is not supported")


def _pad_d(x, Dp):
    if x is None or x.shape[-1] == Dp:
        return x
    return torch.nn.functional.pad(x, (0, Dp - x.shape[-1]))


def _strides3(t):
    return (t.stride(0), t.stride(1), t.stride(2))


def make_desc(q, k, v, o, sel, *, mask, scale, l_valid, dout=None, out_gate=None):
    B, Hq, L, D = q.shape
    _, hsel, nblk, kk = sel.shape
    d = _lib.AttnDesc()
    d.dtype = _dtype_code(q)
    d.mask = mask
    d.B, d.Hq, d.Hkv, d.L, d.D = B, Hq, k.shape[1], L, D
    d.bs = L // nblk
    d.nblk, d.kk, d.hsel = nblk, kk, hsel
    d.l_valid = L if l_valid is None else int(l_valid)
    d.scale = float(scale)
    d.flags = _lib.FLAG_DENSE if isinstance(sel, DenseSelection) else 0
    d.sq[:] = _strides3(q)
    d.sk[:] = _strides3(k)
    d.sv[:] = _strides3(v)
    d.so[:] = _strides3(o)
    d.sdo[:] = _strides3(dout) if dout is not None else (0, 0, 0)
    d.sog[:] = _strides3(out_gate) if out_gate is not None else (0, 0, 0)
    return d


def _check_common(q, k, v, sel, gate):
    if isinstance(sel, DenseSelection):
        if gate is not None:
            raise ValueError("fbsa: a dense selection takes no gate")
        sel = None
    _require_cuda(q, k, v, sel, gate)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("fbsa: q, k, v must be 4-D (B, H, L, D)")
    if k.shape != v.shape or k.shape[0] != q.shape[0] or k.shape[2:] != q.shape[2:]:
        raise ValueError(f"fbsa: shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("fbsa: q, k, v must share a dtype")
    if sel is not None and (sel.dim() != 4 or sel.shape[0] != q.shape[0]):
        raise ValueError(f"fbsa: sel must be (B, Hsel, nblk, kk), got {tuple(sel.shape)}")
    if gate is not None and gate.shape != sel.shape:
        raise ValueError(f"fbsa: gate shape {tuple(gate.shape)} != sel shape {tuple(sel.shape)}")


def prepare_forward(q, k, v, sel, *, mask, scale=None, gate=None, l_valid=None, out_gate=None, need_lse=False):
    """Checks and kernel-ready views for the forward, and its outputs (allocated,
    not yet written). sel must already be the int32 tensor the kernel will read
    (an int32 contiguous sel is used in place, so it may be filled later)."""
    _check_common(q, k, v, sel, gate)
    B, Hq, L, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    Dp = padded_head_dim(D)
    qk = [_kernel_ready(_pad_d(t, Dp)) for t in (q, k, v)]
    og = None
    if out_gate is not None:
        _require_cuda(out_gate)
        if out_gate.shape != q.shape or out_gate.dtype != q.dtype:
            raise ValueError("fbsa: out_gate must match q's shape and dtype")
        og = _pad_d(out_gate, Dp)
        if og.stride(-1) != 1:
            og = og.contiguous()
    dense = isinstance(sel, DenseSelection)
    sel32 = sel if dense else sel.to(torch.int32).contiguous()
    gate32 = gate.to(torch.float32).contiguous() if gate is not None else None
    o = torch.empty(B, Hq, L, Dp, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, Hq, L, dtype=torch.float32, device=q.device) if need_lse else None
    if sel32.shape[2] == 0 or L % sel32.shape[2]:
        raise ValueError(f"fbsa: L={L} is not a multiple of nblk={sel32.shape[2]}")
    d = make_desc(qk[0], qk[1], qk[2], o, sel32, mask=mask, scale=scale, l_valid=l_valid, out_gate=og)
    return {"d": d, "qkv": qk, "sel": None if dense else sel32, "gate": gate32, "og": og, "o": o, "lse": lse,
            "D": D, "Dp": Dp, "nblk": sel32.shape[2]}


def launch_forward(prep, blocks=None):
    """Runs the forward of query blocks [i0, i1) (all when None) on the current stream."""
    i0, i1 = (0, prep["nblk"]) if blocks is None else blocks
    qk = prep["qkv"]
    lib = _lib.load()
    _lib.check(lib.fbsa_fwd_rows(prep["d"], i0, i1, _ptr(qk[0]), _ptr(qk[1]), _ptr(qk[2]), _ptr(prep["sel"]),
                                 _ptr(prep["gate"]), _ptr(prep["og"]), _ptr(prep["o"]), _ptr(prep["lse"]),
                                 _stream()), "fbsa_fwd")


def finish_forward(prep, need_lse):
    o = prep["o"]
    if prep["Dp"] != prep["D"]:
        o = o[..., :prep["D"]]
    return (o, prep["lse"]) if need_lse else o


def attention_forward(q, k, v, sel, *, mask, scale=None, gate=None, l_valid=None,
                      out_gate=None, need_lse=False):
    """Fused block-sparse attention forward.

    q (B,Hq,L,D); k, v (B,Hkv,L,D); sel (B,Hsel,nblk,kk) integer block ids with
    Hsel in {1, Hkv}, or a ``DenseSelection`` (every block, no list); gate (B,Hsel,nblk,kk) additive bias (cast to fp32);
    out_gate (B,Hq,L,D) (any strides): o <- o * sigmoid(out_gate).
    Returns o (and the fp32 natural-log LSE (B,Hq,L) when need_lse).
    """
    prep = prepare_forward(q, k, v, sel, mask=mask, scale=scale, gate=gate, l_valid=l_valid, out_gate=out_gate,
                           need_lse=need_lse)
    launch_forward(prep)
    return finish_forward(prep, need_lse)


def attention_backward(q, k, v, sel, o, lse, dout, *, mask, scale=None, gate=None, l_valid=None,
                       out_gate=None, need_dgate=False):
    """Backward of ``attention_forward`` (no atomics; bitwise repeatable).

    o and lse are the forward's outputs (o gated when out_gate is given).
    Returns (dq, dk, dv, dgate, dout_gate): dq (B,Hq,L,D), dk/dv (B,Hkv,L,D) in
    q's dtype; dgate (B,Hsel,nblk,kk) fp32 when need_dgate (the gradient of the
    additive gate, summed over the heads sharing the selection), else None;
    dout_gate (B,Hq,L,D) when out_gate is given, else None.
    """
    _check_common(q, k, v, sel, gate)
    _require_cuda(o, lse, dout, out_gate)
    B, Hq, L, D = q.shape
    if o.shape != q.shape or dout.shape != q.shape:
        raise ValueError("fbsa: o and dout must have q's shape")
    if lse.shape != (B, Hq, L) or lse.dtype != torch.float32:
        raise ValueError("fbsa: lse must be fp32 (B, Hq, L)")
    scale = D ** -0.5 if scale is None else scale
    Dp = padded_head_dim(D)
    qk = [_kernel_ready(_pad_d(t, Dp)) for t in (q, k, v)]
    o_p = _kernel_ready(_pad_d(o.to(q.dtype), Dp))
    do_p = _kernel_ready(_pad_d(dout.to(q.dtype), Dp))
    og = None
    if out_gate is not None:
        if out_gate.shape != q.shape or out_gate.dtype != q.dtype:
            raise ValueError("fbsa: out_gate must match q's shape and dtype")
        og = _pad_d(out_gate, Dp)
        if og.stride(-1) != 1:
            og = og.contiguous()
    dense = isinstance(sel, DenseSelection)
    sel32 = sel if dense else sel.to(torch.int32).contiguous()
    gate32 = gate.to(torch.float32).contiguous() if gate is not None else None
    lse_c = lse.contiguous()
    nblk = sel32.shape[2]
    if nblk == 0 or L % nblk:
        raise ValueError(f"fbsa: L={L} is not a multiple of nblk={nblk}")
    dev = q.device
    dq = torch.empty(B, Hq, L, Dp, dtype=q.dtype, device=dev)
    dk = torch.empty(B, k.shape[1], L, Dp, dtype=q.dtype, device=dev)
    dv = torch.empty_like(dk)
    dgate = torch.empty(sel32.shape, dtype=torch.float32, device=dev) if need_dgate else None
    dog = torch.empty(B, Hq, L, Dp, dtype=q.dtype, device=dev) if og is not None else None
    d = make_desc(qk[0], qk[1], qk[2], o_p, sel32, mask=mask, scale=scale, l_valid=l_valid, dout=do_p,
                  out_gate=og)
    d.flags |= (_lib.FLAG_OUT_GATE if og is not None else 0) | (_lib.FLAG_DGATE if need_dgate else 0)
    lib = _lib.load()
    nbytes = lib.fbsa_bwd_workspace_bytes(d)
    if nbytes == 0:
        _lib.check(_lib.EINVAL, "fbsa_bwd_workspace_bytes")
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=dev)
    base = ws.data_ptr()
    wp = (base + 255) // 256 * 256
    _lib.check(lib.fbsa_bwd(d, _ptr(qk[0]), _ptr(qk[1]), _ptr(qk[2]), _ptr(o_p), _ptr(do_p), _ptr(lse_c),
                            None if dense else _ptr(sel32), _ptr(gate32), _ptr(og), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dgate),
                            _ptr(dog), wp, nbytes, _stream()), "fbsa_bwd")
    if Dp != D:
        dq, dk, dv = dq[..., :D], dk[..., :D], dv[..., :D]
        dog = dog[..., :D] if dog is not None else None
    return dq, dk, dv, dgate, dog


def block_mass(q, k, bs, scale=None):
    """Dense causal per-block attention mass (B, Hq, nblk, nblk) fp32 on the GPU
    kernel: entry (i, j) is the mean over query block i's rows t of the softmax
    probability summed over key block j's keys s <= t, zero above the diagonal
    (``capture_mass``, src/eval_qwen_ppl.py:65-108, before its group mean).
    Scores are rnd(rnd(q.k) * scale) in q's dtype, as torch's 16-bit matmul
    rounds them; the softmax is fp32. q (B, Hq, L, D), k (B, Hkv, L, D) bf16 or
    fp16, L a multiple of bs (64 or 128), D in {64, 128, 256}."""
    _require_cuda(q, k)
    if q.dim() != 4 or k.dim() != 4 or q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:]:
        raise ValueError("fbsa.block_mass: q (B,Hq,L,D) and k (B,Hkv,L,D) expected")
    if q.dtype != k.dtype or q.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("fbsa.block_mass: q and k must both be bf16 or both fp16")
    B, Hq, L, D = q.shape
    if Hq % k.shape[1]:
        raise ValueError(f"fbsa.block_mass: Hq={Hq} not a multiple of Hkv={k.shape[1]}")
    if L % bs:
        raise ValueError(f"fbsa.block_mass: L={L} is not a multiple of bs={bs}")
    scale = D ** -0.5 if scale is None else scale
    qk = [_kernel_ready(t) for t in (q, k)]
    nblk = L // bs
    d = _lib.AttnDesc()
    d.dtype, d.mask = _dtype_code(q), _lib.MASK_TOKEN_CAUSAL
    d.B, d.Hq, d.Hkv, d.L, d.D = B, Hq, k.shape[1], L, D
    d.bs, d.nblk, d.kk, d.hsel, d.l_valid = bs, nblk, 1, 1, L
    d.scale, d.flags = float(scale), 0
    d.sq[:] = _strides3(qk[0])
    d.sk[:] = _strides3(qk[1])
    lib = _lib.load()
    mass = torch.empty(B, Hq, nblk, nblk, dtype=torch.float32, device=q.device)
    ws = torch.empty((lib.fbsa_block_mass_workspace_bytes(d) + 3) // 4, dtype=torch.float32, device=q.device)
    _lib.check(lib.fbsa_block_mass(d, _ptr(qk[0]), _ptr(qk[1]), _ptr(mass), _ptr(ws), _stream()), "fbsa_block_mass")
    return mass

