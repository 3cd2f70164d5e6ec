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
    d.flags = 0
    d.sq[:] = _strides3(q)
    d.sk[:] = _strides3(k)
    d.sv[:] = _strides3(v)
    d.so[:] = _strides3(o)
    d.sdo[:] = _strides3(dout) if dout is not None else (0, 0, 0)
    d.sog[:] = _strides3(out_gate) if out_gate is not None else (0, 0, 0)
    return d


def _check_common(q, k, v, sel, gate):
    _require_cuda(q, k, v, sel, gate)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("fbsa: q, k, v must be 4-D (B, H, L, D)")
    if k.shape != v.shape or k.shape[0] != q.shape[0] or k.shape[2:] != q.shape[2:]:
        raise ValueError(f"fbsa: shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("fbsa: q, k, v must share a dtype")
    if sel.dim() != 4 or sel.shape[0] != q.shape[0]:
        raise ValueError(f"fbsa: sel must be (B, Hsel, nblk, kk), got {tuple(sel.shape)}")
    if gate is not None and gate.shape != sel.shape:
        raise ValueError(f"fbsa: gate shape {tuple(gate.shape)} != sel shape {tuple(sel.shape)}")


def attention_forward(q, k, v, sel, *, mask, scale=None, gate=None, l_valid=None,
                      out_gate=None, need_lse=False):
    """Fused block-sparse attention forward.

    q (B,Hq,L,D); k, v (B,Hkv,L,D); sel (B,Hsel,nblk,kk) integer block ids with
    Hsel in {1, Hkv}; gate (B,Hsel,nblk,kk) additive bias (cast to fp32);
    out_gate (B,Hq,L,D) (any strides): o <- o * sigmoid(out_gate).
    Returns o (and the fp32 natural-log LSE (B,Hq,L) when need_lse).
    """
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
    sel32 = sel.to(torch.int32).contiguous()
    gate32 = gate.to(torch.float32).contiguous() if gate is not None else None
    o = torch.empty(B, Hq, L, Dp, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, Hq, L, dtype=torch.float32, device=q.device) if need_lse else None
    if sel32.shape[2] == 0 or L % sel32.shape[2]:
        raise ValueError(f"fbsa: L={L} is not a multiple of nblk={sel32.shape[2]}")
    d = make_desc(qk[0], qk[1], qk[2], o, sel32, mask=mask, scale=scale, l_valid=l_valid, out_gate=og)
    lib = _lib.load()
    _lib.check(lib.fbsa_fwd(d, _ptr(qk[0]), _ptr(qk[1]), _ptr(qk[2]), _ptr(sel32), _ptr(gate32),
                            _ptr(og), _ptr(o), _ptr(lse), _stream()), "fbsa_fwd")
    if Dp != D:
        o = o[..., :D]
    return (o, lse) if need_lse else o
