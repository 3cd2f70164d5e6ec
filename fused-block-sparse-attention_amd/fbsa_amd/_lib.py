"""ctypes binding of libfbsa.so (the gfx950 HIP library) -- the only compute path.

There is no fallback: if the library is missing or fails to load, every op
raises. Build it with ``make -C fused-block-sparse-attention_amd`` (or
``__graft_entry__.build()``).
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfbsa.so")

F32, BF16, F16 = 0, 1, 2
MASK_NONE, MASK_SLOT_CAUSAL, MASK_TOKEN_CAUSAL = 0, 1, 2
OK, EINVAL, EUNSUPPORTED, EHIP, EWORKSPACE = 0, 1, 2, 3, 4
POOL_MEAN_TOK_THEN_GRP, POOL_MEAN_GRP_THEN_TOK, POOL_MAX, POOL_MIN, POOL_MINMAX = 0, 1, 2, 3, 4
SCORE_DOT, SCORE_MAX2, SCORE_QUEST = 0, 1, 2
SEL_OWN_FIRST, SEL_SORTED_SINK, SEL_SORTED_TOPK = 0, 1, 2
QMAX_EXACT = 1
SEL_CHUNK_SHIFT = 8
FLAG_OUT_GATE, FLAG_DENSE, FLAG_DGATE = 1, 2, 4
SELECT_SCRATCH_BYTES = 32 << 20   # FBSA_SELECT_SCRATCH_BYTES

_i64x3 = ctypes.c_int64 * 3


class AttnDesc(ctypes.Structure):
    """Mirror of ``fbsa_attn_desc`` (include/fbsa.h)."""
    _fields_ = [
        ("dtype", ctypes.c_int32), ("mask", ctypes.c_int32),
        ("B", ctypes.c_int64), ("Hq", ctypes.c_int64), ("Hkv", ctypes.c_int64),
        ("L", ctypes.c_int64), ("D", ctypes.c_int64), ("bs", ctypes.c_int64),
        ("nblk", ctypes.c_int64), ("kk", ctypes.c_int64), ("hsel", ctypes.c_int64),
        ("l_valid", ctypes.c_int64),
        ("scale", ctypes.c_float), ("flags", ctypes.c_int32),
        ("sq", _i64x3), ("sk", _i64x3), ("sv", _i64x3), ("so", _i64x3),
        ("sdo", _i64x3), ("sog", _i64x3),
    ]


class PoolDesc(ctypes.Structure):
    """Mirror of ``fbsa_pool_desc``."""
    _fields_ = [
        ("dtype", ctypes.c_int32), ("op", ctypes.c_int32),
        ("B", ctypes.c_int64), ("H", ctypes.c_int64), ("L", ctypes.c_int64),
        ("D", ctypes.c_int64), ("bs", ctypes.c_int64), ("nblk", ctypes.c_int64),
        ("grp", ctypes.c_int64), ("l_valid", ctypes.c_int64),
        ("sx", _i64x3),
    ]


class SelectDesc(ctypes.Structure):
    """Mirror of ``fbsa_select_desc``."""
    _fields_ = [
        ("dtype", ctypes.c_int32), ("score", ctypes.c_int32), ("convention", ctypes.c_int32),
        ("causal", ctypes.c_int32), ("sink", ctypes.c_int32), ("flags", ctypes.c_int32),
        ("B", ctypes.c_int64), ("H", ctypes.c_int64), ("nblk", ctypes.c_int64),
        ("D", ctypes.c_int64), ("topk", ctypes.c_int64), ("kk", ctypes.c_int64),
    ]


class QmaxDesc(ctypes.Structure):
    """Mirror of ``fbsa_qmax_desc``."""
    _fields_ = [
        ("dtype", ctypes.c_int32), ("convention", ctypes.c_int32), ("sink", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("B", ctypes.c_int64), ("H", ctypes.c_int64), ("nblk", ctypes.c_int64),
        ("D", ctypes.c_int64), ("tok", ctypes.c_int64), ("la", ctypes.c_int64),
        ("topk", ctypes.c_int64), ("kk", ctypes.c_int64), ("ncand", ctypes.c_int64),
    ]


_vp = ctypes.c_void_p
# name -> (restype, argtypes); every symbol declared in include/fbsa.h
SIGNATURES = {
    "fbsa_last_error": (ctypes.c_char_p, []),
    "fbsa_version": (ctypes.c_int, []),
    "fbsa_fwd": (ctypes.c_int, [ctypes.POINTER(AttnDesc), _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "fbsa_fwd_rows": (ctypes.c_int, [ctypes.POINTER(AttnDesc), ctypes.c_int64, ctypes.c_int64]
                      + [_vp] * 9),
    "fbsa_block_mass_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(AttnDesc)]),
    "fbsa_block_mass": (ctypes.c_int, [ctypes.POINTER(AttnDesc), _vp, _vp, _vp, _vp, _vp]),
    "fbsa_pool": (ctypes.c_int, [ctypes.POINTER(PoolDesc), _vp, _vp, _vp, _vp]),
    "fbsa_select_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(SelectDesc)]),
    "fbsa_select": (ctypes.c_int, [ctypes.POINTER(SelectDesc), _vp, _vp, _vp, _vp, _vp, _vp,
                                   ctypes.c_size_t, _vp]),
    "fbsa_select_rows": (ctypes.c_int, [ctypes.POINTER(SelectDesc), ctypes.c_int64, ctypes.c_int64,
                                        _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "fbsa_select_noalloc": (ctypes.c_int, [ctypes.POINTER(SelectDesc), _vp, _vp, _vp, _vp, _vp, _vp]),
    "fbsa_select_mean_pooled": (ctypes.c_int, [ctypes.POINTER(PoolDesc), _vp, _vp, ctypes.POINTER(PoolDesc), _vp, _vp,
                                               ctypes.POINTER(SelectDesc), _vp, _vp, _vp, ctypes.c_size_t, _vp]),
    "fbsa_select_qmax_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(QmaxDesc)]),
    "fbsa_select_qmax": (ctypes.c_int, [ctypes.POINTER(QmaxDesc), _vp, _vp, _vp, _vp, _vp, _vp,
                                        ctypes.c_size_t, _vp]),
    "fbsa_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(AttnDesc)]),
    "fbsa_bwd_prep": (ctypes.c_int, [ctypes.POINTER(AttnDesc)] + [_vp] * 6 + [ctypes.c_size_t, _vp]),
    "fbsa_transpose_index": (ctypes.c_int, [ctypes.POINTER(AttnDesc), _vp, _vp, ctypes.c_size_t, _vp]),
    "fbsa_bwd_dq": (ctypes.c_int, [ctypes.POINTER(AttnDesc)] + [_vp] * 9 + [ctypes.c_size_t, _vp]),
    "fbsa_bwd_dkdv": (ctypes.c_int, [ctypes.POINTER(AttnDesc)] + [_vp] * 8 + [ctypes.c_size_t, _vp]),
    "fbsa_bwd": (ctypes.c_int, [ctypes.POINTER(AttnDesc)] + [_vp] * 15 + [ctypes.c_size_t, _vp]),
}

_lib = None


def open_library(path):
    """ctypes handle of a libfbsa build at `path` with every entry point typed."""
    if not os.path.exists(path):
        raise RuntimeError(f"fbsa: HIP library not built ({path} missing); "
                           "run `make -C fused-block-sparse-attention_amd`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def load():
    """Load libfbsa.so once; raise if it is absent (no CPU fallback)."""
    global _lib
    if _lib is None:
        _lib = open_library(LIB_PATH)
    return _lib


def use(lib):
    """Route every op through `lib` (a handle from open_library; None restores
    the default build on the next call). Returns the handle in use before."""
    global _lib
    prev, _lib = _lib, lib
    return prev


class FbsaError(RuntimeError):
    pass


def check(status, what):
    """Map a C status to a Python exception (ValueError for bad arguments)."""
    if status == OK:
        return
    msg = load().fbsa_last_error().decode(errors="replace")
    if status in (EINVAL, EUNSUPPORTED, EWORKSPACE):
        raise ValueError(f"{what}: {msg}")
    raise FbsaError(f"{what}: {msg}")
