"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, and rejects bad arguments on the host before any launch."""
import ctypes
import os
import re

import pytest

from fbsa_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "fbsa.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(fbsa_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert "fbsa_fwd" in names and "fbsa_select" in names and "fbsa_bwd" in names
    for n in names:
        assert hasattr(lib, n), f"libfbsa.so does not export {n}"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with include/fbsa.h"


def test_struct_layout_matches_header():
    # int32 dtype/mask, 10 int64 sizes, float scale + int32 flags, 6 x 3 int64 strides
    assert ctypes.sizeof(_lib.AttnDesc) == 8 + 10 * 8 + 8 + 18 * 8
    assert ctypes.sizeof(_lib.PoolDesc) == 8 + 8 * 8 + 3 * 8
    assert ctypes.sizeof(_lib.SelectDesc) == 6 * 4 + 6 * 8


def _desc(**kw):
    d = _lib.AttnDesc()
    d.dtype, d.mask = _lib.BF16, _lib.MASK_SLOT_CAUSAL
    d.B, d.Hq, d.Hkv, d.L, d.D, d.bs, d.nblk, d.kk, d.hsel, d.l_valid = 1, 2, 2, 256, 64, 64, 4, 3, 1, 256
    d.scale = 0.125
    for s in ("sq", "sk", "sv", "so", "sdo", "sog"):
        getattr(d, s)[:] = (2 * 256 * 64, 256 * 64, 64)
    for k, v in kw.items():
        setattr(d, k, v)
    return d


DUMMY = 1 << 20  # never dereferenced: validation fails first


@pytest.mark.parametrize("field,value,needle", [
    ("bs", 48, "block size"),
    ("D", 80, "head dim"),
    ("L", 250, "nblk*bs"),
    ("Hkv", 3, "multiple"),
    ("hsel", 3, "hsel"),
    ("l_valid", 0, "l_valid"),
    ("dtype", 7, "dtype"),
    ("mask", 9, "mask"),
    ("kk", 0, "positive"),
])
def test_fwd_rejects_bad_descriptor(field, value, needle):
    lib = _lib.load()
    d = _desc(**{field: value})
    st = lib.fbsa_fwd(d, DUMMY, DUMMY, DUMMY, DUMMY, None, None, DUMMY, None, None)
    assert st in (_lib.EINVAL, _lib.EUNSUPPORTED)
    assert needle in lib.fbsa_last_error().decode()


def test_fwd_rejects_null_and_misaligned_pointers():
    lib = _lib.load()
    d = _desc()
    assert lib.fbsa_fwd(d, None, DUMMY, DUMMY, DUMMY, None, None, DUMMY, None, None) == _lib.EINVAL
    assert lib.fbsa_fwd(d, DUMMY + 2, DUMMY, DUMMY, DUMMY, None, None, DUMMY, None, None) == _lib.EINVAL
    assert "aligned" in lib.fbsa_last_error().decode()
    d.sq[2] = 65  # row stride not a multiple of 16 bytes
    assert lib.fbsa_fwd(d, DUMMY, DUMMY, DUMMY, DUMMY, None, None, DUMMY, None, None) == _lib.EINVAL


def test_select_rejects_bad_budget():
    lib = _lib.load()
    d = _lib.SelectDesc()
    d.dtype, d.score, d.convention, d.causal = _lib.BF16, _lib.SCORE_DOT, _lib.SEL_OWN_FIRST, 1
    d.B, d.H, d.nblk, d.D, d.topk, d.kk = 1, 1, 64, 64, 8, 8   # convention A needs kk = 9
    assert lib.fbsa_select(d, DUMMY, DUMMY, None, DUMMY, None, None, 0, None) == _lib.EINVAL
    assert "kk" in lib.fbsa_last_error().decode()
    # budgets past the wave lists run one workgroup per row, up to 4096
    d.nblk, d.topk, d.kk = 8192, 4097, 4098
    assert lib.fbsa_select(d, DUMMY, DUMMY, None, DUMMY, None, None, 0, None) == _lib.EUNSUPPORTED
    assert "4096" in lib.fbsa_last_error().decode()


def test_select_flags_and_workspace_size():
    lib = _lib.load()
    d = _lib.SelectDesc()
    d.dtype, d.score, d.convention, d.causal = _lib.BF16, _lib.SCORE_DOT, _lib.SEL_OWN_FIRST, 1
    d.B, d.H, d.nblk, d.D, d.topk, d.kk = 1, 8, 4096, 64, 16, 17
    d.flags = 1  # only the chunk field (bits 8..23) is defined
    assert lib.fbsa_select(d, DUMMY, DUMMY, None, DUMMY, None, None, 0, None) == _lib.EINVAL
    assert "flags" in lib.fbsa_last_error().decode()
    # MFMA engine workspace: 4 padded norm arrays + per-(row, chunk) partial top-k lists
    d.flags = 0
    auto = lib.fbsa_select_workspace_bytes(d)
    npad = 8 * 4096
    assert auto >= 4 * npad * 4
    d.flags = 4 << _lib.SEL_CHUNK_SHIFT   # 16 chunks of 4 tiles: larger partial-list area
    assert lib.fbsa_select_workspace_bytes(d) == 4 * npad * 4 + 256 + 8 * 4096 * 16 * 16 * 8
    # automatic chunking: rows are cut into chunks (of at least 8 tiles) only
    # when the row blocks alone leave the GPU idle
    d.flags = 0
    assert auto == 4 * npad * 4 + 256 + 8 * 4096 * 1 * 16 * 8      # 512 row blocks: whole rows
    d.H = 1
    assert lib.fbsa_select_workspace_bytes(d) == 4 * 4096 * 4 + 256 + 4096 * 8 * 16 * 8  # 64 row blocks: 8 chunks
    d.H = 8
    d.dtype = _lib.F32   # fp32 operands take the fp64 engine: no workspace
    assert lib.fbsa_select_workspace_bytes(d) == 0


def test_select_mean_pooled_validates_descriptors():
    lib = _lib.load()

    def pdesc(H):
        d = _lib.PoolDesc()
        d.dtype, d.op = _lib.BF16, _lib.POOL_MEAN_TOK_THEN_GRP
        d.B, d.H, d.L, d.D, d.bs, d.nblk, d.grp, d.l_valid = 1, H, 4096, 64, 64, 64, H, 4096
        d.sx[:] = (H * 4096 * 64, 4096 * 64, 64)
        return d
    dq, dk = pdesc(8), pdesc(2)
    s = _lib.SelectDesc()
    s.dtype, s.score, s.convention, s.causal = _lib.BF16, _lib.SCORE_DOT, _lib.SEL_OWN_FIRST, 1
    s.B, s.H, s.nblk, s.D, s.topk, s.kk = 1, 1, 64, 64, 16, 17

    def call():
        return lib.fbsa_select_mean_pooled(dq, DUMMY, DUMMY, dk, DUMMY, DUMMY, s, DUMMY, None, None, 0, None)
    dq.op = _lib.POOL_MEAN_GRP_THEN_TOK
    assert call() == _lib.EINVAL and "MEAN_TOK_THEN_GRP" in lib.fbsa_last_error().decode()
    dq.op = _lib.POOL_MEAN_TOK_THEN_GRP
    s.score = _lib.SCORE_MAX2
    assert call() == _lib.EINVAL and "DOT" in lib.fbsa_last_error().decode()
    s.score = _lib.SCORE_DOT
    for field, bad in (("H", 2), ("nblk", 32), ("D", 32)):
        good = getattr(s, field)
        setattr(s, field, bad)
        assert call() == _lib.EINVAL and "disagree" in lib.fbsa_last_error().decode(), field
        setattr(s, field, good)
    dk.l_valid = 4000
    assert call() == _lib.EINVAL and "disagree" in lib.fbsa_last_error().decode()
    dk.l_valid = 4096
    s.kk = 16
    assert call() == _lib.EINVAL and "kk" in lib.fbsa_last_error().decode()


def test_row_range_entry_points_validate_ranges():
    lib = _lib.load()
    d = _lib.SelectDesc()
    d.dtype, d.score, d.convention, d.causal = _lib.BF16, _lib.SCORE_DOT, _lib.SEL_OWN_FIRST, 1
    d.B, d.H, d.nblk, d.D, d.topk, d.kk = 1, 1, 64, 64, 8, 9
    for r0, r1 in ((-1, 10), (10, 5), (0, 65)):
        assert lib.fbsa_select_rows(d, r0, r1, DUMMY, DUMMY, None, DUMMY, None, None, 0, None) == _lib.EINVAL
        assert "range" in lib.fbsa_last_error().decode()
    a = _desc()
    for r0, r1 in ((-1, 1), (3, 2), (0, a.nblk + 1)):
        assert lib.fbsa_fwd_rows(a, r0, r1, DUMMY, DUMMY, DUMMY, DUMMY, None, None, DUMMY, None, None) == _lib.EINVAL
        assert "range" in lib.fbsa_last_error().decode()


def test_pipeline_row_splits_cover_rows():
    from fbsa_amd.pipeline import _row_splits
    for nblk in (1, 63, 64, 65, 700, 4096, 65536):
        for splits in (1, 2, 4, 7):
            r = _row_splits(nblk, splits)
            assert r[0][0] == 0 and r[-1][1] == nblk
            assert all(a < b for a, b in r) and all(r[x][1] == r[x + 1][0] for x in range(len(r) - 1))
            assert all(a % 64 == 0 for a, _ in r)


def test_python_ops_require_gpu_tensors():
    import torch
    from fbsa_amd import ops
    q = torch.zeros(1, 1, 64, 64, dtype=torch.bfloat16)
    sel = torch.zeros(1, 1, 1, 1, dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        ops.attention_forward(q, q, q, sel, mask=ops.MASK_SLOT_CAUSAL)


def test_dense_flag_validation_and_small_backward_workspace():
    # FBSA_FLAG_DENSE: implicit all-blocks list (kk == nblk, no sel, no gate,
    # token-causal or none); its backward stores only the list offsets
    lib = _lib.load()
    d = _desc(kk=4, mask=_lib.MASK_TOKEN_CAUSAL)
    d.flags = _lib.FLAG_DENSE
    d.kk = 3
    assert lib.fbsa_fwd(d, DUMMY, DUMMY, DUMMY, None, None, None, DUMMY, None, None) == _lib.EINVAL
    assert "kk == nblk" in lib.fbsa_last_error().decode()
    d.kk, d.mask = 4, _lib.MASK_SLOT_CAUSAL
    assert lib.fbsa_fwd(d, DUMMY, DUMMY, DUMMY, None, None, None, DUMMY, None, None) == _lib.EINVAL
    assert "TOKEN_CAUSAL" in lib.fbsa_last_error().decode()
    d.mask = _lib.MASK_TOKEN_CAUSAL
    assert lib.fbsa_fwd(d, DUMMY, DUMMY, DUMMY, None, DUMMY, None, DUMMY, None, None) == _lib.EINVAL
    assert "gate" in lib.fbsa_last_error().decode()
    d.flags = 0   # a list-less call needs the dense flag
    assert lib.fbsa_fwd(d, DUMMY, DUMMY, DUMMY, None, None, None, DUMMY, None, None) == _lib.EINVAL
    assert "sel is NULL" in lib.fbsa_last_error().decode()
    # 1M tokens at block 64 (16384 blocks), 8 heads: the dense backward's workspace is
    # the row statistics plus the list offsets, no per-entry arrays
    big = _desc(mask=_lib.MASK_TOKEN_CAUSAL, Hq=8, Hkv=8, L=16384 * 64, nblk=16384, kk=16384, l_valid=16384 * 64)
    for s in ("sq", "sk", "sv", "so", "sdo", "sog"):
        getattr(big, s)[:] = (8 * 16384 * 64 * 64, 16384 * 64 * 64, 64)
    big.flags = _lib.FLAG_DENSE
    rows = 8 * 16384 * 64
    nbytes = lib.fbsa_bwd_workspace_bytes(big)
    assert rows * 8 <= nbytes <= rows * 8 + (16384 + 1) * 4 + 1024
    big.flags = 0   # the same shape as an explicit list would need nblk^2 sort entries: refused
    assert lib.fbsa_bwd_workspace_bytes(big) == 0


def test_bench_warm_up_runs_at_least_w_steps_then_until_the_time_floor(monkeypatch):
    """bench.warm_up: never fewer than W untimed steps; with a time floor it
    keeps stepping until that much time has passed, and reports the count."""
    import sys
    import time
    import torch
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    monkeypatch.setattr(torch.cuda, "synchronize", lambda: None)
    calls = []
    assert bench.warm_up(lambda: calls.append(1), 7, 0.0) == 7 and len(calls) == 7
    calls.clear()
    t0 = time.perf_counter()
    n = bench.warm_up(lambda: (calls.append(1), time.sleep(0.002)), 3, 0.05)
    assert time.perf_counter() - t0 >= 0.05 and n == len(calls) and n > 3


@pytest.mark.parametrize("dtype", ["BF16", "F32"])
def test_bwd_validates_before_launching(dtype):
    # bf16 without an output gate (row statistics formed in dQ, the index on a
    # second stream): fbsa_bwd checks the arguments of all four stages before it
    # launches anything, with the stages' own messages. fp32 runs the stages in
    # order, each checking its own arguments first: the prep stage's are checked
    # before any launch.
    lib = _lib.load()
    d = _desc()
    d.dtype = getattr(_lib, dtype)
    nbytes = lib.fbsa_bwd_workspace_bytes(d)
    assert nbytes > 0
    ws = 1 << 24  # 256-byte aligned, never dereferenced

    def call(n=nbytes, **kw):
        a = dict(q=DUMMY, k=DUMMY, v=DUMMY, o=DUMMY, dout=DUMMY, lse=DUMMY, sel=DUMMY, gate=None, og=None,
                 dq=DUMMY, dk=DUMMY, dv=DUMMY, dgate=None, dog=None)
        a.update(kw)
        return lib.fbsa_bwd(d, a["q"], a["k"], a["v"], a["o"], a["dout"], a["lse"], a["sel"], a["gate"], a["og"],
                            a["dq"], a["dk"], a["dv"], a["dgate"], a["dog"], ws, n, None)

    cases = [(dict(lse=None), "fbsa_bwd_prep: o/dout"), (dict(o=DUMMY + 4), "fbsa_bwd_prep: o/dout")]
    if dtype == "BF16":
        cases += [(dict(q=None), "fbsa_bwd_dq: null q/k/v"), (dict(dq=DUMMY + 2), "fbsa_bwd_dq: dq must"),
                  (dict(sel=DUMMY + 2), "sel/gate/dgate must be 4-byte aligned"),
                  (dict(dk=None), "fbsa_bwd_dkdv: dk/dv must"), (dict(dv=DUMMY + 8), "fbsa_bwd_dkdv: dk/dv must")]
    for kw, needle in cases:
        assert call(**kw) == _lib.EINVAL, kw
        assert needle in lib.fbsa_last_error().decode(), (kw, lib.fbsa_last_error().decode())
    assert call(n=nbytes - 256) == _lib.EWORKSPACE  # short of what the shape needs
