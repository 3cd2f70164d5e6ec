"""The LDS chunk swizzle (``swz`` in csrc/fbsa_common.h) keeps every tile access
of the kernels on distinct banks, under gfx950's LDS pass structure as measured
with the bank-conflict counters (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE):

* 64 banks of 4 bytes;
* ds_read_b128: 4 passes of 16 lanes; lanes l, l' share a pass iff they agree
  in lane bit 5 and in the parity of lane bits 2..4;
* ds_read_b64_tr_b16: 2 passes (lanes 0-31, 32-63);
* 4-byte reads: one pass.

The swizzle table is printed by a host program compiled against the header, so
the test follows the kernels' own definition."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "fused-block-sparse-attention_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"

PROG = r"""
#include <stdio.h>
#include "fbsa_common.h"
int main() {
  const int cprs[4] = {4, 8, 16, 32};
  for (int c = 0; c < 4; ++c)
    for (int r = 0; r < 64; ++r) printf("%d %d %d\n", cprs[c], r, fbsa::swz(r, cprs[c]));
  return 0;
}
"""


@pytest.fixture(scope="module")
def table(tmp_path_factory):
    if not os.path.exists(HIPCC) or shutil.which("g++") is None:
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("swz")
    src, exe = d / "swz.cpp", d / "swz"
    src.write_text(PROG)
    subprocess.run([HIPCC, "-x", "hip", "--offload-arch=gfx950", "-std=c++17", "-I" + CSRC,
                    "-I" + os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True,
                   capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    t = {}
    for line in out.split("\n"):
        if line.strip():
            c, r, s = map(int, line.split())
            t[(c, r)] = s
    return t


def _passes_b128():
    groups = {}
    for l in range(64):
        groups.setdefault((bin(l & 0b011100).count("1") & 1, l >> 5), []).append(l)
    return list(groups.values())


def _cycles(addr, groups, nbytes):
    """Passes needed: per group, the most lanes landing on one bank."""
    tot = 0
    for grp in groups:
        cnt = {}
        for l in grp:
            for w in range(addr[l] // 4, (addr[l] + nbytes) // 4):
                cnt[w % 64] = cnt.get(w % 64, 0) + 1
        tot += max(cnt.values())
    return tot


@pytest.mark.parametrize("cpr", [4, 8, 16, 32])
def test_swizzle_bank_conflict_free(table, cpr):
    sw = lambda r: table[(cpr, r % 64)]  # noqa: E731
    for r in range(64):
        assert 0 <= sw(r) < cpr, "swizzle must permute chunks within the row"
    # (a) MFMA operand loads: lane (g, p) reads row 16m + p, chunk 4ks + g (b128)
    for m in range(4):
        for ks in range(cpr // 4):
            addr = {l: ((16 * m + (l & 15)) * cpr + ((4 * ks + (l >> 4)) ^ sw(16 * m + (l & 15)))) * 16
                    for l in range(64)}
            assert _cycles(addr, _passes_b128(), 16) == 4, (m, ks)
    # (b) transposing loads: rows 32k2 + 4g + p/4 (+16), chunks 2mt + (p&3)/2, half p&1
    for mt in range(cpr // 2):
        for k2 in range(2):
            for hi in (0, 16):
                addr = {}
                for l in range(64):
                    g, p = l >> 4, l & 15
                    ra = 32 * k2 + 4 * g + (p >> 2) + hi
                    addr[l] = (ra * cpr + ((2 * mt + ((p & 3) >> 1)) ^ sw(ra))) * 16 + (p & 1) * 8
                assert _cycles(addr, [range(32), range(32, 64)], 8) == 2, (mt, k2, hi)
    if cpr >= 16:
        # (c) fp32 operand loads: 16 rows x 4 B of one chunk; 4 rows x 4 chunks
        for m in range(2):
            for ks in range(cpr):
                addr = {l: ((16 * m + (l & 15)) * cpr + (ks ^ sw(16 * m + (l & 15)))) * 16 + (l >> 4) * 4
                        for l in range(64)}
                assert _cycles(addr, [range(64)], 4) == 1
            for t in range(cpr // 4):
                for r in range(4):
                    addr = {l: ((16 * m + 4 * (l >> 4) + r) * cpr + ((4 * t + ((l & 15) >> 2)) ^
                                                                   sw(16 * m + 4 * (l >> 4) + r))) * 16
                            + (l & 3) * 4 for l in range(64)}
                    assert _cycles(addr, [range(64)], 4) == 1


def test_pass_model_rejects_the_unswizzled_layout(table):
    # the model itself: an unswizzled MFMA operand load is 8-way conflicted
    # (32 passes measured), so the checks above are not vacuous
    cpr = 32
    addr = {l: ((l & 15) * cpr + (l >> 4)) * 16 for l in range(64)}
    assert _cycles(addr, _passes_b128(), 16) == 32
