"""The offline CDNA4 decision LUT (include/leanstream/hip_kernel_lut.h) against the sweeps it
was synthesized from (profiles/kernel_lut_sweep_*.json, leanstream_amd/lut_sweep.py), and the
backend built with it selecting the measured winner for every (layer, io bucket)
(docs/kernel_selection.md: offline characterization -> offline table -> O(1) lookup)."""
import ctypes as C
import json
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from leanstream_amd import _native, lut_sweep

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "leanstream" / "hip_kernel_lut.h"
SWEEPS = sorted((ROOT / "profiles").glob("kernel_lut_sweep_*.json"))


def _header_rows():
    rows = {}
    for m in re.finditer(r"kLutD(\d+)G(\d+)\[8\] = \{([^}]*)\}", HEADER.read_text()):
        rows[(int(m.group(1)), int(m.group(2)))] = [int(v) for v in m.group(3).split(",")]
    return rows


def test_sweeps_cover_the_four_batch1_shapes():
    """C1/C3 (d 1024), C2 (d 4096), C4 (d 8192) and Group2 (d 4096, groups of 2)."""
    shapes = {(json.loads(p.read_text())["width"], json.loads(p.read_text())["group_size"]) for p in SWEEPS}
    assert {(1024, 64), (4096, 64), (8192, 64), (4096, 2)} <= shapes


def test_identical_launches_are_measured_once():
    """The plain-walk candidate is the default's launch where the shape walks plain already
    (d 8192), and the whole-tile candidate where the staged walk never takes quarters
    (d > 2048) or does not run (groups of 2)."""
    resident = 511
    _, first = lut_sweep.effective_configs(resident, 8192, 64)
    assert first[6] == 1 and first[7] == 1
    _, first = lut_sweep.effective_configs(resident, 4096, 64)
    assert first[6] == 6 and first[7] == 1
    _, first = lut_sweep.effective_configs(resident, 1024, 64)
    assert first[6] == 6 and first[7] == 7
    _, first = lut_sweep.effective_configs(resident, 4096, 2)
    assert first[6] == 6 and first[7] == 1
    assert first[4] == 4 and first[3] == 3   # split entry points stay launches of their own


@pytest.mark.parametrize("path", SWEEPS, ids=lambda p: p.stem)
def test_header_rows_are_the_measured_winners(path):
    r = json.loads(path.read_text())
    med = np.asarray(r["median_us"])
    assert med.shape == (lut_sweep.BUCKETS, len(lut_sweep.CANDIDATES))
    win = lut_sweep.winners(r)
    assert _header_rows()[(r["width"], r["group_size"])] == win
    for q, c in enumerate(win):
        # a winner is the fastest launch or within the tie margin of it
        assert med[q, c] <= med[q].min() * 1.02 + 1e-9, (q, c)
        # and every bucket was measured at a remaining load that quantizes to it
        assert lut_sweep.quantize_io_load(r["remaining"][q], r["active"]) == q


@pytest.mark.parametrize("path", SWEEPS, ids=lambda p: p.stem)
def test_backend_with_the_table_selects_the_winner(path):
    r = json.loads(path.read_text())
    row = _header_rows()[(r["width"], r["group_size"])]
    layers = 36
    lib = _native.library()
    table = (C.c_uint8 * (layers * 8))(*(row * layers))
    ctx = lib.ls_hip_create_table(table, layers, 8)
    try:
        for layer in (0, 17, 35):
            for q in range(8):
                assert lib.ls_hip_select(ctx, layer, q) == row[q]
        # remaining-load quantization feeding the lookup
        k = r["active"]
        for rem in range(k + 1):
            assert lib.ls_hip_select(ctx, 0, lib.ls_quantize_io_load(rem, k, 8)) == row[lut_sweep.quantize_io_load(rem, k)]
    finally:
        lib.ls_hip_destroy(ctx)


def test_header_compiles_and_fills_rows(tmp_path):
    src = tmp_path / "lut.cpp"
    src.write_text(r'''
#include "leanstream/hip_kernel_lut.h"
#include <cstdio>
int main() {
    using namespace leanstream::runtime;
    uint8_t storage[3 * cdna4::kLutBuckets];
    KernelDecisionTable t = cdna4::hip_lut_rows(cdna4::kLutD4096G64, 3, storage);
    for (uint32_t i = 0; i < t.layers * t.io_buckets; ++i) std::printf("%u ", t.entries[i]);
    return 0;
}
''')
    exe = tmp_path / "lut"
    subprocess.run(["g++", "-std=c++17", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True,
                   capture_output=True)
    out = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert out == _header_rows()[(4096, 64)] * 3
