"""Host-side address model of the one-token decode gate_up kernel.

``qmv64_flat_kernel`` (titan_amd/csrc/qmv.hip) runs kFlatWaves waves per
workgroup.  These tests restate its address arithmetic in numpy for every
(block, wave, lane) of a launch and check each access against the extent of
the buffer it touches, at the workload shapes and at ragged edges:

* the shipped indexing (lane = threadIdx.x % 64, item = xcd_item(block) * W +
  wave, LDS staging per wave, waves past the list leave) stays in bounds;
* the single-wave indexing it replaced (lane = threadIdx.x, item =
  xcd_item(block), one wave's LDS) does not once a workgroup holds more than
  64 threads: lanes 64.. read x and the weight tensor past their ends (lane
  l reads x from element 32 l and 16 bytes at byte 16 l of each weight row:
  at workload 1's shape up to 12 KiB past x and 3 KiB past the last row).  That is the out-of-bounds access a 2- or 4-wave launch of the
  single-wave kernel makes.

``qmv64_paired_lines_kernel`` (the tile-layout gate_up the one-copy MoE block
decodes with) is modelled the same way: every access in bounds and every
output index stored once, at the block's shapes and ragged ones.

The reference's rule (a bounds test at the largest real shape before a kernel
is enabled, docs/ops/INCIDENTS.md:29) is what this model gives on the CPU.
"""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

SRC = Path(__file__).resolve().parents[1] / "titan_amd" / "csrc" / "qmv.hip"


def _const(name: str) -> int:
    m = re.search(rf"constexpr int {name} = (\d+);", SRC.read_text())
    assert m, f"{name} not found in {SRC}"
    return int(m.group(1))


FLAT_RG = _const("kFlatRG")
FLAT_WAVES = _const("kFlatWaves")
U32 = np.uint64(0xFFFFFFFF)


def xcd_item(b: np.ndarray, nb: int) -> np.ndarray:
    """xcd_item(b, nb) of qmv.hip: XCD-contiguous permutation when 8 | nb."""
    if nb % 8:
        return b
    return (b % 8) * (nb // 8) + b // 8


def flat_accesses(E, k, n_out, NV, GS, W, threads, legacy=False):
    """Byte ranges [lo, hi) each buffer sees from one launch of the flat kernel.

    W waves per workgroup as compiled; ``threads`` per workgroup as launched.
    legacy: the single-wave indexing (lane = threadIdx.x, item = block)."""
    n_w = 2 * n_out
    KE = 2048 * NV
    G = KE // GS
    UPR = G // 8
    UNITS = 4 * FLAT_RG * UPR
    UPL = (UNITS + 63) // 64
    KW = KE // 8
    total = k * n_out
    nitems = (total + FLAT_RG - 1) // FLAT_RG
    if legacy:
        blocks = nitems // W  # the same waves in W-wave workgroups
    else:
        blocks = (nitems + W - 1) // W
    b = np.repeat(np.arange(blocks, dtype=np.int64), threads)
    t = np.tile(np.arange(threads, dtype=np.int64), blocks)
    if legacy:
        lane = t
        wave = np.zeros_like(t)
        item = xcd_item(b, nitems)
    else:
        lane = t % 64
        wave = t // 64
        item = xcd_item(b, (nitems + W - 1) // W) * W + wave
    live = item < nitems
    b, lane, wave, item = b[live], lane[live], wave[live], item[live]
    ids = (E - 1 - 7 * np.arange(k, dtype=np.int64)) % E  # in range, the last expert first
    f0 = item * FLAT_RG
    flast = np.minimum(f0 + FLAT_RG - 1, total - 1)
    ra, rb = f0 // n_out, flast // n_out
    acc = {"experts": [], "x": [], "w": [], "sb": [], "lds": [], "out": []}
    acc["experts"] += [(ra * 4, ra * 4 + 4), (rb * 4, rb * 4 + 4)]
    ea = ids[np.minimum(ra, k - 1)]  # the model reads in-range ids; the ranges above are checked
    eb = ids[np.minimum(rb, k - 1)]
    for v in range(NV):
        lo = (v * 2048 + lane * 32) * 2
        acc["x"].append((lo, lo + 64))
    fb = (ra + 1) * n_out
    sp = fb - f0
    smax = total - 1 - f0
    row_a = (ea * n_w + f0 - (fb - n_out)).astype(np.uint64) & U32
    row_b = (eb * n_w + f0 - fb).astype(np.uint64) & U32

    def slot_row(s, g, sel=slice(None)):
        """Weight row of slot s (gate g = 0, up g = 1) for the lanes sel."""
        se = np.minimum(s, smax[sel]).astype(np.uint64)
        base = np.where(se < sp[sel].astype(np.uint64), row_a[sel], row_b[sel])
        return ((base + se + np.uint64(n_out if g else 0)) & U32).astype(np.int64)

    for g in range(2):
        for s in range(FLAT_RG):
            row = slot_row(s, g)
            for v in range(NV):
                lo = row * KW * 4 + lane * 16 + v * 1024
                acc["w"].append((lo, lo + 16))
    for j in range(UPL):
        u = lane + 64 * j
        idx = np.nonzero(u < UNITS if UNITS % 64 else np.ones_like(u, dtype=bool))[0]
        uu = u[idx]
        seg, up = uu // UPR, uu % UPR  # seg = (slot * 2 + gate/up) * 2 + scale/bias
        rows = np.empty_like(uu)
        for sg in np.unique(seg):
            pick = seg == sg
            rows[pick] = slot_row(int(sg) >> 2, (int(sg) >> 1) & 1, idx[pick])
        lo = rows * G * 2 + up * 16
        acc["sb"].append((lo, lo + 16))
        lds = wave[idx] * UNITS * 16 + uu * 16
        acc["lds"].append((lds, lds + 16))
    q = lane >> 3
    st4 = lane == 1
    f = f0 + np.where(st4, 4, q)
    m = (lane < 32) & (((lane & 7) == 0) | st4) & (f < total)
    acc["out"].append((f[m] * 2, f[m] * 2 + 2))
    ext = {"experts": k * 4, "x": KE * 2, "w": E * n_w * KW * 4, "sb": E * n_w * G * 2,
           "lds": W * UNITS * 16, "out": total * 2}
    return acc, ext


def overruns(acc, ext):
    """Per buffer: how many bytes the accesses reach past the end (<= 0 in bounds),
    and whether any starts below zero."""
    res = {}
    for name, ranges in acc.items():
        if not ranges:
            continue
        lo = min(int(r[0].min()) for r in ranges if r[0].size)
        hi = max(int(r[1].max()) for r in ranges if r[1].size)
        res[name] = (lo, hi - ext[name])
    return res


SHAPES = [
    # E, top_k, I (n_out), NV, group size: workload 1, other group sizes and K,
    # a ragged list (10 * 509 slots, not a multiple of 5 * W) and few experts
    (256, 10, 512, 1, 64),
    (256, 10, 512, 1, 32),
    (256, 10, 512, 1, 128),
    (256, 9, 512, 2, 64),
    (512, 10, 512, 4, 128),
    (256, 10, 509, 1, 64),
    (4, 3, 7, 1, 64),
]


@pytest.mark.parametrize("E,k,n_out,NV,GS", SHAPES)
def test_flat_kernel_accesses_in_bounds(E, k, n_out, NV, GS):
    acc, ext = flat_accesses(E, k, n_out, NV, GS, FLAT_WAVES, 64 * FLAT_WAVES)
    for name, (lo, over) in overruns(acc, ext).items():
        assert lo >= 0, (name, lo)
        assert over <= 0, (name, over)


@pytest.mark.parametrize("E,k,n_out,NV,GS", SHAPES)
def test_flat_kernel_covers_every_slot_once(E, k, n_out, NV, GS):
    acc, ext = flat_accesses(E, k, n_out, NV, GS, FLAT_WAVES, 64 * FLAT_WAVES)
    stores = np.concatenate([r[0] for r in acc["out"]]) // 2
    assert np.array_equal(np.sort(stores), np.arange(k * n_out))


@pytest.mark.parametrize("W", [2, 4])
def test_single_wave_indexing_overruns_in_wider_workgroups(W):
    """The single-wave kernel's indexing under a 64 * W-thread launch: lanes
    64.. read past x and past the last weight row (the accesses a multi-wave
    launch of the unchanged kernel makes; its scale staging is guarded by
    u < UNITS, so it stays in bounds)."""
    acc, ext = flat_accesses(256, 10, 512, 1, 64, 1, 64 * W, legacy=True)
    over = overruns(acc, ext)
    assert over["x"][1] == (64 * W - 64) * 64  # lane 64W - 1 reads x elements up to 2048 W
    assert over["w"][1] == (64 * W - 64) * 16  # and weight bytes up to 16 * 64W into the last row
    # the same indexing at 64 threads (as the kernel was written) stays in bounds
    acc1, ext1 = flat_accesses(256, 10, 512, 1, 64, 1, 64, legacy=True)
    assert all(o <= 0 and lo >= 0 for lo, o in overruns(acc1, ext1).values())


PAIRED_RG = int(re.search(r"#define QMOE_PAIRED_LINES_RG (\d+)", SRC.read_text()).group(1))


def paired_lines_accesses(E, T, k, n_out, NV, W=1, RG=None):
    """Byte ranges each buffer sees from one launch of qmv64_paired_lines_kernel
    (tile-layout gate_up + SwiGLU, the form that takes expert ids): one 64-lane
    wave per workgroup, item = xcd_item(block, grid), as launch_qmv_paired
    sizes the grid.  (W > 1 models W waves per workgroup, item =
    xcd_item(block) * W + wave, with per-wave LDS staging and waves past the
    last item leaving.)"""
    RG = RG or PAIRED_RG
    NCH, NP, NJ = 64 * NV, 4 * NV, RG // 4
    K = 2048 * NV
    G = 32 * NV
    n_w = 2 * n_out
    NC = n_w // 64
    n_pairs = T * k
    nblk = n_out // RG
    nitems = n_pairs * nblk
    blocks = (nitems + W - 1) // W
    threads = 64 * W
    b = np.repeat(np.arange(blocks, dtype=np.int64), threads)
    t = np.tile(np.arange(threads, dtype=np.int64), blocks)
    lane, wave = t % 64, t // 64
    item = xcd_item(b, blocks) * W + wave if W > 1 else xcd_item(b, blocks)
    live = item < nitems
    lane, wave, item = lane[live], wave[live], item[live]
    r, sl = lane >> 3, lane & 7
    jr = np.zeros_like(r) if RG == 8 else r >> 2
    rr = r if RG == 8 else r & 3
    pr = item // nblk
    i0 = (item - pr * nblk) * RG
    xr = pr // k
    ids = (E - 1 - 7 * np.arange(n_pairs, dtype=np.int64)) % E
    e = ids[pr]
    c, l0 = i0 >> 5, i0 & 31
    cbase = (e * NC + c) * G
    acc = {"experts": [(pr * 4, pr * 4 + 4)], "x": [], "w": [], "sb": [], "lds": [], "out": []}
    for v in range(NV):
        lo = (xr * K + v * 2048 + lane * 32) * 2
        acc["x"].append((lo, lo + 64))
        for q in range(4):
            lds = ((wave * 4 + q) * NCH + v * 64 + lane) * 16
            acc["lds"].append((lds, lds + 16))
    for pp in range(NP):
        chunk = cbase + 8 * pp + sl
        for jj in range(NJ):
            wd = chunk * 64 + l0 + rr + 32 * (jr + jj)
            acc["sb"].append((wd * 4, wd * 4 + 4))
            for h in range(2):
                u = ((chunk * 2 + jr + jj) * 2 + h) * 32 + l0 + rr
                acc["w"].append((u * 16, u * 16 + 16))
    m = (sl == 0) & (r < RG)
    o = pr[m] * n_out + i0[m] + r[m]
    acc["out"].append((o * 2, o * 2 + 2))
    ext = {"experts": n_pairs * 4, "x": T * K * 2, "w": E * n_w * K // 2, "sb": E * NC * G * 64 * 4,
           "lds": W * 4 * NCH * 16, "out": n_pairs * n_out * 2}
    return acc, ext


PAIRED_SHAPES = [
    # E, tokens, top_k, I, NV: workload 1's block shape, two tokens, K = 4096,
    # an item count that is not a multiple of W, and few experts
    (256, 1, 10, 512, 1),
    (256, 2, 10, 512, 1),
    (256, 1, 8, 512, 2),
    (64, 3, 7, 96, 1),
    (4, 1, 3, 32, 1),
]


@pytest.mark.parametrize("E,T,k,n_out,NV", PAIRED_SHAPES)
def test_paired_lines_kernel_accesses_in_bounds(E, T, k, n_out, NV):
    acc, ext = paired_lines_accesses(E, T, k, n_out, NV)
    for name, (lo, over) in overruns(acc, ext).items():
        assert lo >= 0, (name, lo)
        assert over <= 0, (name, over)


@pytest.mark.parametrize("E,T,k,n_out,NV", PAIRED_SHAPES)
def test_paired_lines_kernel_covers_every_output_once(E, T, k, n_out, NV):
    acc, _ = paired_lines_accesses(E, T, k, n_out, NV)
    stores = np.concatenate([r[0] for r in acc["out"]]) // 2
    assert np.array_equal(np.sort(stores), np.arange(T * k * n_out))
