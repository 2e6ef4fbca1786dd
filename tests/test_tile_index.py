"""The tile-layout decode kernels' address arithmetic, restated on the CPU.

qmv64_paired_kernel (fused gate_up + SwiGLU over gate/up-paired tile weights),
qmv64_tiled_kernel (row form) and down_pair_tiled_kernel (fused down + weighted
sum) must read, for every lane and row, the same 16 bytes of codes and the same
scale|bias word as their MLX-layout counterparts, and nothing outside the
arrays.  Each index formula below is the kernel's, term for term; the arrays
are built with the tile layout's documented permutation (include/qmoe.h,
qmoe_repack_tiles), independently of the device repack."""

import numpy as np
import pytest

from titan_amd import synth


def tile_layout(w, s, b):
    """wp[e][c][g][j][h][l][t] = w[e][64c + 32j + l][8g + 4h + t];
    sb[e][c][g][i] = s[e][64c + i][g] | b[e][64c + i][g] << 16."""
    E, N, KW = w.shape
    G = KW // 8
    wp = w.reshape(E, N // 64, 2, 32, G, 2, 4).transpose(0, 1, 4, 2, 5, 3, 6)
    sb = (s.astype(np.uint32) | (b.astype(np.uint32) << 16)).reshape(E, N // 64, 64, G).transpose(0, 1, 3, 2)
    return np.ascontiguousarray(wp).reshape(-1, 4), np.ascontiguousarray(sb).reshape(-1)


def pair_rows(I):
    """Paired row order: row 64c + j is gate row 32c + j (j < 32) or up row I + 32c + j - 32."""
    t = np.arange(2 * I)
    c, j = t // 64, t % 64
    return np.where(j < 32, 32 * c + j, I + 32 * c + j - 32)


def xcd_item(b, nb):
    return b if nb % 8 else (b % 8) * (nb // 8) + b // 8


@pytest.mark.parametrize("K,I,E,RG", [(2048, 512, 4, 8), (4096, 96, 3, 8), (6144, 64, 2, 4), (8192, 32, 2, 4)])
def test_paired_gate_up_reads_the_mlx_words(K, I, E, RG):
    rng = np.random.default_rng(K + I)
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K)
    perm = pair_rows(I)
    wp, sb = tile_layout(w[:, perm], s[:, perm], b[:, perm])
    NV, G, NC = K // 2048, K // 64, 2 * I // 64
    n_pairs = 3
    nblk = I // RG
    nb = n_pairs * nblk
    seen_items = set()
    idx = rng.integers(0, E, size=n_pairs)
    for blk in range(nb):
        item = xcd_item(blk, nb)
        seen_items.add(item)
        r, i0 = item // nblk, (item % nblk) * RG
        e = int(idx[r])
        c, l0 = i0 >> 5, i0 & 31
        for lane in range(64):
            h = lane & 1
            chunk0 = (e * NC + c) * G + (lane >> 1)
            for v in range(NV):
                for t in range(RG // 4):
                    base = (chunk0 + v * 32) * 64 + l0 + 4 * t
                    assert base + 32 + 3 < sb.size
                    for k in range(4):
                        i = i0 + 4 * t + k
                        gi = v * 32 + lane // 2  # the MLX kernel's group for this lane
                        assert sb[base + k] == (int(s[e, i, gi]) | int(b[e, i, gi]) << 16)
                        assert sb[base + 32 + k] == (int(s[e, I + i, gi]) | int(b[e, I + i, gi]) << 16)
                for q in range(RG):
                    unit = ((chunk0 + v * 32) * 4 + h) * 32 + l0 + q
                    assert unit + 64 < wp.shape[0]
                    word0 = v * 256 + 4 * lane  # the MLX kernel's 16 bytes: words 4 lane .. of chunk v
                    assert np.array_equal(wp[unit], w[e, i0 + q, word0:word0 + 4])
                    assert np.array_equal(wp[unit + 64], w[e, I + i0 + q, word0:word0 + 4])
    assert seen_items == set(range(nb))


@pytest.mark.parametrize("K,N,E", [(2048, 4096, 1), (4096, 192, 3)])
def test_tiled_row_form_reads_the_mlx_words(K, N, E):
    rng = np.random.default_rng(K + N)
    w, s, b = synth.quant_weights(rng, (E, N), K)
    wp, sb = tile_layout(w, s, b)
    NV, G, NC = K // 2048, K // 64, N // 64
    nblk = (N + 7) // 8
    n_pairs = 2
    nb = n_pairs * nblk
    ex = rng.integers(0, E, size=n_pairs)
    for blk in range(nb):
        item = xcd_item(blk, nb)
        r, n0 = item // nblk, (item % nblk) * 8
        e = int(ex[r])
        nq = min(n0, N - 8)
        for lane in range(0, 64, 5):
            h = lane & 1
            for v in range(NV):
                g = v * 32 + (lane >> 1)
                for u in range(2):
                    chunk = (e * NC + nq // 64) * G + g
                    for k in range(4):
                        n = nq + 4 * u + k
                        assert sb[chunk * 64 + (nq & 63) + 4 * u + k] == (int(s[e, n, g]) | int(b[e, n, g]) << 16)
                for q in range(8):
                    n = nq + q
                    unit = ((((e * NC + n // 64) * G + g) * 2 + ((n & 63) >> 5)) * 2 + h) * 32 + (n & 31)
                    word0 = v * 256 + 4 * lane
                    assert np.array_equal(wp[unit], w[e, n, word0:word0 + 4])


@pytest.mark.parametrize("R", [8, 16])
def test_tiled_down_reads_the_mlx_words(R):
    """down_pair_tiled_kernel: lane (rg, l) reads unit (g = l / 2, h = l % 2) of
    rows d0 + 4i + rg -- the 16 bytes its MLX-layout counterpart reads."""
    rng = np.random.default_rng(R)
    E, D, I = 3, 256, 512
    w, s, b = synth.quant_weights(rng, (E, D), I)
    wp, sb = tile_layout(w, s, b)
    NCd = D // 64
    for d0 in range(0, D, R):
        for e in range(E):
            for lane in range(64):
                rg, l = lane >> 4, lane & 15
                g, h = l >> 1, l & 1
                for i in range(R // 4):
                    row = min(d0 + 4 * i + rg, D - 1)
                    chunk = (e * NCd + (row >> 6)) * 8 + g
                    unit = ((chunk * 2 + ((row >> 5) & 1)) * 2 + h) * 32 + (row & 31)
                    assert unit < wp.shape[0] and chunk * 64 + (row & 63) < sb.size
                    # the MLX kernel: 16 bytes at word 4 l of the row, scale/bias of group (32 l) / 64
                    assert np.array_equal(wp[unit], w[e, row, 4 * l:4 * l + 4])
                    gi = (l * 32) // 64
                    assert sb[chunk * 64 + (row & 63)] == (int(s[e, row, gi]) | int(b[e, row, gi]) << 16)


@pytest.mark.parametrize("K,I,E,RG", [(2048, 512, 4, 8), (4096, 96, 3, 8), (6144, 64, 2, 4), (8192, 32, 2, 4)])
def test_paired_gate_up_reads_the_mlx_words(K, I, E, RG):
    rng = np.random.default_rng(K + I)
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K)
    perm = pair_rows(I)
    wp, sb = tile_layout(w[:, perm], s[:, perm], b[:, perm])
    NV, G, NC = K // 2048, K // 64, 2 * I // 64
    n_pairs = 3
    nblk = I // RG
    nb = n_pairs * nblk
    seen_items = set()
    idx = rng.integers(0, E, size=n_pairs)
    for blk in range(nb):
        item = xcd_item(blk, nb)
        seen_items.add(item)
        r, i0 = item // nblk, (item % nblk) * RG
        e = int(idx[r])
        c, l0 = i0 >> 5, i0 & 31
        for lane in range(64):
            h = lane & 1
            chunk0 = (e * NC + c) * G + (lane >> 1)
            for v in range(NV):
                for t in range(RG // 4):
                    base = (chunk0 + v * 32) * 64 + l0 + 4 * t
                    assert base + 32 + 3 < sb.size
                    for k in range(4):
                        i = i0 + 4 * t + k
                        gi = v * 32 + lane // 2  # the MLX kernel's group for this lane
                        assert sb[base + k] == (int(s[e, i, gi]) | int(b[e, i, gi]) << 16)
                        assert sb[base + 32 + k] == (int(s[e, I + i, gi]) | int(b[e, I + i, gi]) << 16)
                for q in range(RG):
                    unit = ((chunk0 + v * 32) * 4 + h) * 32 + l0 + q
                    assert unit + 64 < wp.shape[0]
                    word0 = v * 256 + 4 * lane  # the MLX kernel's 16 bytes: words 4 lane .. of chunk v
                    assert np.array_equal(wp[unit], w[e, i0 + q, word0:word0 + 4])
                    assert np.array_equal(wp[unit + 64], w[e, I + i0 + q, word0:word0 + 4])
    assert seen_items == set(range(nb))


@pytest.mark.parametrize("K,N,E", [(2048, 4096, 1), (4096, 192, 3)])
def test_tiled_row_form_reads_the_mlx_words(K, N, E):
    rng = np.random.default_rng(K + N)
    w, s, b = synth.quant_weights(rng, (E, N), K)
    wp, sb = tile_layout(w, s, b)
    NV, G, NC = K // 2048, K // 64, N // 64
    nblk = (N + 7) // 8
    n_pairs = 2
    nb = n_pairs * nblk
    ex = rng.integers(0, E, size=n_pairs)
    for blk in range(nb):
        item = xcd_item(blk, nb)
        r, n0 = item // nblk, (item % nblk) * 8
        e = int(ex[r])
        nq = min(n0, N - 8)
        for lane in range(0, 64, 5):
            h = lane & 1
            for v in range(NV):
                g = v * 32 + (lane >> 1)
                for u in range(2):
                    chunk = (e * NC + nq // 64) * G + g
                    for k in range(4):
                        n = nq + 4 * u + k
                        assert sb[chunk * 64 + (nq & 63) + 4 * u + k] == (int(s[e, n, g]) | int(b[e, n, g]) << 16)
                for q in range(8):
                    n = nq + q
                    unit = ((((e * NC + n // 64) * G + g) * 2 + ((n & 63) >> 5)) * 2 + h) * 32 + (n & 31)
                    word0 = v * 256 + 4 * lane
                    assert np.array_equal(wp[unit], w[e, n, word0:word0 + 4])


@pytest.mark.parametrize("R", [8, 16])
def test_tiled_down_reads_the_mlx_words(R):
    """down_pair_tiled_kernel: lane 8r + q, 8-row group m, chunk slot u: unit
    (gh = q + 8u, row d0 + 8m + r) holds the row's codes of h chunk gh."""
    rng = np.random.default_rng(R)
    E, D, I = 3, 256, 512
    w, s, b = synth.quant_weights(rng, (E, D), I)
    wp, sb = tile_layout(w, s, b)
    NCd = D // 64
    for d0 in range(0, D, R):
        for e in range(E):
            rows_seen = set()
            for lane in range(64):
                r, q = lane >> 3, lane & 7
                for m in range(R // 8):
                    row = d0 + 8 * m + r
                    assert row < D
                    rows_seen.add(row)
                    for u in range(2):
                        gh = q + 8 * u
                        chunk = (e * NCd + (row >> 6)) * 8 + (gh >> 1)
                        unit = ((chunk * 2 + ((row >> 5) & 1)) * 2 + (gh & 1)) * 32 + (row & 31)
                        assert unit < wp.shape[0] and chunk * 64 + (row & 63) < sb.size
                        assert np.array_equal(wp[unit], w[e, row, 4 * gh:4 * gh + 4])
                        g = gh >> 1
                        assert sb[chunk * 64 + (row & 63)] == (int(s[e, row, g]) | int(b[e, row, g]) << 16)
            assert rows_seen == set(range(d0, d0 + R))


@pytest.mark.parametrize("K,I,E,RG", [(2048, 512, 3, 8), (4096, 64, 2, 8), (2048, 96, 2, 4), (4096, 32, 2, 4)])
def test_paired_lines_kernel_reads_the_mlx_words(K, I, E, RG):
    """qmv64_paired_lines_kernel: lane 8r + s, step p, half h, j: unit
    (g = 8p + s, j, h, l0 + r) -- the row's 32 codes of group g, half h -- and
    the matching x chunk 2g + h and scale|bias word 32j + l0 + r."""
    rng = np.random.default_rng(K * 3 + I)
    w, s, b = synth.quant_weights(rng, (E, 2 * I), K)
    perm = pair_rows(I)
    wp, sb = tile_layout(w[:, perm], s[:, perm], b[:, perm])
    NV, G, NC = K // 2048, K // 64, 2 * I // 64
    nblk = I // RG
    n_pairs = 2
    nb = n_pairs * nblk
    ex = rng.integers(0, E, size=n_pairs)
    covered = np.zeros((n_pairs, I, 2), bool)
    for blk in range(nb):
        item = xcd_item(blk, nb)
        pr, i0 = item // nblk, (item % nblk) * RG
        e = int(ex[pr])
        c, l0 = i0 >> 5, i0 & 31
        cbase = (e * NC + c) * G
        for lane in range(64):
            r, sl = lane >> 3, lane & 7
            jr, rr = (0, r) if RG == 8 else (r >> 2, r & 3)
            halves = (0, 1) if RG == 8 else (jr,)
            for pp in range(4 * NV):
                g = 8 * pp + sl
                chunk = cbase + g
                for j in halves:
                    row = i0 + rr + I * j
                    covered[pr, i0 + rr, j] = True
                    word = int(sb[chunk * 64 + l0 + rr + 32 * j])
                    assert word == (int(s[e, row, g]) | int(b[e, row, g]) << 16)
                    for h in range(2):
                        unit = ((chunk * 2 + j) * 2 + h) * 32 + l0 + rr
                        assert unit < wp.shape[0]
                        ch = 2 * g + h  # x chunk: elements 32 ch .. 32 ch + 31
                        assert np.array_equal(wp[unit], w[e, row, 4 * ch:4 * ch + 4])
    assert covered.all()
