"""CPU model of the int8 DMA kernel's buffer addressing (no GPU needed).

gemm_i8_dma_kernel and gemm_i8_h128_kernel (mind_amd/csrc/det_gemm_i8.hip)
move operand chunks
global -> LDS with buffer_load_dwordx4 ... lds.  The buffer unit's range
check covers the per-lane voffset only; the full-tile loops advance K through the
SGPR soffset, so every (voffset + soffset) it issues, including the steps it
issues past the end of K, must lie inside the operand.  The edge-tile loop
expresses out-of-range chunks as voffset = OOB_OFFSET (range-checked, a zero
fill) and must keep every other chunk inside.  This test restates the lane ->
chunk assignment and the issue schedule of both loops and checks every
address they can form, for the shapes the library routes to each loop.
"""
import numpy as np
import pytest

BM = BN = 256
BK = 64
NSTAGE = 4
OOB = 0x80000000


def _lane_chunks():
    """Per (wave, j, lane): A row / k-chunk and B k-row / n-chunk of the
    wave's DMA share (the inverse of the LDS swizzles)."""
    wave = np.arange(8)[:, None, None]
    j = np.arange(2)[None, :, None]
    lane = np.arange(64)[None, None, :]
    slot = 64 * (2 * wave + j) + lane
    ar = slot >> 2
    ac = (slot & 3) ^ ((ar >> 2) & 3)
    br = slot >> 4
    bc = (slot & 15) ^ ((br & 7) << 1)
    return ar.ravel(), 16 * ac.ravel(), br.ravel(), 16 * bc.ravel()


def _issued_steps(K):
    nk = (K + BK - 1) // BK
    # prologue: steps 0..2; MEM(s) for s = 0..nk-1 issues step s + 3
    return np.arange(0, nk + NSTAGE - 1) * BK


def _full_addresses(M, N, K):
    ar, akc, br, bnc = _lane_chunks()
    lim_a, lim_b = M * K, K * N
    lo_a = hi_a = lo_b = hi_b = None
    for m0 in range(0, M, BM):
        a_off = (m0 + ar) * K + akc
        for n0 in range(0, N, BN):
            b_off = br * N + n0 + bnc
            for k0 in _issued_steps(K):
                sa = k0 if k0 < K else K - BK
                sb = k0 * N if k0 < K else (K - BK) * N
                va, vb = a_off + sa, b_off + sb
                lo_a = va.min() if lo_a is None else min(lo_a, va.min())
                hi_a = va.max() if hi_a is None else max(hi_a, va.max())
                lo_b = vb.min() if lo_b is None else min(lo_b, vb.min())
                hi_b = vb.max() if hi_b is None else max(hi_b, vb.max())
    return (lo_a, hi_a + 16, lim_a), (lo_b, hi_b + 16, lim_b)


def _edge_addresses(M, N, K):
    ar, akc, br, bnc = _lane_chunks()
    worst = []
    for m0 in range(0, M, BM):
        for n0 in range(0, N, BN):
            a_ok = m0 + ar < M
            b_ok = n0 + bnc < N
            for k0 in _issued_steps(K):
                oka = a_ok & (k0 + akc < K)
                okb = b_ok & (k0 + br < K)
                va = np.where(oka, (m0 + ar) * K + akc + k0, OOB)
                vb = np.where(okb, (br + k0) * N + n0 + bnc, OOB)
                for v, ok, lim in ((va, oka, M * K), (vb, okb, K * N)):
                    inside = v[ok]
                    if inside.size:
                        worst.append(inside.max() + 16 - lim)
                    # every chunk flagged outside must be the range-checked OOB offset
                    assert np.all(v[~ok] == OOB)
    return max(worst) if worst else -1


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (512, 256, 1024), (256, 768, 512), (1024, 1024, 2048),
                                   (4096, 4096, 4096), (256, 256, 8192)])
def test_full_tile_dma_stays_inside_operands(M, N, K):
    assert M % BM == 0 and N % BN == 0 and K % (BK * NSTAGE) == 0 and K > 0
    (lo_a, end_a, lim_a), (lo_b, end_b, lim_b) = _full_addresses(M, N, K)
    assert lo_a >= 0 and end_a <= lim_a, (end_a, lim_a)
    assert lo_b >= 0 and end_b <= lim_b, (end_b, lim_b)


def test_full_tile_model_catches_the_old_past_end_offset():
    """The model is load-bearing: expressing a past-end step as soffset =
    operand size (the form the kernel used before) reads past A and B."""
    ar, akc, br, bnc = _lane_chunks()
    M = N = K = 256
    k0 = _issued_steps(K)[-1]
    assert k0 >= K
    assert ((ar * K + akc) + M * K).max() + 16 > M * K
    assert ((br * N + bnc) + K * N).max() + 16 > K * N


def _h128_addresses(M, N, K, tn=256):
    """gemm_i8_h128_kernel: 128-row tiles of width tn, K steps of 128 as two
    64-wide sub-stages, each wave one A block and tn / 128 B blocks per
    sub-stage; the prologue issues steps 0 and 1 (and 2 for the second wave
    group), the MFMA phase of step s issues step s + 2 (first group) or s + 3
    (second group), so steps up to nk + 2 are issued."""
    KS = 2 * BK
    nj = tn // 128
    wave = np.arange(8)[:, None]
    lane = np.arange(64)[None, :]
    slot = (64 * wave + lane).ravel()
    ar = slot >> 2
    akc = 16 * ((slot & 3) ^ ((ar >> 1) & 3))
    bslot = (64 * (nj * np.arange(8)[:, None, None] + np.arange(nj)[None, :, None])
             + np.arange(64)[None, None, :]).ravel()
    br, bc = _b_chunk(bslot, tn)
    bnc = 16 * bc
    assert ar.max() < 128 and br.max() < 64 and bnc.max() + 16 <= tn
    nk = K // KS
    lo = [None, None]
    hi = [None, None]
    for m0 in range(0, M, 128):
        a_off = (m0 + ar) * K + akc
        for n0 in range(0, N, tn):
            b_off = br * N + n0 + bnc
            for step in range(0, nk + 3):
                k0 = step * KS
                sa = k0 if k0 < K else K - KS
                sb = k0 * N if k0 < K else (K - KS) * N
                for u in range(2):
                    for i, v in enumerate((a_off + sa + u * BK, b_off + sb + u * BK * N)):
                        lo[i] = v.min() if lo[i] is None else min(lo[i], v.min())
                        hi[i] = v.max() if hi[i] is None else max(hi[i], v.max())
    return (lo[0], hi[0] + 16, M * K), (lo[1], hi[1] + 16, K * N)


@pytest.mark.parametrize("M,N,K,tn", [(128, 256, 128, 256), (4096, 4096, 4096, 256), (384, 512, 384, 256),
                                      (2048, 2048, 2048, 256), (128, 768, 1152, 256), (128, 128, 128, 128),
                                      (2048, 2048, 2048, 128), (384, 640, 1152, 128)])
def test_h128_tile_dma_stays_inside_operands(M, N, K, tn):
    assert M % 128 == 0 and N % tn == 0 and K % 128 == 0 and K > 0
    for lo, end, lim in _h128_addresses(M, N, K, tn):
        assert lo >= 0 and end <= lim, (end, lim)


@pytest.mark.parametrize("M,N,K", [(1, 16, 16), (100, 48, 80), (257, 272, 320), (300, 1008, 48), (256, 256, 64)])
def test_edge_tile_dma_stays_inside_operands(M, N, K):
    assert K % 16 == 0 and N % 16 == 0
    assert _edge_addresses(M, N, K) <= 0


def _pad_row_chunks(src, base, rows, cols, dcols):
    """pad_i8_kernel's reads for one operand, restated: returns the padded
    panel it writes and checks every load stays inside the source buffer.
    `src` is the buffer's bytes, `base` its address modulo 4."""
    total = rows * cols
    out = np.zeros((rows, dcols), np.uint8)
    for row in range(rows):
        for c0 in range(0, dcols, 16):
            if c0 >= cols:
                continue
            p = row * cols + c0
            at = base + p
            a = at & ~3
            if c0 + 16 <= cols and a >= base and a + 20 <= base + total:
                lo = a - base
                assert 0 <= lo and lo + 20 <= total
                v = src[lo:lo + 20].view("<u4").astype(np.uint64)
                sh = at & 3
                w = [int((((v[i + 1] << np.uint64(32)) | v[i]) >> np.uint64(8 * sh)) & np.uint64(0xFFFFFFFF))
                     for i in range(4)]
                out[row, c0:c0 + 16] = np.array(w, "<u4").view(np.uint8)
            else:
                nv = min(16, cols - c0)
                assert 0 <= p and p + nv <= total
                out[row, c0:c0 + nv] = src[p:p + nv]
    return out


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 17), (5, 33), (7, 4095), (2, 64), (4, 20)])
@pytest.mark.parametrize("base", [0, 1, 2, 3])
def test_pad_kernel_reads_stay_inside_and_assemble_the_rows(rows, cols, base):
    rng = np.random.default_rng(rows * 131 + cols + base)
    src = rng.integers(0, 256, rows * cols, dtype=np.uint8)
    dcols = (cols + 15) // 16 * 16
    got = _pad_row_chunks(src, base, rows, cols, dcols)
    want = np.zeros((rows, dcols), np.uint8)
    want[:, :cols] = src.reshape(rows, cols)
    np.testing.assert_array_equal(got, want)


def _cx(row, tn):
    """Chunk XOR of k-row `row` in a B sub-stage (Tile<TN>::cx)."""
    if tn == 256:
        return ((row & 7) << 1) ^ ((row >> 4) & 1)
    return (((row >> 1) & 3) << 1) ^ ((row >> 4) & 1)


def _b_chunk(slot, tn):
    """LDS slot (16-byte unit) of a B sub-stage -> (k-row, n-chunk) it holds
    (Tile<TN>::b_chunk)."""
    br = slot // (tn // 16)
    return br, (slot % (tn // 16)) ^ _cx(br, tn)


def _b_swz(row, chunk, tn):
    """Byte offset of (k-row, n-chunk) in a B sub-stage (Tile<TN>::swz)."""
    return row * tn + ((chunk ^ _cx(row, tn)) << 4)


@pytest.mark.parametrize("tn", [256, 128])
def test_h128_b_stage_layout_round_trips_and_reads_conflict_free(tn):
    """The B sub-stage of gemm_i8_h128_kernel<., ., TN>: the DMA places the
    global chunk b_chunk(slot) at slot (16 bytes per lane); the transposing
    reads (ds_read_b64_tr_b8: lane t of a 16-lane group gets byte t & 7 of
    the segments of lanes 2j + (t >> 3)) must hand lane l the 16x16x64 MFMA
    B operand B[16 (l >> 4) + 0..15][wn + 16 j + (l & 15)], and each
    half-wave must touch all 64 four-byte banks exactly once."""
    nj = tn // 64
    rng = np.random.default_rng(tn)
    tile = rng.integers(0, 256, size=(64, tn), dtype=np.uint8)   # one sub-stage: B[k][n]
    lds = np.zeros(64 * tn, np.uint8)
    written = np.zeros(64 * tn, bool)
    for slot in range(64 * tn // 16):
        br, bc = _b_chunk(slot, tn)
        assert 0 <= br < 64 and 0 <= bc < tn // 16
        assert _b_swz(br, bc, tn) == 16 * slot
        lds[16 * slot:16 * slot + 16] = tile[br, 16 * bc:16 * bc + 16]
        written[16 * slot:16 * slot + 16] = True
    assert written.all()
    lane = np.arange(64)
    tg, l16 = lane >> 4, lane & 15
    for wn in range(0, tn, tn // 4):
        for j in range(nj):
            got = np.zeros((64, 16), np.uint8)
            for half, dr in enumerate((0, 8)):
                r = 16 * tg + (l16 >> 1) + dr
                cb = (wn + 16 * j) >> 4
                addr = np.array([_b_swz(int(r[i]), cb, tn) for i in range(64)]) + 8 * (l16 & 1)
                for w in (slice(0, 32), slice(32, 64)):
                    banks = np.concatenate([(addr[w] // 4) % 64, (addr[w] // 4 + 1) % 64])
                    assert len(set(banks.tolist())) == 64
                for t in range(64):
                    g = 16 * (t >> 4)
                    for jj in range(8):
                        src = g + 2 * jj + ((t & 15) >> 3)
                        got[t, 8 * half + jj] = lds[addr[src] + (t & 7)]
            want = np.stack([tile[16 * (t >> 4):16 * (t >> 4) + 16, wn + 16 * j + (t & 15)] for t in range(64)])
            np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("rows", [128, 256])
def test_a_stage_layout_round_trips(rows):
    """A sub-stage [rows][64 k] of gemm_i8_h128_kernel (128 rows) and
    gemm_i8_t256_kernel (256 rows), chunk c of row r at c ^ ((r >> 1) & 3):
    the DMA lane -> chunk assignment (the inverse) fills every slot once, and
    the 16x16x64 operand read (lane l: row 16 i + (l & 15), chunk l >> 4)
    gets row r's chunk (l >> 4)."""
    rng = np.random.default_rng(7)
    tile = rng.integers(0, 256, size=(rows, 64), dtype=np.uint8)
    lds = np.zeros(rows * 64, np.uint8)
    seen = np.zeros(rows * 64 // 16, bool)
    for slot in range(rows * 64 // 16):
        ar = slot >> 2
        ac = (slot & 3) ^ ((ar >> 1) & 3)
        lds[16 * slot:16 * slot + 16] = tile[ar, 16 * ac:16 * ac + 16]
        seen[slot] = True
    assert seen.all()
    lane = np.arange(64)
    for i in range(rows // 16):
        row = 16 * i + (lane & 15)
        chunk = lane >> 4
        addr = row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4)
        for t in range(64):
            np.testing.assert_array_equal(lds[addr[t]:addr[t] + 16], tile[row[t], 16 * chunk[t]:16 * chunk[t] + 16])


def _t256_addresses(M, N, K):
    """gemm_i8_t256_kernel: 256 x 256 tiles, K steps of 64; each of the 8
    waves moves 2 A blocks (16 rows x 64 k) and 2 B blocks (4 k-rows x 256 n)
    per step.  The prologue issues steps 0-2 (and 3 for the first wave
    group), the memory phases of step j issue step j + 4 (first group) or
    j + 3 (second group), so steps up to nk + 3 are issued (those past the
    end re-load step nk - 1)."""
    slot = (64 * (2 * np.arange(8)[:, None, None] + np.arange(2)[None, :, None])
            + np.arange(64)[None, None, :]).ravel()
    assert sorted(slot.tolist()) == list(range(1024))   # every slot of both 16 KiB halves once
    ar = slot >> 2
    akc = 16 * ((slot & 3) ^ ((ar >> 1) & 3))
    br, bc = _b_chunk(slot, 256)
    bnc = 16 * bc
    assert ar.max() < 256 and br.max() < 64 and bnc.max() + 16 <= 256
    nk = K // BK
    lo = [None, None]
    hi = [None, None]
    for m0 in range(0, M, 256):
        a_off = (m0 + ar) * K + akc
        for n0 in range(0, N, 256):
            b_off = br * N + n0 + bnc
            for step in range(0, nk + 4):
                k0 = step * BK
                sa = k0 if k0 < K else K - BK
                sb = k0 * N if k0 < K else (K - BK) * N
                for i, v in enumerate((a_off + sa, b_off + sb)):
                    lo[i] = v.min() if lo[i] is None else min(lo[i], v.min())
                    hi[i] = v.max() if hi[i] is None else max(hi[i], v.max())
    return (lo[0], hi[0] + 16, M * K), (lo[1], hi[1] + 16, K * N)


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (4096, 4096, 4096), (512, 768, 1024), (4096, 11008, 4096),
                                   (256, 512, 8192)])
def test_t256_tile_dma_stays_inside_operands(M, N, K):
    assert M % 256 == 0 and N % 256 == 0 and K % 256 == 0
    for lo, end, lim in _t256_addresses(M, N, K):
        assert lo >= 0 and end <= lim, (end, lim)


def _permlane16_swap(a, b):
    """v_permlane16_swap_b32 on 64-lane vectors: the second 16 lanes of each
    32-lane half of `a` trade places with the first 16 of `b`."""
    r0, r1 = a.copy(), b.copy()
    for base in (0, 32):
        r0[base + 16:base + 32] = b[base:base + 16]
        r1[base:base + 16] = a[base + 16:base + 32]
    return r0, r1


def test_t256_int16_epilogue_lane_algebra():
    """The int16 epilogue of gemm_i8_t256_kernel, restated lane by lane: from
    the 16x16x64 result layout (lane l, element r = row 4 (l >> 4) + r,
    column l & 15 of each block) through the per-lane limb combination, the
    DPP exchange between lanes 2c and 2c + 1 and v_permlane16_swap, every
    store must put sum_{X,Y} 2^(8 (X + Y)) c[2 i' + X][2 j' + Y] (mod 2^32) at
    int16 row 8 i + 2 s + p + 4 (l >> 5), column col16(l) of the wave's
    64 x 32 output block, and together the stores must cover it once."""
    rng = np.random.default_rng(5)
    c8 = rng.integers(-2**31, 2**31, size=(128, 64), dtype=np.int64).astype(np.uint32)   # wave's int8-GEMM block
    want = np.zeros((64, 32), np.uint64)
    for X in range(2):
        for Y in range(2):
            want += c8[X::2, Y::2].astype(np.uint64) << np.uint64(8 * (X + Y))
    want &= np.uint64(0xFFFFFFFF)
    lane = np.arange(64)
    odd = lane & 1
    col16 = 16 * ((lane >> 4) & 1) + 8 * (lane & 1) + ((lane & 15) >> 1)
    seen = np.zeros((64, 32), int)
    for i in range(8):
        for p in range(2):
            v = []
            for jp in range(2):
                part = []
                for jj in range(2):
                    j = 2 * jp + jj
                    rows = 16 * i + 4 * (lane >> 4)
                    cols = 16 * j + (lane & 15)
                    lo = c8[rows + 2 * p, cols].astype(np.uint64)
                    hi = c8[rows + 2 * p + 1, cols].astype(np.uint64)
                    part.append(((lo + (hi << np.uint64(8))) << (np.uint64(8) * odd.astype(np.uint64)))
                                & np.uint64(0xFFFFFFFF))
                send = np.where(odd == 1, part[0], part[1])
                keep = np.where(odd == 1, part[1], part[0])
                recv = send[lane ^ 1]                      # quad_perm [1, 0, 3, 2]
                v.append((keep + recv) & np.uint64(0xFFFFFFFF))
            sw = _permlane16_swap(v[0], v[1])
            for s in range(2):
                row = 8 * i + 2 * s + p + 4 * (lane >> 5)
                np.testing.assert_array_equal(sw[s], want[row, col16])
                np.add.at(seen, (row, col16), 1)
    assert (seen == 1).all()


@pytest.mark.parametrize("mi,nj", [(8, 4), (4, 4), (4, 2)])
def test_int8_store_pairs_cover_the_wave_tile(mi, nj):
    """store_c of gemm_i8_t256_kernel (8 x 4 blocks per wave) and
    gemm_i8_h128_kernel (4 x 4, 4 x 2): store e pairs blocks 2 jp and
    2 jp + 1 of row block i through v_permlane16_swap and writes lane l to
    row 16 i + r + 4 h + 8 (l >> 5), column 32 jp + (l & 31); every element
    of the 16 mi x 16 nj wave tile must be written once, with its own value."""
    rng = np.random.default_rng(mi * 10 + nj)
    tile = rng.integers(0, 2**32, size=(16 * mi, 16 * nj), dtype=np.uint64)
    lane = np.arange(64)
    # element r of block (i, j) in lane l: row 16 i + 4 (l >> 4) + r, column 16 j + (l & 15)
    acc = [[[tile[16 * i + 4 * (lane >> 4) + r, 16 * j + (lane & 15)] for r in range(4)] for j in range(nj)]
           for i in range(mi)]
    got = np.full(tile.shape, np.uint64(2**63))
    count = np.zeros(tile.shape, int)
    for e in range(mi * nj * 4):
        h, jp, r, i = e & 1, (e >> 1) % (nj // 2), (e // nj) & 3, e // (4 * nj)
        sw = _permlane16_swap(acc[i][2 * jp][r], acc[i][2 * jp + 1][r])
        row = 16 * i + r + 4 * h + 8 * (lane >> 5)
        col = 32 * jp + (lane & 31)
        got[row, col] = sw[h]
        np.add.at(count, (row, col), 1)
    assert (count == 1).all()
    np.testing.assert_array_equal(got, tile)


def _pad_model(src, base_mis, rows, cols, rows_out, dcols):
    """pad_i8_kernel's lane algebra for one operand: per wave of 64 chunks,
    aligned 16-byte loads (byte loads where a chunk leaves the buffer), the
    lane + 1 exchange, the funnel shift by the row's offset into the 16-byte
    grid and the tail mask.  Returns the panel and asserts every vector load
    is aligned and inside the buffer."""
    total = rows * cols
    buf = np.frombuffer(src.tobytes(), np.uint8)

    def load16(o):
        if o >= 0 and o + 16 <= total:
            assert (base_mis + o) % 16 == 0
            return buf[o:o + 16].copy()
        out = np.zeros(16, np.uint8)
        for e in range(16):
            if 0 <= o + e < total:
                out[e] = buf[o + e]
        return out

    panel = np.zeros((rows_out, dcols), np.uint8)
    for cw in range(0, dcols, 1024):
        for row in range(rows_out):
            if row >= rows or cw >= cols:
                continue
            p = row * cols + cw
            sh = (base_mis + p) % 16
            o = p - sh
            q = [load16(o + 16 * lane) for lane in range(64)]
            nxt = q[1:] + [load16(o + 16 * 64)]
            for lane in range(64):
                c0 = cw + 16 * lane
                if c0 >= dcols:
                    continue
                w = np.concatenate([q[lane], nxt[lane]])[sh:sh + 16]
                valid = cols - c0
                if valid < 16:
                    w[max(valid, 0):] = 0
                panel[row, c0:c0 + 16] = w
    return panel


@pytest.mark.parametrize("rows,cols,mis", [(5, 4095, 3), (3, 1000, 0), (4, 17, 13), (2, 2100, 7), (3, 1, 1),
                                           (6, 300, 15)])
def test_pad_kernel_lane_algebra(rows, cols, mis):
    rng = np.random.default_rng(rows * 131 + cols + mis)
    src = rng.integers(-128, 128, (rows, cols), dtype=np.int8)
    rows_out, dcols = -(-rows // 256) * 256, -(-cols // 256) * 256
    want = np.zeros((rows_out, dcols), np.uint8)
    want[:rows, :cols] = src.view(np.uint8)
    assert np.array_equal(_pad_model(src, mis, rows, cols, rows_out, dcols), want)


# ------------------------------------------------------------------ batched GEMV W ring
# gemv8_kernel (mind_amd/csrc/det_gemv_mfma.hip) streams W rows into a register
# ring with buffer loads whose step offset is the uniform soffset, which the
# range check does not cover: voffset = this lane's row / K-group base + 64 j,
# soffset = 256 * step, the step clamped to the last of the wave's K half, so
# the reloads past the end re-read that step.  Every load must stay inside
# the lane's own W row.
GEMV_DEPTH = 4


def _gemv8_w_addresses(M, K):
    nsteps = K // 64
    half = nsteps // 2
    blocks = (M + 63) // 64
    b = np.arange(blocks)[:, None, None]
    w = np.arange(8)[None, :, None]
    lane = np.arange(64)[None, None, :]
    rg, kh = w & 3, w >> 2
    r, g = lane & 15, lane >> 4
    myrow = np.minimum(b * 64 + rg * 16 + r, M - 1)
    wbase = (myrow * K + 4 * g) * 4
    sbeg = kh * half
    steps = [sbeg + d for d in range(GEMV_DEPTH)]                                   # prologue
    steps += [np.minimum(sbeg + ls + GEMV_DEPTH, sbeg + half - 1) for ls in range(half)]   # ring reloads
    lo = hi = None
    for st in steps:
        for j in range(4):
            addr = wbase + 64 * j + 256 * st
            row_lo, row_hi = myrow * K * 4, (myrow + 1) * K * 4
            assert (addr >= row_lo).all() and (addr + 16 <= row_hi).all()
            lo = addr.min() if lo is None else min(lo, addr.min())
            hi = (addr + 16).max() if hi is None else max(hi, (addr + 16).max())
    return lo, hi


@pytest.mark.parametrize("M,K", [(16, 512), (16384, 16384), (11922, 4096), (130, 32768), (100, 1024)])
def test_gemv8_w_ring_stays_inside_each_row(M, K):
    lo, hi = _gemv8_w_addresses(M, K)
    assert lo >= 0 and hi <= M * K * 4


# ---------------------------------------------------------------- Q16 K split
# det_gemm_q16x.hip: grids of 64 x 64 tiles that fill at most half the CUs
# run kspl workgroups per tile (q16x_ksplit), workgroup ks over the 64-k
# steps [ks NK / kspl, (ks + 1) NK / kspl) of NK = ceil(K / 64); its DMA
# reaches step kt0 + min(kt + 2, nk - 1) at most.  Restated here: the ranges
# must partition [0, NK) with at least one step each, the split count must
# stay within 8 and the idle CUs, and no issued step may leave [0, NK).

def _q16x_ksplit(M, N, K, cus):
    tiles = ((M + 63) // 64) * ((N + 63) // 64)
    nk = (K + 63) // 64
    if 2 * tiles > cus or nk < 2:
        return 1
    k = min(8, cus // tiles, nk)
    steps = (nk + k - 1) // k
    return (nk + steps - 1) // steps


@pytest.mark.parametrize("cus", [256, 80, 32])
def test_q16x_k_split_ranges_partition_k(cus):
    rng = np.random.default_rng(cus)
    shapes = [(256, 256, 256), (512, 512, 512), (7, 5000, 130), (100, 4200, 70), (200, 4160, 300), (64, 64, 64),
              (1000, 4100, 33), (512, 2048, 512), (1024, 1024, 1024), (1, 65535, 1)]
    shapes += [tuple(int(v) for v in rng.integers(1, 3000, 3)) for _ in range(300)]
    for M, K, N in shapes:
        tiles = ((M + 63) // 64) * ((N + 63) // 64)
        NK = (K + 63) // 64
        kspl = _q16x_ksplit(M, N, K, cus)
        assert 1 <= kspl <= 8 and (kspl == 1 or tiles * kspl <= cus), (M, K, N, kspl)
        covered = []
        for ks in range(kspl):
            kt0 = ks * NK // kspl
            nk = (ks + 1) * NK // kspl - kt0
            assert nk >= 1, (M, K, N, ks)
            issued = [kt0 + min(kt + 2, nk - 1) for kt in range(nk)] + [kt0, kt0 + (1 if nk > 1 else 0)]
            assert 0 <= min(issued) and max(issued) < NK, (M, K, N, ks)
            covered += list(range(kt0, kt0 + nk))
        assert covered == list(range(NK)), (M, K, N)
        # every split but the longest is at most one step shorter
        lens = [(ks + 1) * NK // kspl - ks * NK // kspl for ks in range(kspl)]
        assert max(lens) - min(lens) <= 1


# ---------------------------------------------------------------- tiny GEMMs
# det_gemm_small.hip (int8 / int16) and det_gemm_q16s.hip stage A rows and B
# columns as [16][row stride] in LDS; each thread of a 16-lane group reads
# 16 K-contiguous bytes of its own column c at the same k.  With the padded
# strides (272 bytes for int8 / int16, 260 dwords for Q16) the 16 columns'
# 16-byte reads land on 64 distinct 4-byte banks, and every row start stays
# 16-byte aligned.

@pytest.mark.parametrize("stride_bytes", [272, 260 * 4], ids=["int8_int16", "q16"])
def test_tiny_kernel_lds_reads_conflict_free(stride_bytes):
    assert stride_bytes % 16 == 0
    for k_bytes in range(0, 256, 16):
        banks = []
        for c in range(16):
            d0 = (c * stride_bytes + k_bytes) // 4
            banks += [(d0 + e) % 64 for e in range(4)]
        assert sorted(banks) == list(range(64)), k_bytes
