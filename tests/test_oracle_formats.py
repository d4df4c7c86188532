"""Pins for the oracle's layout and encoding functions.

The reference ships no fixtures, so each function is pinned here by values
computed by hand (written as literals), by an independent library (torch's
float8_e5m2 and float16 types, torch.gather), by brute force over bits, or by
round trips through an independently written encoder.
"""
import numpy as np
import pytest
import torch

from oracle import wlq_oracle as O


# ---------------------------------------------------------------- packing KATs

def test_pack_row_aligned_4bit_hand():
    codes = np.array([[1, 2, 3, 4, 5, 6, 7, 8, 9], [15, 0, 0, 0, 0, 0, 0, 0, 1]], dtype=np.uint8)
    q, wpr = O.pack_row_aligned(codes, 4)
    assert wpr == 4  # ceil(9/8)=2 words rounded up to 4
    assert q.tolist() == [0x87654321, 0x9, 0, 0, 0x0000000F, 0x1, 0, 0]


def test_pack_row_aligned_3bit_hand():
    codes = np.array([[1, 2, 3, 4, 5, 6, 7, 0, 1, 2, 3, 4]], dtype=np.uint8)
    q, wpr = O.pack_row_aligned(codes, 3)
    assert wpr == 4
    # word0 = 1 | 2<<3 | 3<<6 | 4<<9 | 5<<12 | 6<<15 | 7<<18 | 0<<21 | 1<<24 | 2<<27, top 2 bits unused
    assert q.tolist() == [0x111F58D1, 0x23, 0, 0]


def test_pack_row_aligned_2bit_1bit_hand():
    q, wpr = O.pack_row_aligned(np.array([[3, 0, 1, 2, 3]], dtype=np.uint8), 2)
    assert wpr == 4 and q.tolist() == [0x393, 0, 0, 0]
    q, wpr = O.pack_row_aligned(np.ones((1, 33), dtype=np.uint8), 1)
    assert wpr == 4 and q.tolist() == [0xFFFFFFFF, 0x1, 0, 0]


def test_words_per_row_hand():
    assert O.words_per_row(3584, 4) == 448
    assert O.words_per_row(18944, 4) == 2368
    assert O.words_per_row(896, 4) == 112
    assert O.words_per_row(3584, 3) == 360
    assert O.words_per_row(1, 1) == 4
    assert O.chunk_width(3) == 640 and O.chunk_width(4) == 512
    assert O.num_chunks(3584, 4) == 7 and O.num_chunks(18944, 4) == 37 and O.num_chunks(3584, 3) == 6


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_pack_bit_by_bit(bits):
    rng = np.random.default_rng(bits)
    N, K = 5, 77
    codes = rng.integers(0, 1 << bits, (N, K), dtype=np.uint8)
    q, wpr = O.pack_row_aligned(codes, bits)
    spw = 10 if bits == 3 else 32 // bits
    words = [int(w) for w in q]
    for n in range(N):
        for k in range(K):
            w = words[n * wpr + k // spw]
            val = 0
            for b in range(bits):  # read bit by bit
                val |= ((w >> ((k % spw) * bits + b)) & 1) << b
            assert val == codes[n, k]
        # padding slots/words are zero
        used = {(k // spw, (k % spw)) for k in range(K)}
        for wi in range(wpr):
            for slot in range(32 // bits if bits != 3 else 10):
                if (wi, slot) not in used:
                    assert (words[n * wpr + wi] >> (slot * bits)) & ((1 << bits) - 1) == 0
        if bits == 3:
            assert all((words[n * wpr + wi] >> 30) == 0 for wi in range(wpr))
    assert np.array_equal(O.unpack_row_aligned(q, N, K, bits), codes)


def test_continuous_hand_and_repack():
    codes = np.array([[1, 2, 3, 4, 5], [6, 7, 8, 9, 10]], dtype=np.uint8)
    cont = O.pack_continuous(codes, 4)
    assert cont.tolist() == [0x87654321, 0xA9]
    assert np.array_equal(O.unpack_continuous(cont, 2, 5, 4), codes)
    q, wpr = O.repack_row_aligned(cont, 2, 5, 4)
    assert wpr == 4 and q.tolist() == [0x54321, 0, 0, 0, 0xA9876, 0, 0, 0]
    # symbols past the end of the source read as zero
    q, _ = O.repack_row_aligned(np.array([0x87654321], dtype=np.uint32), 2, 5, 4)
    assert q.tolist() == [0x54321, 0, 0, 0, 0x876, 0, 0, 0]


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_continuous_round_trip(bits):
    rng = np.random.default_rng(10 + bits)
    codes = rng.integers(0, 1 << bits, (7, 131), dtype=np.uint8)
    assert np.array_equal(O.unpack_continuous(O.pack_continuous(codes, bits), 7, 131, bits), codes)
    q, _ = O.repack_row_aligned(O.pack_continuous(codes, bits), 7, 131, bits)
    assert np.array_equal(O.unpack_row_aligned(q, 7, 131, bits), codes)


# ------------------------------------------------------------------ e5m2 bytes

def test_e5m2_decode_exhaustive_vs_torch():
    u8 = np.arange(256, dtype=np.uint8)
    ours = O.e5m2_to_fp16_bits(u8).view(np.float16).astype(np.float32)
    ref = torch.from_numpy(u8).view(torch.float8_e5m2).to(torch.float32).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], ref[~nan])


def test_e5m2_encode_vs_torch_off_ties():
    """Round-half-up on the magnitude equals round-to-nearest-even except on exact ties."""
    u16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = u16.view(np.float16)
    ours = O.fp16_bits_to_e5m2(u16)
    ref = torch.from_numpy(f.copy()).to(torch.float8_e5m2).view(torch.uint8).numpy()
    finite = np.isfinite(f) & (np.abs(f.astype(np.float32)) < 57344.0)
    off_tie = (u16 & 0xFF) != 0x80
    sel = finite & off_tie
    assert np.array_equal(ours[sel], ref[sel])


def test_e5m2_encode_hand_ties_and_clamp():
    cases = {0x3C00: 0x3C, 0x3C7F: 0x3C, 0x3C80: 0x3D, 0x3D80: 0x3E, 0xBC80: 0xBD, 0x0080: 0x01,
             0xFF7F: 0xFF, 0xFF80: 0xFF, 0xFFFF: 0xFF, 0x7B80: 0x7C}
    for u, e in cases.items():
        assert int(O.fp16_bits_to_e5m2(np.array([u], dtype=np.uint16))[0]) == e, hex(u)
    assert O.e5m2_to_fp16_bits(np.array([0x3C], dtype=np.uint8)).view(np.float16)[0] == 1.0
    assert O.e5m2_to_fp16_bits(np.array([0xC1], dtype=np.uint8)).view(np.float16)[0] == -2.5


# ------------------------------------------------------------------- chunk CSR

def test_chunk_csr_hand():
    mask = np.zeros((2, 1100), dtype=bool)
    for r, c in [(0, 5), (0, 600), (1, 1099), (1, 0), (1, 513)]:
        mask[r, c] = True
    vals = np.array([1.0, -2.0, 0.5, 4.0, -0.25], dtype=np.float16)  # row-major nonzero order
    off, cols, v = O.build_chunk_csr(mask, vals, 512)
    assert off.tolist() == [[0, 1, 2, 2], [2, 3, 4, 5]]
    assert cols.tolist() == [5, 88, 0, 1, 75]
    assert v.tolist() == [0x3C, 0xC0, 0x38, 0x44, 0xB4]


def test_chunk_csr_brute_force():
    rng = np.random.default_rng(3)
    for K, C in [(1000, 512), (1500, 640), (512, 512)]:
        mask = rng.random((9, K)) < 0.03
        off, cols, _ = O.build_chunk_csr(mask, None, C)
        nch = -(-K // C)
        assert off.shape == (9, nch + 1) and off[0, 0] == 0 and off[-1, -1] == mask.sum()
        assert np.all(np.diff(off.ravel()) >= 0)
        for n in range(9):
            for c in range(nch):
                seg = cols[off[n, c]:off[n, c + 1]].astype(int).tolist()
                want = [k - c * C for k in range(c * C, min(K, (c + 1) * C)) if mask[n, k]]
                assert seg == want
            if n + 1 < 9:
                assert off[n, nch] == off[n + 1, 0]


# ----------------------------------------------------------------- dequantize

def _lut_rows(N, groups, bits, seed):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((N, groups, 1 << bits)).astype(np.float16)


def test_dequant_hand():
    lut = np.array([i * 0.25 - 2.0 for i in range(16)], dtype=np.float16)[None, :]  # -2.0 .. 1.75
    codes = np.array([[0, 15, 3, 8, 1, 2, 9, 10, 4, 5]], dtype=np.uint8)
    q, wpr = O.pack_row_aligned(codes, 4)
    W = O.dequant(q, lut, 1, 10, 4)
    assert W.astype(np.float32).tolist() == [[-2.0, 1.75, -1.25, 0.0, -1.75, -1.5, 0.25, 0.5, -1.0, -0.75]]
    off = np.array([[0, 2]], dtype=np.int32)
    cols = np.array([3, 9], dtype=np.uint16)
    vals = np.array([0x3C, 0xC1], dtype=np.uint8)  # 1.0, -2.5
    W = O.dequant(q, lut, 1, 10, 4, off, cols, vals)
    assert W.astype(np.float32).tolist() == [[-2.0, 1.75, -1.25, 1.0, -1.75, -1.5, 0.25, 0.5, -1.0, -2.5]]


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_dequant_per_row_equals_torch_gather(bits):
    rng = np.random.default_rng(bits)
    N, K = 6, 301
    codes = rng.integers(0, 1 << bits, (N, K), dtype=np.uint8)
    lut = _lut_rows(N, 1, bits, bits)[:, 0, :]
    q, _ = O.pack_row_aligned(codes, bits)
    W = O.dequant(q, lut, N, K, bits)
    ref = torch.gather(torch.from_numpy(lut), 1, torch.from_numpy(codes.astype(np.int64))).numpy()
    assert np.array_equal(W.view(np.uint16), ref.view(np.uint16))


def test_dequant_groups_loops_and_outliers():
    rng = np.random.default_rng(5)
    N, K, G, bits = 4, 300, 64, 4
    codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
    lut = _lut_rows(N, -(-K // G), bits, 9)
    q, _ = O.pack_row_aligned(codes, bits)
    mask = rng.random((N, K)) < 0.05
    vals = rng.standard_normal(mask.sum()).astype(np.float16)
    off, cols, v = O.build_chunk_csr(mask, vals, 512)
    W = O.dequant(q, lut, N, K, bits, off, cols, v, group_size=G)
    e = v.astype(np.uint16) << 8
    j = 0
    for n in range(N):
        for k in range(K):
            if mask[n, k]:
                assert W.view(np.uint16)[n, k] == e[j]
                j += 1
            else:
                assert W.view(np.uint16)[n, k] == lut.view(np.uint16)[n, k // G, codes[n, k]]
    # group_size >= K is the per-row layout
    W1 = O.dequant(q, lut[:, :1, :], N, K, bits, group_size=K)
    W0 = O.dequant(q, lut[:, 0, :], N, K, bits)
    assert np.array_equal(W1.view(np.uint16), W0.view(np.uint16))


def test_outlier_delta_hand():
    lut = np.array([i * 0.25 - 2.0 for i in range(16)], dtype=np.float16)[None, :]  # -2.0 .. 1.75
    codes = np.array([[0, 15, 3, 8, 1, 2, 9, 10, 4, 5]], dtype=np.uint8)
    q, _ = O.pack_row_aligned(codes, 4)
    off = np.array([[0, 3]], dtype=np.int32)
    cols = np.array([3, 9, 11], dtype=np.uint16)  # column 11 is past K = 10: dropped
    vals = np.array([0x3C, 0xC1, 0x3C], dtype=np.uint8)  # 1.0, -2.5, 1.0
    gcol, delta = O.outlier_delta(q, lut, 1, 10, 4, off, cols, vals)
    assert gcol.tolist() == [3, 9, 0]
    # code 8 -> 0.0, code 5 -> -0.75
    assert delta.tolist() == [1.0, -1.75, 0.0]


def test_outlier_delta_loops_and_invariant():
    rng = np.random.default_rng(8)
    N, K, G, bits = 5, 1100, 64, 4
    codes = rng.integers(0, 16, (N, K), dtype=np.uint8)
    lut = _lut_rows(N, -(-K // G), bits, 3)
    q, _ = O.pack_row_aligned(codes, bits)
    mask = rng.random((N, K)) < 0.03
    vals = (rng.standard_normal(mask.sum()) * 0.2).astype(np.float16)
    off, cols, v = O.build_chunk_csr(mask, vals, 512)
    gcol, delta = O.outlier_delta(q, lut, N, K, bits, off, cols, v, group_size=G)
    e = 0
    for n in range(N):
        for k in range(K):
            if mask[n, k]:
                w_true = np.float32((v[e].astype(np.uint16) << 8).view(np.float16))
                w_lut = np.float32(lut[n, k // G, codes[n, k]])
                assert gcol[e] == k
                assert delta[e] == np.float32(w_true - w_lut)
                e += 1
    # sum of delta * x over a row's entries == (W0 - W_lut) . x
    x = rng.standard_normal(K)
    W0 = O.dequant(q, lut, N, K, bits, off, cols, v, group_size=G).astype(np.float64)
    Wl = O.dequant(q, lut, N, K, bits, group_size=G).astype(np.float64)
    _, rows, _ = O.csr_to_coo(off, cols, 512)
    corr = np.zeros(N)
    np.add.at(corr, rows, delta.astype(np.float64) * x[gcol])
    assert np.allclose(corr, (W0 - Wl) @ x, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------- Elias-Fano

def test_ef_hand_bitstream():
    # tile 4x4 (U=16), entries at local 1, 6, 11 -> m=3, L=floor(log2(16/3))=2
    # low bits (LSB first): 1->10, 2->01, 3->11 ; unary highs 0,1,2 -> 1, 01, 01
    # stream: 1 0 0 1 1 1 | 1 0 1 0 1 -> bits 0,3,4,5,6,8,10 -> 0x579
    meta = np.array([[0, 3]], dtype=np.int64)
    bs = np.array([0x579], dtype=np.uint32)
    mask = O.ef_decode_mask(meta, bs, 4, 4, 4)
    assert sorted(zip(*np.nonzero(mask))) == [(0, 1), (1, 2), (2, 3)]
    m2, b2 = O.ef_encode(mask, 4)
    assert m2.tolist() == [[0, 3]] and b2.tolist() == [0x579]


def test_ef_round_trip_random():
    rng = np.random.default_rng(0)
    for (H, W, T, d) in [(20, 37, 8, 0.1), (64, 64, 16, 0.02), (9, 100, 32, 0.5), (5, 5, 4, 1.0), (17, 40, 8, 0.0)]:
        mask = rng.random((H, W)) < d
        meta, bs = O.ef_encode(mask, T)
        assert np.array_equal(O.ef_decode_mask(meta, bs, H, W, T), mask)
        off, cols = O.ef_decode_to_chunk_csr(meta, bs, H, W, T, 16)
        off2, cols2, _ = O.build_chunk_csr(mask, None, 16)
        assert np.array_equal(off, off2) and np.array_equal(cols, cols2)


def test_ef_vectorized_encoder_matches_the_oracle():
    """formats.ef_encode_coords (the checkpoint writer's encoder) emits the oracle encoder's
    meta and bitstream bit for bit, including empty and full tiles and ragged edges, and the
    hand-coded example above."""
    from qwen_wlqfastshot_helen_beta_amd import formats

    meta, bs = formats.ef_encode_coords([0, 1, 2], [1, 2, 3], 4, 4, 4)
    assert meta.tolist() == [[0, 3]] and bs.tolist() == [0x579]
    rng = np.random.default_rng(3)
    for (H, W, T, d) in [(20, 37, 8, 0.1), (64, 64, 16, 0.02), (9, 100, 32, 0.5), (5, 5, 4, 1.0), (17, 40, 8, 0.0),
                         (130, 200, 64, 0.005), (70, 65, 64, 0.3)]:
        mask = rng.random((H, W)) < d
        r, c = np.nonzero(mask)
        perm = rng.permutation(r.size)  # any input order
        meta, bs = formats.ef_encode_coords(r[perm], c[perm], H, W, T)
        m2, b2 = O.ef_encode(mask, T)
        assert np.array_equal(meta, m2), (H, W, T, d)
        assert np.array_equal(bs, b2), (H, W, T, d)
    with pytest.raises(ValueError):
        formats.ef_encode_coords([1, 1], [2, 2], 4, 4, 4)
