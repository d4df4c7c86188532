"""CPU pins of the prepared layout: the selector-ready code encoding and its decode
sequence, and the outlier patch lists of the M = 9..128 kernel.

The decode kernel expands one 32-bit word into 8 fp16 weights with five selector ops,
twelve V_PERM_B32 and four ANDs (wlq_device.h, dequant_word4s).  This test emulates that
sequence with V_PERM_B32 as the CDNA ISA defines it (selector byte s picks byte s of the
64-bit {src0:src1} for s < 8; 8..11 replicate the sign bit of bytes 1, 3, 5, 7; 12 gives
0x00; >= 13 gives 0xFF) on words built by the test helper's encoder, and checks the
result against a direct table lookup lut[c_j] in natural column order, for every code
value at every position and for random words and LUTs."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import apply_wide_patches, selector_encode, wide_patches_reference
from oracle import wlq_oracle as O
from qwen_wlqfastshot_helen_beta_amd import synth


def v_perm(src0: np.ndarray, src1: np.ndarray, sel: np.ndarray) -> np.ndarray:
    data = (src0.astype(np.uint64) << np.uint64(32)) | src1.astype(np.uint64)
    out = np.zeros(np.broadcast(src0, sel).shape, dtype=np.uint32)
    for byte in range(4):
        s = (np.asarray(sel, np.uint32) >> np.uint32(8 * byte)) & np.uint32(0xFF)
        picked = (data >> (np.uint64(8) * (s.astype(np.uint64) & np.uint64(7)))) & np.uint64(0xFF)
        sign = {8: 15, 9: 31, 10: 47, 11: 63}
        val = picked.astype(np.uint32)
        for k, bit in sign.items():
            val = np.where(s == k, np.where((data >> np.uint64(bit)) & np.uint64(1), 0xFF, 0x00), val)
        val = np.where(s == 12, 0, val)
        val = np.where(s >= 13, 0xFF, val)
        out |= (val.astype(np.uint32) & np.uint32(0xFF)) << np.uint32(8 * byte)
    return out


def planes(lut16: np.ndarray):
    """fp16 LUT [..., 16] -> (lo[4], hi[4]) plane registers (bytes of entries 4p..4p+3)."""
    u = lut16.view(np.uint16).astype(np.uint32)
    lo = [(u[..., 4 * p] & 0xFF) | ((u[..., 4 * p + 1] & 0xFF) << 8) | ((u[..., 4 * p + 2] & 0xFF) << 16)
          | ((u[..., 4 * p + 3] & 0xFF) << 24) for p in range(4)]
    hi = [(u[..., 4 * p] >> 8) | ((u[..., 4 * p + 1] >> 8) << 8) | ((u[..., 4 * p + 2] >> 8) << 16)
          | ((u[..., 4 * p + 3] >> 8) << 24) for p in range(4)]
    return lo, hi


def dequant_word4s(w: np.ndarray, lo, hi) -> np.ndarray:
    """The kernel's sequence, step by step -> fp16 bit patterns [..., 8]."""
    w = w.astype(np.uint32)
    sa = w & np.uint32(0x87878787)
    rb = (w >> np.uint32(4)) | (w << np.uint32(28))
    sb = rb & np.uint32(0x87878787)

    def lookup(sel):
        sel_b = sel ^ np.uint32(0x80808080)
        l_ = v_perm(lo[1], lo[0], sel) & v_perm(lo[3], lo[2], sel_b)
        h_ = v_perm(hi[1], hi[0], sel) & v_perm(hi[3], hi[2], sel_b)
        return l_, h_

    la, ha = lookup(sa)
    lb, hb = lookup(sb)
    pairs = [v_perm(ha, la, np.uint32(0x05010400)), v_perm(ha, la, np.uint32(0x07030602)),
             v_perm(hb, lb, np.uint32(0x05010400)), v_perm(hb, lb, np.uint32(0x07030602))]
    out = np.stack([(p >> np.uint32(16 * h)) & np.uint32(0xFFFF) for p in pairs for h in (0, 1)], axis=-1)
    return out.astype(np.uint16)


def test_v_perm_emulation_known_answers():
    src0, src1 = np.uint32(0x8877_6655), np.uint32(0x4433_2211)
    assert int(v_perm(src0, src1, np.uint32(0x07000301))) == 0x88_11_44_22
    assert int(v_perm(src0, src1, np.uint32(0x0D0C0B08))) == 0xFF_00_FF_00  # byte 7 sign 1, byte 1 sign 0


def test_every_code_at_every_position():
    rng = np.random.default_rng(0)
    lut = rng.standard_normal(16).astype(np.float16)
    lo, hi = planes(lut)
    for pos in range(8):
        c = np.zeros((16, 8), dtype=np.uint32)
        c[:, pos] = np.arange(16)
        c[:, (pos + 3) % 8] = 15 - np.arange(16)  # a different code in a neighbour position
        w = selector_encode(c)
        got = dequant_word4s(w, lo, hi)
        want = lut.view(np.uint16)[c]
        assert np.array_equal(got, want), pos


def test_random_words_and_luts():
    rng = np.random.default_rng(1)
    n = 4096
    c = rng.integers(0, 16, size=(n, 8)).astype(np.uint32)
    lut = rng.standard_normal((n, 16)).astype(np.float16)
    lo, hi = planes(lut)
    got = dequant_word4s(selector_encode(c), lo, hi)
    want = np.take_along_axis(lut.view(np.uint16), c.astype(np.int64), axis=1)
    assert np.array_equal(got, want)
    # 3-bit codes (values 0..7) against an 8-entry LUT padded with zeros to 16
    c3 = rng.integers(0, 8, size=(n, 8)).astype(np.uint32)
    lut3 = np.zeros((n, 16), dtype=np.float16)
    lut3[:, :8] = rng.standard_normal((n, 8)).astype(np.float16)
    lo3, hi3 = planes(lut3)
    got3 = dequant_word4s(selector_encode(c3), lo3, hi3)
    assert np.array_equal(got3, np.take_along_axis(lut3.view(np.uint16), c3.astype(np.int64), axis=1))


def _dense_without_outliers(L):
    return O.dequant(L.q, L.lut, L.N, L.K, L.bits, group_size=L.group_size)


def _with_csr(L, offsets, cols, vals):
    return O.dequant(L.q, L.lut, L.N, L.K, L.bits, offsets, cols, vals, group_size=L.group_size)


@pytest.mark.parametrize("N,K,bits,gs,density,heavy", [
    (77, 1000, 4, 128, 0.02, 0.0),   # ragged rows and slabs, K not a multiple of 128
    (64, 3584, 4, 0, 0.005, 0.1),    # heavy rows
    (40, 1928, 3, 64, 0.03, 0.0),    # 3-bit: 640-column chunks (5 slabs)
    (32, 1024, 4, 128, 0.2, 0.0),    # > 256 patches in one 16 x 128 block
])
def test_wide_patch_lists_reproduce_the_overwrite(N, K, bits, gs, density, heavy):
    """The prepared layout's patch lists (numpy builder of the device layout), applied the
    way the M = 9..128 kernel applies them (lane and element decoded from the patch), turn
    the LUT-only W0 into the oracle's W0 with the outlier overwrite, bit for bit."""
    L = synth.make_layer(N=N, K=K, bits=bits, group_size=gs, rank=0, density=density, seed=N + K,
                         heavy_frac=heavy)
    wpidx, wpatch = wide_patches_reference(N, K, bits, L.offsets, L.cols, L.vals)
    assert wpidx[-1] == wpatch.size <= L.nnz
    got = apply_wide_patches(_dense_without_outliers(L), wpidx, wpatch, K)
    want = O.dequant(L.q, L.lut, N, K, bits, L.offsets, L.cols, L.vals, group_size=gs)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    if density >= 0.2:
        assert np.diff(wpidx).max() > 256  # the kernel's global-memory overflow path is exercised


def test_wide_patch_lists_edge_entries():
    """Last write wins for a repeated column, a column >= K is dropped (as the dense
    overwrite does), and the lists group by (tile, slab) in row order."""
    N, K, bits = 20, 1000, 4
    C = O.chunk_width(bits)
    L = synth.make_layer(N=N, K=K, bits=bits, group_size=128, rank=0, density=0.0, seed=5)
    # row 3: column 7 twice (values 0x3C then 0x40), column 130; row 17: column 999 and
    # chunk column C - 1 of the last chunk (column 1023 >= K: dropped)
    nch = -(-K // C)
    offsets = np.zeros((N, nch + 1), dtype=np.int32)
    entries = {3: [(0, 7, 0x3C), (0, 7, 0x40), (0, 130, 0x44)], 17: [(1, 999 - C, 0x48), (1, C - 1, 0x7C)]}
    cols, vals, pos = [], [], 0
    for n in range(N):
        for c in range(nch):
            offsets[n, c] = pos
            for cc, col, v in entries.get(n, []):
                if cc == c:
                    cols.append(col)
                    vals.append(v)
                    pos += 1
        offsets[n, nch] = pos
    cols = np.array(cols, dtype=np.uint16)
    vals = np.array(vals, dtype=np.uint8)
    wpidx, wpatch = wide_patches_reference(N, K, bits, offsets, cols, vals)
    assert wpatch.size == 3  # one of the two column-7 entries and the column >= K are gone
    got = apply_wide_patches(_dense_without_outliers(L), wpidx, wpatch, K)
    want = _with_csr(L, offsets, cols, vals)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    assert got.view(np.uint16)[3, 7] == 0x4000  # the later value
    S = -(-K // 128)
    assert [int(wpidx[t * S + s + 1] - wpidx[t * S + s]) for t, s in ((0, 0), (0, 1), (1, 7))] == [1, 1, 1]
