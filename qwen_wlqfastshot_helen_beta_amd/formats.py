"""Host-side layout helpers for WLQ weights (numpy).

These are the data formats the device kernels consume:

* ``q_packed_aligned``: int32 ``[N * wpr]``.  Code (n, k) sits in word
  ``n*wpr + k//spw`` at bit ``(k % spw) * bits``, LSB first, zero padded; spw is
  10 for 3-bit (top two bits unused) and 32/bits otherwise; wpr is the raw word
  count rounded up to a multiple of 4 so every row starts 16-byte aligned
  (vllm_wlq/linear_method.py:326-338).
* on-disk continuous packing: flat index ``n*K + k`` goes to word ``//spw``,
  slot ``%spw`` (vllm_wlq/linear_method.py:315-323).
* chunk CSR outliers: ``chunk_offsets`` int32 ``[N, nch+1]`` (global prefix sums
  in row-major (row, chunk) order), ``chunk_cols`` uint16 (column inside the
  chunk), ``chunk_vals`` uint8 (fp8-e5m2 bit pattern; the weight is the fp16
  with bits ``v << 8``).  The chunk is 512 columns, 640 for 3-bit
  (vllm_wlq/linear_method.py:284-312, csrc/vllm_binding.cpp:279).
* LUTs: fp16 ``[N, 2**bits]`` per row (the reference) or ``[N, ceil(K/G), 2**bits]``
  per group of G input columns (this build's extension, ``group_size=G``).
"""
from __future__ import annotations

from typing import Tuple

import numpy as np


def symbols_per_word(bits: int) -> int:
    if bits not in (1, 2, 3, 4):
        raise ValueError(f"unsupported bits={bits}; supported widths are 1, 2, 3, 4")
    return 10 if bits == 3 else 32 // bits


def words_per_row(K: int, bits: int) -> int:
    spw = symbols_per_word(bits)
    return ((K + spw - 1) // spw + 3) // 4 * 4


def chunk_width(bits: int) -> int:
    return 640 if bits == 3 else 512


def num_chunks(K: int, bits: int) -> int:
    return (K + chunk_width(bits) - 1) // chunk_width(bits)


def num_groups(K: int, group_size: int) -> int:
    return 1 if group_size <= 0 else (K + group_size - 1) // group_size


def pack_indices_row_aligned(q_idx_2d: np.ndarray, bits: int) -> Tuple[np.ndarray, int]:
    """Pack codes ``[N, K]`` into the row-aligned layout; returns (uint32 flat, wpr)."""
    N, K = q_idx_2d.shape
    spw = symbols_per_word(bits)
    wpr = words_per_row(K, bits)
    out = np.empty((N, wpr), dtype=np.uint32)
    shifts = (np.arange(spw, dtype=np.uint32) * np.uint32(bits))[None, None, :]
    step = max(1, (1 << 24) // max(1, wpr * spw))
    for r0 in range(0, N, step):
        blk = q_idx_2d[r0:r0 + step]
        pad = np.zeros((blk.shape[0], wpr * spw), dtype=np.uint32)
        pad[:, :K] = blk
        words = pad.reshape(blk.shape[0], wpr, spw) << shifts
        out[r0:r0 + step] = np.bitwise_or.reduce(words, axis=2)
    return out.ravel(), wpr


def unpack_indices_continuous(q_packed: np.ndarray, N: int, K: int, bits: int) -> np.ndarray:
    """Continuous on-disk packing -> codes ``[N, K]`` (uint32)."""
    spw = symbols_per_word(bits)
    mask = np.uint32((1 << bits) - 1)
    q = np.ascontiguousarray(q_packed).view(np.uint32)
    shifts = np.arange(spw, dtype=np.uint32) * np.uint32(bits)
    flat = ((q[:, None] >> shifts[None, :]) & mask).ravel()
    total = N * K
    if flat.size < total:
        flat = np.concatenate([flat, np.zeros(total - flat.size, dtype=np.uint32)])
    return flat[:total].reshape(N, K)


def pack_indices_continuous(q_idx_2d: np.ndarray, bits: int) -> np.ndarray:
    """Codes ``[N, K]`` -> continuous on-disk packing (uint32)."""
    spw = symbols_per_word(bits)
    flat = np.ascontiguousarray(q_idx_2d, dtype=np.uint32).ravel()
    nwords = (flat.size + spw - 1) // spw
    pad = np.zeros(nwords * spw, dtype=np.uint32)
    pad[:flat.size] = flat
    shifts = np.arange(spw, dtype=np.uint32) * np.uint32(bits)
    return np.bitwise_or.reduce(pad.reshape(nwords, spw) << shifts[None, :], axis=1)


def fp16_to_e5m2_u8(values_fp16: np.ndarray) -> np.ndarray:
    """fp16 values -> e5m2 bytes with the checkpoint loader's rounding
    ``clamp((u16 + 0x80) >> 8, 0, 255)`` (vllm_wlq/linear_method.py:306-308)."""
    u16 = np.ascontiguousarray(values_fp16, dtype=np.float16).view(np.uint16).astype(np.int32)
    return np.clip((u16 + 0x80) >> 8, 0, 255).astype(np.uint8)


def ef_encode_coords(rows: np.ndarray, cols: np.ndarray, N: int, K: int, tile_size: int = 64):
    """Outlier positions -> the checkpoint's Elias-Fano tiles (``ef_tile_meta`` int64
    ``[tiles, 2]`` = (start bit, count), ``ef_bitstream`` uint32), the format the loader
    decodes (vllm_wlq/linear_method.py:243-281, csrc/vllm_binding.cpp:94-196).

    Tiles of ``tile_size``^2 cells in row-major tile order over the padded matrix; in a
    tile the positions are local indices ``(row % T) * T + col % T`` in ascending order,
    coded with L = max(0, floor(log2(T^2 / m))) low bits each (LSB first, one after
    another), then the high parts ``index >> L`` in unary: a 0 per increment over the
    previous element's, a 1 per element.  The stream is the tiles' codes back to back,
    packed LSB first into 32-bit words (at least one).  Vectorized over all positions."""
    rows = np.asarray(rows, dtype=np.int64).ravel()
    cols = np.asarray(cols, dtype=np.int64).ravel()
    T = int(tile_size)
    U = T * T
    nty, ntx = -(-N // T), -(-K // T)
    ntiles = nty * ntx
    tile = (rows // T) * ntx + cols // T
    loc = (rows % T) * T + cols % T
    order = np.lexsort((loc, tile))
    tile, loc = tile[order], loc[order]
    if tile.size > 1 and np.any((tile[1:] == tile[:-1]) & (loc[1:] == loc[:-1])):
        raise ValueError("repeated outlier position")
    m = np.bincount(tile, minlength=ntiles).astype(np.int64)
    L = np.zeros(ntiles, dtype=np.int64)
    nz = m > 0
    L[nz] = np.maximum(0, np.floor(np.log2(U / m[nz].astype(np.float64)))).astype(np.int64)
    first = np.zeros(ntiles + 1, dtype=np.int64)
    first[1:] = np.cumsum(m)
    rank = np.arange(tile.size, dtype=np.int64) - first[tile]
    Le = L[tile]
    high = loc >> Le
    high_last = np.zeros(ntiles, dtype=np.int64)
    high_last[nz] = high[first[1:][nz] - 1]  # ascending within a tile: the last is the largest
    nbits = m * L + np.where(nz, high_last + m, 0)
    start = np.zeros(ntiles, dtype=np.int64)
    start[1:] = np.cumsum(nbits)[:-1]
    total = int(nbits.sum())
    bits = np.zeros(max(1, -(-total // 32)) * 32, dtype=np.uint8)
    base = start[tile] + rank * Le
    for b in range(int(L.max()) if ntiles else 0):
        sel = Le > b
        bits[base[sel] + b] = ((loc[sel] >> b) & 1).astype(np.uint8)
    bits[start[tile] + m[tile] * Le + high + rank] = 1
    meta = np.stack([start, m], axis=1)
    return meta, np.packbits(bits, bitorder="little").view(np.uint32).copy()


def chunk_csr_from_coords(rows: np.ndarray, cols: np.ndarray, N: int, K: int, chunk_m: int):
    """Sorted-or-not (row, col) outlier coordinates -> (offsets int32 [N, nch+1],
    chunk_cols uint16, order) where ``order`` is the permutation that puts the
    entries into row-major order (apply it to the values)."""
    rows = np.asarray(rows, dtype=np.int64)
    cols = np.asarray(cols, dtype=np.int64)
    nch = (K + chunk_m - 1) // chunk_m
    order = np.lexsort((cols, rows))
    rows_s, cols_s = rows[order], cols[order]
    flat = rows_s * nch + cols_s // chunk_m
    counts = np.bincount(flat, minlength=N * nch).reshape(N, nch)
    offsets = np.zeros((N, nch + 1), dtype=np.int64)
    offsets[:, 1:] = np.cumsum(counts, axis=1)
    row_tot = offsets[:, -1].copy()
    starts = np.zeros(N, dtype=np.int64)
    starts[1:] = np.cumsum(row_tot)[:-1]
    offsets += starts[:, None]
    if offsets[-1, -1] > np.iinfo(np.int32).max:
        raise OverflowError("too many outliers for int32 offsets")
    return offsets.astype(np.int32), (cols_s % chunk_m).astype(np.uint16), order


def build_chunk_csr(mask_2d: np.ndarray, values, chunk_m: int):
    """Dense bool mask ``[N, K]`` (+ values in row-major nonzero order, fp16 or
    e5m2 bytes) -> (chunk_offsets, chunk_cols, chunk_vals)."""
    N, K = mask_2d.shape
    rows, cols = np.nonzero(mask_2d)
    offsets, ccols, order = chunk_csr_from_coords(rows, cols, N, K, chunk_m)
    if values is None or np.asarray(values).size == 0:
        vals = np.zeros(0 if values is not None else ccols.size, dtype=np.uint8)
    else:
        v = np.asarray(values)
        vals = fp16_to_e5m2_u8(v) if v.dtype == np.float16 else v.view(np.uint8)
        vals = vals[order]
    return offsets, ccols, vals
