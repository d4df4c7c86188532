"""CPU oracle for the WLQ metalog-LUT quantized linear layer.

TEST INFRASTRUCTURE ONLY.  This module is a plain numpy restatement of the
reference's arithmetic for the hot path.  It is the checker, never the thing
measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``qwen_wlqfastshot_helen_beta_amd``) never imports it and has no CPU fallback.

Citations are ``path:line`` in the reference tree
(wichtelLabs/qwen_wlqFastShot_helen_beta).  The reference ships no tests,
fixtures or golden vectors, and cannot be built or imported here (its
extension needs nvcc, its Python needs vLLM), so each function below is
pinned by the independent checks named in its docstring (hand-computed
known-answer vectors, torch's own float8/float16 conversions, brute force on
tiny inputs, algebraic invariants).  Tests live in ``tests/test_oracle_*.py``.

Pins per function (all in tests/test_oracle_formats.py unless noted):
  pack_row_aligned / unpack_row_aligned    hand-computed words, bit-by-bit brute force, round trip
  pack_continuous / unpack_continuous      hand-computed words, round trip
  repack_row_aligned                       hand-computed words, == pack(unpack_continuous)
  fp16_bits_to_e5m2 / e5m2_to_fp16_bits    exhaustive vs torch.float8_e5m2 (off-tie values), hand ties
  build_chunk_csr                          dense-mask brute force, invariants, hand example
  dequant                                  closed form by loops, torch.gather special case, hand example
  outlier_delta                            per-entry loops, lut + delta == w_true where exact, hand example
  ef_encode / ef_decode_*                  hand-built bitstream, round trip on random masks
  dora_gamma / merge_dora / lora_scale     closed form on hand matrices (tests/test_oracle_layer.py)
  linear_forward / lora_h                  brute-force loops, one-hot rows, r=0, linearity
                                           (tests/test_oracle_layer.py)
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np

# ---------------------------------------------------------------------------
# Layout constants
# ---------------------------------------------------------------------------


def symbols_per_word(bits: int) -> int:
    """Codes per 32-bit word: 10 for 3-bit (top 2 bits unused), else 32/bits.

    Reference: vllm_wlq/linear_method.py:316,328; csrc/vllm_binding.cpp:208.
    """
    if bits not in (1, 2, 3, 4):
        raise ValueError(f"bits must be 1..4, got {bits}")
    return 10 if bits == 3 else 32 // bits


def words_per_row(K: int, bits: int) -> int:
    """Row stride in words: raw words rounded up to a multiple of 4 (one uint4).

    Reference: vllm_wlq/linear_method.py:329-330; csrc/vllm_binding.cpp:209-210.
    """
    spw = symbols_per_word(bits)
    raw = -(-K // spw)
    return -(-raw // 4) * 4


def chunk_width(bits: int) -> int:
    """Outlier chunk width in columns. Reference: csrc/vllm_binding.cpp:279,351."""
    return 640 if bits == 3 else 512


def num_chunks(K: int, bits: int) -> int:
    """Reference: csrc/vllm_binding.cpp:280,352."""
    c = chunk_width(bits)
    return -(-K // c)


def num_groups(K: int, group_size: int) -> int:
    """LUT groups per row. group_size 0 means one LUT per row (the reference layout,
    csrc/gemv_kernel.cu:126-130 indexes lut_c[row*K_CB + sym])."""
    if group_size <= 0:
        return 1
    return -(-K // group_size)


# ---------------------------------------------------------------------------
# Code packing
# ---------------------------------------------------------------------------


def pack_row_aligned(codes: np.ndarray, bits: int) -> Tuple[np.ndarray, int]:
    """Row-aligned packing: code (n,k) -> word n*wpr + k//spw, bit (k%spw)*bits.

    Restates vllm_wlq/linear_method.py:326-338 as a per-element scatter (each
    code is OR-ed into its own word), not as the reference's reshape/reduce.
    Padding words and slots are zero.
    """
    codes = np.asarray(codes)
    N, K = codes.shape
    spw = symbols_per_word(bits)
    wpr = words_per_row(K, bits)
    out = np.zeros(N * wpr, dtype=np.uint64)
    n_idx, k_idx = np.meshgrid(np.arange(N, dtype=np.int64), np.arange(K, dtype=np.int64), indexing="ij")
    word = (n_idx * wpr + k_idx // spw).ravel()
    shift = ((k_idx % spw) * bits).ravel().astype(np.uint64)
    vals = (codes.astype(np.uint64).ravel() & np.uint64((1 << bits) - 1)) << shift
    np.bitwise_or.at(out, word, vals)
    return out.astype(np.uint32), wpr


def unpack_row_aligned(q: np.ndarray, N: int, K: int, bits: int) -> np.ndarray:
    """Inverse of pack_row_aligned: the read every consumer performs,
    ``(q[n*wpr + k/spw] >> ((k%spw)*bits)) & mask`` (csrc/gemv_kernel.cu:279-282,
    csrc/gemm_kernel.cu:352-425)."""
    q = np.asarray(q).view(np.uint32) if np.asarray(q).dtype == np.int32 else np.asarray(q, dtype=np.uint32)
    spw = symbols_per_word(bits)
    wpr = words_per_row(K, bits)
    k = np.arange(K, dtype=np.int64)
    words = q.reshape(N, wpr)[:, k // spw]
    return ((words >> ((k % spw) * bits).astype(np.uint32)) & np.uint32((1 << bits) - 1)).astype(np.uint8)


def pack_continuous(codes: np.ndarray, bits: int) -> np.ndarray:
    """On-disk continuous packing: flat index f=n*K+k -> word f//spw, slot f%spw.

    This is the inverse of vllm_wlq/linear_method.py:315-323 (the reference has no
    packer for this layout; checkpoints arrive packed).
    """
    flat = np.asarray(codes).astype(np.uint64).ravel()
    spw = symbols_per_word(bits)
    nwords = -(-flat.size // spw)
    out = np.zeros(nwords, dtype=np.uint64)
    f = np.arange(flat.size, dtype=np.int64)
    np.bitwise_or.at(out, f // spw, (flat & np.uint64((1 << bits) - 1)) << ((f % spw) * bits).astype(np.uint64))
    return out.astype(np.uint32)


def unpack_continuous(q: np.ndarray, N: int, K: int, bits: int) -> np.ndarray:
    """Reference: vllm_wlq/linear_method.py:315-323."""
    q = np.asarray(q).view(np.uint32) if np.asarray(q).dtype == np.int32 else np.asarray(q, dtype=np.uint32)
    spw = symbols_per_word(bits)
    f = np.arange(N * K, dtype=np.int64)
    w = f // spw
    vals = np.where(w < q.size, q[np.minimum(w, q.size - 1)], 0).astype(np.uint32)
    return ((vals >> ((f % spw) * bits).astype(np.uint32)) & np.uint32((1 << bits) - 1)).reshape(N, K).astype(np.uint8)


def repack_row_aligned(q_raw: np.ndarray, N: int, K: int, bits: int) -> Tuple[np.ndarray, int]:
    """Continuous -> row-aligned. Reference: csrc/vllm_binding.cpp:198-236
    (symbols past the end of the source read as 0, :225-227)."""
    return pack_row_aligned(unpack_continuous(q_raw, N, K, bits), bits)


# ---------------------------------------------------------------------------
# Outlier value encoding (fp8-e5m2 bit patterns)
# ---------------------------------------------------------------------------


def fp16_bits_to_e5m2(u16: np.ndarray) -> np.ndarray:
    """fp16 -> e5m2 byte: ``clamp((u16 + 0x80) >> 8, 0, 255)`` on the unsigned
    bit pattern (round half up on the magnitude bits; 0xFF80..0xFFFF clamp to 0xFF).

    Reference: vllm_wlq/linear_method.py:306-308, :519-521, :784-786.
    """
    v = np.asarray(u16).astype(np.uint16).astype(np.int64)
    return np.clip((v + 0x80) >> 8, 0, 255).astype(np.uint8)


def e5m2_to_fp16_bits(u8: np.ndarray) -> np.ndarray:
    """e5m2 byte -> fp16 bits ``u8 << 8``. Reference: csrc/gemv_kernel.cu:273,
    csrc/gemm_kernel.cu:223,440."""
    return (np.asarray(u8).astype(np.uint16) << np.uint16(8)).astype(np.uint16)


def e5m2_to_float(u8: np.ndarray) -> np.ndarray:
    return e5m2_to_fp16_bits(u8).view(np.float16).astype(np.float64)


# ---------------------------------------------------------------------------
# Chunked CSR outliers
# ---------------------------------------------------------------------------


def build_chunk_csr(mask: np.ndarray, values: Optional[np.ndarray], chunk_m: int):
    """Dense outlier mask -> chunk CSR.

    offsets int32 [N, nch+1]: global prefix sums in row-major (row, chunk) order;
    cols uint16: column within the chunk (k % chunk_m), ascending inside a chunk;
    vals uint8: e5m2 bytes in np.nonzero (row-major) order; fp16 input is converted
    with fp16_bits_to_e5m2.

    Restates vllm_wlq/linear_method.py:284-312 with an explicit per-row/per-chunk
    walk instead of bincount/cumsum.
    """
    mask = np.asarray(mask, dtype=bool)
    N, K = mask.shape
    nch = -(-K // chunk_m)
    offsets = np.zeros((N, nch + 1), dtype=np.int64)
    cols_list = []
    running = 0
    for n in range(N):
        offsets[n, 0] = running
        nz = np.flatnonzero(mask[n])
        ch = nz // chunk_m
        for c in range(nch):
            sel = nz[ch == c]
            cols_list.append((sel % chunk_m).astype(np.uint16))
            running += sel.size
            offsets[n, c + 1] = running
    cols = np.concatenate(cols_list) if cols_list else np.zeros(0, np.uint16)
    if values is None:
        vals = np.zeros(cols.size, dtype=np.uint8)
    else:
        values = np.asarray(values)
        if values.dtype == np.float16:
            vals = fp16_bits_to_e5m2(values.view(np.uint16))
        else:
            vals = values.astype(np.uint8)
    if offsets.max(initial=0) > np.iinfo(np.int32).max:
        raise OverflowError("chunk offsets exceed int32")
    return offsets.astype(np.int32), cols.astype(np.uint16), vals


def csr_to_coo(offsets: np.ndarray, cols: np.ndarray, chunk_m: int):
    """Expand chunk CSR to (entry index, row, global column) in storage order.

    Entries of (row n, chunk c) are cols[offsets[n,c] : offsets[n,c+1]] and sit in
    columns c*chunk_m + cols[e] (csrc/gemv_kernel.cu:263-276, csrc/gemm_kernel.cu:431-437).
    """
    offsets = np.asarray(offsets).astype(np.int64)
    cols = np.asarray(cols)
    N, nchp1 = offsets.shape
    ent, rows, gcols = [], [], []
    for n in range(N):
        for c in range(nchp1 - 1):
            s, e = int(offsets[n, c]), int(offsets[n, c + 1])
            if e > s:
                idx = np.arange(s, e, dtype=np.int64)
                ent.append(idx)
                rows.append(np.full(e - s, n, dtype=np.int64))
                gcols.append(c * chunk_m + cols[s:e].astype(np.int64))
    if not ent:
        z = np.zeros(0, dtype=np.int64)
        return z, z, z
    return np.concatenate(ent), np.concatenate(rows), np.concatenate(gcols)


# ---------------------------------------------------------------------------
# Dequantization
# ---------------------------------------------------------------------------


def dequant(q, lut, N: int, K: int, bits: int, offsets=None, cols=None, vals=None,
            group_size: int = 0) -> np.ndarray:
    """W0[n,k] = lut[n, g(k), code(n,k)] as an fp16 bit copy, then outliers
    overwrite: W0[n, c*C + col] = fp16 bits (u8 << 8) for every CSR entry with
    column < K.

    Reference: csrc/gemm_kernel.cu:322-445 (per-row LUT, group_size 0) and
    vllm_wlq/linear_method.py:881-888 (torch.gather + masked overwrite).  The
    group-LUT form lut[n, k // group_size, code] is this build's extension; with
    group_size 0 or >= K it is exactly the reference.  Returns float16 [N, K].
    """
    codes = unpack_row_aligned(q, N, K, bits).astype(np.int64)
    lut = np.asarray(lut)
    ncb = 1 << bits
    ng = num_groups(K, group_size)
    lut_bits = lut.view(np.uint16) if lut.dtype == np.float16 else np.asarray(lut, dtype=np.uint16)
    lut_bits = lut_bits.reshape(N, ng, -1)
    if lut_bits.shape[2] < ncb:
        raise ValueError("LUT narrower than 2**bits")
    g = np.zeros(K, dtype=np.int64) if group_size <= 0 else np.arange(K) // group_size
    W = lut_bits[np.arange(N)[:, None], g[None, :], codes]
    if offsets is not None and cols is not None and vals is not None and np.asarray(cols).size > 0:
        C = chunk_width(bits)
        ent, rows, gcols = csr_to_coo(offsets, cols, C)
        ok = gcols < K
        W[rows[ok], gcols[ok]] = e5m2_to_fp16_bits(np.asarray(vals)[ent[ok]])
    return W.astype(np.uint16).view(np.float16)


def outlier_delta(q, lut, N: int, K: int, bits: int, offsets, cols, vals, group_size: int = 0):
    """Per CSR entry (storage order): its global column and the fp32 correction
    delta_w = fp32(fp16 bits (u8 << 8)) - fp32(lut[n, g(col), code(n, col)]) of the
    reference GEMV's outlier pass (csrc/gemv_kernel.cu:268-286); entries with
    column >= K are dropped there (`col < M`), here they get delta 0 and the
    chunk's first column.  Returns (gcol int64 [nnz], delta float32 [nnz])."""
    cols = np.asarray(cols)
    nnz = cols.size
    gcol = np.zeros(nnz, dtype=np.int64)
    delta = np.zeros(nnz, dtype=np.float32)
    if nnz == 0:
        return gcol, delta
    C = chunk_width(bits)
    ent, rows, gc = csr_to_coo(offsets, cols, C)
    codes = unpack_row_aligned(q, N, K, bits).astype(np.int64)
    ng = num_groups(K, group_size)
    lut16 = np.asarray(lut).view(np.uint16).reshape(N, ng, -1).view(np.float16)
    ok = gc < K
    gcol[ent] = np.where(ok, gc, (gc // C) * C)
    okc = np.where(ok, gc, 0)
    g = np.zeros_like(okc) if group_size <= 0 else np.minimum(okc // group_size, ng - 1)
    w_true = e5m2_to_fp16_bits(np.asarray(vals)[ent]).view(np.float16).astype(np.float32)
    w_lut = lut16[rows, g, codes[rows, okc]].astype(np.float32)
    delta[ent] = np.where(ok, w_true - w_lut, np.float32(0.0)).astype(np.float32)
    return gcol, delta


# ---------------------------------------------------------------------------
# Elias-Fano outlier masks
# ---------------------------------------------------------------------------


def _ef_low_bits(U: int, m: int) -> int:
    """L = max(0, floor(log2(U/m))). Reference: vllm_wlq/linear_method.py:212,263;
    csrc/vllm_binding.cpp:140-144."""
    if m <= 0:
        return 0
    if U <= m:
        return 0
    return max(0, int(math.floor(math.log2(U / m))))


def ef_encode(mask: np.ndarray, tile_size: int):
    """Textbook Elias-Fano (Elias 1974; Fano 1971) per tile of tile_size^2 cells,
    tiles in row-major tile order, local index row*T+col, low bits LSB-first,
    then unary high parts (a 0 per increment of the high part, a 1 per element).

    Independent encoder used to pin the decoders by round trip; the layout it
    emits is what vllm_wlq/linear_method.py:243-281 consumes.
    Returns (meta int64 [tiles, 2] = (start_bit, m), bitstream uint32).
    """
    mask = np.asarray(mask, dtype=bool)
    H, W = mask.shape
    T = tile_size
    Hp, Wp = -(-H // T) * T, -(-W // T) * T
    padded = np.zeros((Hp, Wp), dtype=bool)
    padded[:H, :W] = mask
    nty, ntx = Hp // T, Wp // T
    U = T * T
    bits: list = []
    meta = np.zeros((nty * ntx, 2), dtype=np.int64)
    for ty in range(nty):
        for tx in range(ntx):
            k = ty * ntx + tx
            tile = padded[ty * T:(ty + 1) * T, tx * T:(tx + 1) * T]
            idx = np.flatnonzero(tile.ravel())  # row-major local index, ascending
            m = idx.size
            meta[k] = (len(bits), m)
            if m == 0:
                continue
            L = _ef_low_bits(U, m)
            for v in idx:
                low = int(v) & ((1 << L) - 1)
                bits.extend((low >> b) & 1 for b in range(L))
            prev = 0
            for v in idx:
                high = int(v) >> L
                bits.extend([0] * (high - prev))
                bits.append(1)
                prev = high
    nwords = max(1, -(-len(bits) // 32))
    arr = np.zeros(nwords * 32, dtype=np.uint8)
    arr[:len(bits)] = bits
    return meta, np.packbits(arr, bitorder="little").view(np.uint32).copy()


def ef_decode_mask(meta: np.ndarray, bitstream: np.ndarray, N: int, K: int, tile_size: int) -> np.ndarray:
    """Decode per-tile EF bitstreams into a dense [N, K] mask.

    Reference: vllm_wlq/linear_method.py:243-281 (numpy fallback) and :201-237
    (numba).  Bit b of the stream is bit (b & 31) of word (b >> 5).
    """
    meta = np.asarray(meta, dtype=np.int64).reshape(-1, 2)
    bs = np.asarray(bitstream).view(np.uint32) if np.asarray(bitstream).dtype == np.int32 else np.asarray(bitstream, dtype=np.uint32)
    T = tile_size
    Hp, Wp = -(-N // T) * T, -(-K // T) * T
    ntx = Wp // T
    U = T * T
    total_bits = bs.size * 32

    def bit(b):
        return (int(bs[b >> 5]) >> (b & 31)) & 1

    out = np.zeros((Hp, Wp), dtype=bool)
    for k in range(meta.shape[0]):
        start, m = int(meta[k, 0]), int(meta[k, 1])
        if m <= 0:
            continue
        L = _ef_low_bits(U, m)
        lows = [sum(bit(start + i * L + j) << j for j in range(L)) for i in range(m)]
        pos = start + m * L
        high = 0
        ty, tx = divmod(k, ntx)
        for i in range(m):
            while pos < total_bits and bit(pos) == 0:
                high += 1
                pos += 1
            pos += 1  # the terminating 1
            local = (high << L) | lows[i]
            r, c = divmod(local, T)
            if r < T and ty * T + r < Hp and tx * T + c < Wp:
                out[ty * T + r, tx * T + c] = True
    return out[:N, :K]


def ef_decode_to_chunk_csr(meta, bitstream, N: int, K: int, tile_size: int, chunk_m: int):
    """(offsets int32 [N, nch+1], cols uint16). Reference: csrc/vllm_binding.cpp:94-196
    (coordinates outside [0,N)x[0,K) are dropped, :163)."""
    mask = ef_decode_mask(meta, bitstream, N, K, tile_size)
    off, cols, _ = build_chunk_csr(mask, None, chunk_m)
    return off, cols


# ---------------------------------------------------------------------------
# DoRA calibration
# ---------------------------------------------------------------------------


def lora_scale(lora_alpha: Optional[float], r_base: int) -> float:
    """s = lora_alpha / r_base, alpha defaulting to r_base.
    Reference: vllm_wlq/linear_method.py:573-575, :858-860."""
    alpha = r_base if lora_alpha is None else lora_alpha
    return float(alpha) / float(r_base)


def merge_dora(A_list: Sequence[np.ndarray], B_list: Sequence[np.ndarray], m_list: Sequence[Optional[np.ndarray]]):
    """Merged projections (qkv, gate_up): A stacked along rank, B block-diagonal,
    magnitudes concatenated (None if any is missing).
    Reference: vllm_wlq/linear_method.py:577-592, :862-877."""
    if len(A_list) == 1:
        return np.asarray(A_list[0], np.float64), np.asarray(B_list[0], np.float64), m_list[0]
    A = np.concatenate([np.asarray(a, np.float64) for a in A_list], axis=0)
    totN = sum(b.shape[0] for b in B_list)
    totR = sum(b.shape[1] for b in B_list)
    B = np.zeros((totN, totR), dtype=np.float64)
    r0 = c0 = 0
    for b in B_list:
        B[r0:r0 + b.shape[0], c0:c0 + b.shape[1]] = b
        r0 += b.shape[0]
        c0 += b.shape[1]
    m = None if any(x is None for x in m_list) else np.concatenate([np.asarray(x, np.float64).ravel() for x in m_list])
    return A, B, m


def dora_gamma(W0: np.ndarray, A: np.ndarray, B: np.ndarray, s: float, m: Optional[np.ndarray] = None) -> np.ndarray:
    """gamma = fp16(m / max(||W0 + s*B@A||_row, 1e-12)); m defaults to ||W0||_row.
    W0 includes the outlier overwrite.  Reference: vllm_wlq/linear_method.py:625-635,
    :890-897 (computed there in fp32; here in fp64)."""
    W = np.asarray(W0).astype(np.float64)
    V = W + s * (np.asarray(B, np.float64) @ np.asarray(A, np.float64))
    norm_v = np.maximum(np.sqrt((V * V).sum(axis=1)), 1e-12)
    if m is None or np.asarray(m).size != W.shape[0]:
        m = np.sqrt((W * W).sum(axis=1))
    return (np.asarray(m, np.float64).ravel() / norm_v).astype(np.float16)


# ---------------------------------------------------------------------------
# Layer forward
# ---------------------------------------------------------------------------


def lora_h(x: np.ndarray, A: np.ndarray) -> np.ndarray:
    """H = fp32(fp16(x @ A^T)): F.linear in fp16 then .float().
    Reference: vllm_wlq/linear_method.py:963,984."""
    x64 = np.asarray(x, np.float16).astype(np.float64)
    A64 = np.asarray(A, np.float16).astype(np.float64)
    return (x64 @ A64.T).astype(np.float16).astype(np.float32)


def linear_forward(x: np.ndarray, W0: np.ndarray, H: Optional[np.ndarray] = None, B: Optional[np.ndarray] = None,
                   gamma: Optional[np.ndarray] = None, s: float = 1.0, round_gemm_output: Optional[bool] = None,
                   return_f64: bool = False):
    """y = fp16((x @ W0^T [+ s * H @ B^T]) * gamma), accumulated in fp64.

    x fp16 [M, K], W0 fp16 [N, K], H fp32 [M, r] (already fp16-rounded as in
    lora_h), B fp16 [N, r], gamma fp16 [N].

    Rounding points follow the reference: the M==1 GEMV and 2<=M<16 fused kernel
    round once (csrc/gemv_kernel.cu:309-317, csrc/gemm_kernel.cu:280-291); the
    M>=16 path rounds x@W0^T to fp16 before the DoRA epilogue rounds again
    (csrc/vllm_binding.cpp:355-393, csrc/gemm_kernel.cu:462-471).
    ``round_gemm_output`` None picks by M; True/False forces it.  DoRA is active
    only when H, B and gamma are all given and r > 0 (csrc/gemv_kernel.cu:440,
    csrc/gemm_kernel.cu:557, csrc/vllm_binding.cpp:381).  Without DoRA the result
    is fp16(x @ W0^T) for every M.
    """
    x64 = np.asarray(x, np.float16).astype(np.float64)
    if x64.ndim == 1:
        x64 = x64[None, :]
    M = x64.shape[0]
    y = x64 @ np.asarray(W0, np.float16).astype(np.float64).T
    has_dora = H is not None and B is not None and gamma is not None and np.asarray(B).ndim == 2 and np.asarray(B).shape[1] > 0
    if round_gemm_output is None:
        round_gemm_output = M >= 16
    if has_dora:
        if round_gemm_output:
            y = y.astype(np.float16).astype(np.float64)
        H64 = np.asarray(H, np.float32).astype(np.float64).reshape(M, -1)
        B64 = np.asarray(B, np.float16).astype(np.float64)
        y = (y + s * (H64 @ B64.T)) * np.asarray(gamma, np.float16).astype(np.float64)[None, :]
    if return_f64:
        return y
    return y.astype(np.float16)


def apply(x: np.ndarray, W0: np.ndarray, A: Optional[np.ndarray] = None, B: Optional[np.ndarray] = None,
          gamma: Optional[np.ndarray] = None, s: float = 1.0, bias: Optional[np.ndarray] = None,
          out_dtype=np.float16):
    """WLQLinearMethod.apply semantics: flatten to [M, K], cast to fp16, H from
    fp16 F.linear, dispatch by M, cast back to the input dtype, then add bias in
    that dtype.  Reference: vllm_wlq/linear_method.py:937-1009.  ``out_dtype`` is
    numpy float16/float32 (bf16 callers compare in float32)."""
    x = np.asarray(x)
    K = W0.shape[1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K).astype(np.float16)
    H = lora_h(x2, A) if A is not None and B is not None and gamma is not None else None
    y = linear_forward(x2, W0, H, B, gamma, s).astype(out_dtype)
    if bias is not None:
        y = (y + np.asarray(bias).astype(out_dtype)).astype(out_dtype)
    return y.reshape(*lead, W0.shape[0])


def rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    """max|y - ref| / max|ref| over the whole output (fp64)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.max(np.abs(ref)) if ref.size else 0.0
    if denom == 0.0:
        return float(np.max(np.abs(y - ref))) if y.size else 0.0
    return float(np.max(np.abs(y - ref)) / denom)
