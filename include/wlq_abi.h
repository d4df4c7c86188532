/*
 * wlq_abi.h -- C ABI of the MI355X (gfx950) WLQ metalog-LUT quantized linear layer.
 *
 * Library: qwen_wlqfastshot_helen_beta_amd/libwlq_hip.so
 *
 * Every entry point takes plain pointers and sizes (no framework types).  fp16
 * buffers are IEEE binary16 passed as void*.  Device entry points are
 * asynchronous on `stream` and never synchronize; host entry points run on
 * the calling CPU thread.  All return an int status (WLQ_OK on success); the
 * message of the last failure on the calling thread is wlq_last_error().
 *
 * Data layouts (identical to the reference's, vllm_wlq/linear_method.py:284-338):
 *   q_packed      int32 [N * wpr], code (n,k) at word n*wpr + k/spw, bit (k%spw)*bits,
 *                 spw = 10 for 3-bit else 32/bits, wpr = words_per_row(K, bits)
 *   lut_c         fp16 [N, 2^bits] (group_size 0) or [N, ceil(K/G), 2^bits] (group_size G)
 *   chunk_offsets int32 [N, nch+1], chunk_cols uint16 [nnz], chunk_vals uint8 [nnz] (e5m2),
 *                 chunk width 512 (640 for 3-bit), nch = ceil(K / chunk width)
 *   DoRA          lora_B fp16 [N, r], lora_h / lora_H fp32 [M, r], dora_gamma fp16 [N]
 *
 * Optional operands: the outlier correction runs only when chunk_offsets,
 * chunk_cols and chunk_vals are all non-null; the DoRA epilogue only when
 * lora_B and dora_gamma are non-null, r > 0 and H is available (as in the
 * reference, csrc/gemv_kernel.cu:440, csrc/gemm_kernel.cu:557).  H is either
 * passed (lora_h / lora_H, fp32) or, when that pointer is null and lora_A
 * (fp16 [r, K]) is given, computed here as fp32(fp16(x . lora_A^T)) -- the
 * reference caller's F.linear in fp16 followed by .float()
 * (vllm_wlq/linear_method.py:963,984) -- inside the product kernel for r <= 64
 * (prepared layout: M <= 128; row layout: M <= 32), else by a separate kernel
 * before the product.
 *
 * group_size: 0 = one LUT per output row (the reference).  Otherwise a
 * multiple of 32 columns, at least the code window (32/40/64/128 columns for
 * 4/3/2/1 bits) and below 4096; a group_size >= K is the per-row case.
 *
 * Workspace: its first 16 KiB hold arrival counters (the block of the decode
 * kernel that finishes last for a group of 64 output rows applies the
 * epilogue, so no second kernel is needed); the rest holds split-K partial sums
 * (fp32) and, when H is computed from lora_A, its partial sums.  ZERO-FILL A
 * WORKSPACE ONCE AFTER ALLOCATING IT (e.g. hipMemset): the counters must start
 * at zero, and every call leaves them zero again.  Pass the buffer and its
 * size; when it is smaller than wlq_gemm_workspace_bytes() the split count is
 * reduced to what fits.  No workspace is valid unless H has to be computed
 * from lora_A (then WLQ_ERR_CAPACITY reports the minimum).  Calls that share
 * one workspace must be ordered on one stream.
 *
 * Failed hand-offs are reported, not hidden: a kernel that finds a counter beyond
 * what one call can reach (the area was not zero at entry, e.g. two unordered
 * calls on one workspace) or whose wait for the fused DoRA H runs out of polls
 * (~1 s) sets a sticky error word at the end of the counter area and writes the
 * rows concerned as fp16 NaN.  While the word is set every call on the
 * workspace writes NaN rows.  wlq_workspace_status reports it, and
 * wlq_workspace_reset clears the counter area.
 */
#ifndef WLQ_ABI_H
#define WLQ_ABI_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WLQ_ABI_VERSION 5

enum wlq_status {
  WLQ_OK = 0,
  WLQ_ERR_NULL_POINTER = 1, /* a required pointer is null */
  WLQ_ERR_BAD_SHAPE = 2,    /* negative/oversized size or inconsistent words_per_row */
  WLQ_ERR_UNSUPPORTED = 3,  /* bits or group_size outside the supported set */
  WLQ_ERR_CAPACITY = 4,     /* an output buffer is too small */
  WLQ_ERR_HIP = 5,          /* the HIP runtime reported an error */
  WLQ_ERR_FORMAT = 6,       /* malformed input stream */
  WLQ_ERR_SYNC = 7          /* a cross-block hand-off on a workspace failed (see wlq_workspace_status) */
};

int wlq_abi_version(void);
const char* wlq_status_string(int status);
const char* wlq_last_error(void);

/* Words per packed row: 4 * ceil(ceil(K / spw) / 4).
 * Reference: vllm_wlq/linear_method.py:329-330, csrc/vllm_binding.cpp:209-210. */
int64_t wlq_words_per_row(int64_t K, int32_t bits);

/* Outlier chunk width: 640 for 3-bit, else 512. Reference: csrc/vllm_binding.cpp:279,351. */
int32_t wlq_chunk_width(int32_t bits);

/* Workspace bytes wlq_gemm (M rows) would like on `device` for DoRA rank r
 * (r = 0: no DoRA, or H passed by the caller).  wlq_gemv uses M = 1. */
size_t wlq_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t bits, int32_t r, int32_t device);

/* Decode product, one activation row: out[N] = fp16((x . W0^T + s * lora_h . lora_B^T) * gamma).
 * Replaces launch_gemv_chunk_csr (csrc/gemv_kernel.cu:396-457; declared at
 * csrc/vllm_binding.cpp:10-29), whose caller passes M(=K) and num_chunks and a
 * workspace it owns; here num_chunks is derived from K and bits. */
int wlq_gemv(const int32_t* q_packed, const void* lut_c, const void* x, void* out,
             const int32_t* chunk_offsets, const uint16_t* chunk_cols, const uint8_t* chunk_vals,
             const void* lora_B, const float* lora_h, const void* dora_gamma, const void* lora_A,
             float lora_scale, int32_t r, int64_t N, int64_t K, int32_t bits, int32_t group_size,
             void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Product for M activation rows: out[M, N] = fp16((X . W0^T + s * lora_H . lora_B^T) * gamma).
 * Replaces both branches of gemm_forward (csrc/vllm_binding.cpp:318-419): the
 * fused small-M kernel launch_gemm_metalog_dora (csrc/gemm_kernel.cu:527-596,
 * declared csrc/vllm_binding.cpp:31-52) and the M >= 16 sequence
 * dequant -> at::mm_out -> launch_fused_dora_epilogue.  M <= 32 runs the
 * weight-streaming MFMA kernel, larger M the LDS-staged MFMA GEMM.
 * words_per_row must equal wlq_words_per_row(K, bits). */
int wlq_gemm(const void* X, const int32_t* q_packed, const void* lut_c, void* out,
             int64_t M, int64_t N, int64_t K, int32_t bits, int64_t words_per_row, int32_t group_size,
             const int32_t* chunk_offsets, const uint16_t* chunk_cols, const uint8_t* chunk_vals,
             const float* lora_H, const void* lora_B, const void* dora_gamma, const void* lora_A,
             float lora_scale, int32_t r, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Host: wait for `stream`, then read the workspace's sticky error word.  WLQ_OK
 * when no hand-off failed on it (also when workspace_bytes is below the 16 KiB
 * counter area, which then holds no counters), else WLQ_ERR_SYNC with the failure
 * in wlq_last_error().  Synchronizes: not for use inside graph capture.
 * No reference counterpart: the reference's split-K reduce is a second kernel with no
 * cross-block waits (csrc/gemv_kernel.cu:322-353, :449-456). */
int wlq_workspace_status(const void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Device: zero the workspace's counter area (counters and error word) on `stream`
 * with a fill kernel (graph-safe, no hipMemset).  Use once after allocating a
 * workspace, or after wlq_workspace_status reported WLQ_ERR_SYNC and the calls
 * that used the workspace have finished.  No reference counterpart (see above);
 * it takes the place of the reference's zero-initialised workspace tensors
 * (csrc/vllm_binding.cpp:238-251). */
int wlq_workspace_reset(void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Bytes of the prepared (tile-contiguous) layout of a layer, or 0 when the
 * layer has none (it needs 4-bit or 3-bit codes, a per-row LUT or a group size that is a
 * multiple of 32, K % 8 == 0 and K < 65536).  nnz = number of outlier entries.
 * No reference counterpart: the reference streams its row-aligned layout
 * directly (csrc/gemv_kernel.cu:168-190); this layout is built once at load
 * time, like the reference's own row-aligned repack (csrc/vllm_binding.cpp:198-236),
 * so that the decode kernel reads whole 1 KB wave tiles. */
size_t wlq_prepared_bytes(int64_t N, int64_t K, int32_t bits, int32_t group_size, int64_t nnz);

/* Device: build the prepared layout from the reference-format tensors into
 * `prepared` (256-byte aligned, wlq_prepared_bytes() bytes): codes in 16-row x
 * 128-column tiles in MFMA lane order (3-bit codes widened to 4-bit nibbles, their
 * 8-entry LUTs zero-padded to 16), LUT byte planes per 16-row tile, and per
 * outlier its column and the fp32 delta fp16(e5m2 << 8) - lut[code] of the
 * reference's GEMV outlier correction (csrc/gemv_kernel.cu:262-288), and the
 * outliers once more as overwrite patches grouped by (16-row tile, 128-column slab)
 * for the M = 9..128 kernel. */
int wlq_prepare(const int32_t* q_packed, const void* lut_c, int64_t N, int64_t K, int32_t bits, int32_t group_size,
                const int32_t* chunk_offsets, const uint16_t* chunk_cols, const uint8_t* chunk_vals, int64_t nnz,
                void* prepared, size_t prepared_bytes, hipStream_t stream);

/* wlq_gemm with the layer's prepared layout: M <= 8 runs the streaming decode
 * kernel on `prepared` (plus the reference chunk offsets) where its activation
 * staging fits, M = 9..128 the kernel that streams the activations through LDS
 * slab by slab, M = 129..1024 on wide layers with M mod 256 in 1..128 the kernel that
 * dequantizes W in registers, every other case the MFMA GEMM; all of them read the
 * prepared codes, LUT planes and outlier patch lists.  The reference-format tensors
 * stay required (unaligned activations and other fallbacks run the row-layout kernels).
 * Replaces the same reference launchers as wlq_gemm / wlq_gemv
 * (csrc/vllm_binding.cpp:10-52, :318-419). */
int wlq_gemm_prepared(const void* X, const int32_t* q_packed, const void* lut_c, const void* prepared,
                      size_t prepared_bytes, void* out, int64_t M, int64_t N, int64_t K, int32_t bits,
                      int64_t words_per_row, int32_t group_size, const int32_t* chunk_offsets,
                      const uint16_t* chunk_cols, const uint8_t* chunk_vals, int64_t nnz, const float* lora_H,
                      const void* lora_B, const void* dora_gamma, const void* lora_A, float lora_scale, int32_t r,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* wlq_gemm_prepared without a workspace argument, for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): it allocates nothing and calls no allocating routine.  No counterpart in
 * the reference.  Its kernels use the library's own scratch instead: a 16 MiB device
 * array per GPU (a file-scope __device__ array, held until the process ends), counter
 * area first.  A call whose decode plan needs more than that (e.g. the 37888-row
 * gate_up projection at M >= 16, whose K splits write fp32 partials of M * N * splits)
 * returns WLQ_ERR_CAPACITY without launching anything; M > 32 runs the GEMM with the
 * split count the scratch allows.  Every call on a GPU shares that GPU's scratch: calls
 * that overlap in time on one GPU (different streams, or threads without ordering) race
 * and must not be issued.  The scratch's counters are left zero by every call; a failed
 * hand-off (see the workspace notes above) leaves this GPU's scratch poisoned (NaN rows)
 * for the rest of the process. */
int wlq_gemm_prepared_noalloc(const void* X, const int32_t* q_packed, const void* lut_c, const void* prepared,
                              size_t prepared_bytes, void* out, int64_t M, int64_t N, int64_t K, int32_t bits,
                              int64_t words_per_row, int32_t group_size, const int32_t* chunk_offsets,
                              const uint16_t* chunk_cols, const uint8_t* chunk_vals, int64_t nnz,
                              const float* lora_H, const void* lora_B, const void* dora_gamma, const void* lora_A,
                              float lora_scale, int32_t r, hipStream_t stream);

/* Bit-exact W_out[N, K] (fp16) = lut[n, g(k), code(n, k)], outliers overwritten with e5m2 << 8.
 * Replaces launch_dequant_patch_metalog (csrc/gemm_kernel.cu:475-503, declared
 * csrc/vllm_binding.cpp:54-68). */
int wlq_dequant(const int32_t* q_packed, const void* lut_c, void* W_out, int64_t N, int64_t K, int32_t bits,
                int64_t words_per_row, int32_t group_size, const int32_t* chunk_offsets,
                const uint16_t* chunk_cols, const uint8_t* chunk_vals, hipStream_t stream);

/* In place: out[M, N] = fp16((out + s * lora_H . lora_B^T) * gamma).
 * Replaces launch_fused_dora_epilogue (csrc/gemm_kernel.cu:505-525, declared
 * csrc/vllm_binding.cpp:70-80). */
int wlq_dora_epilogue(void* out, const float* lora_H, const void* lora_B, const void* dora_gamma,
                      float lora_scale, int32_t r, int64_t M, int64_t N, hipStream_t stream);

/* Host: continuous (on-disk) packing -> row-aligned packing; symbols past the
 * end of src read as 0.  dst must hold N * wlq_words_per_row(K, bits) words.
 * Replaces repack_q_indices_row_aligned_cpp (csrc/vllm_binding.cpp:198-236). */
int wlq_repack_row_aligned(const uint32_t* src, int64_t src_words, int64_t N, int64_t K, int32_t bits,
                           uint32_t* dst, int64_t dst_words);

/* Host: number of outliers an Elias-Fano tile stream declares (sum of m over
 * tiles), an upper bound for wlq_ef_decode_chunk_csr's cols capacity. */
int64_t wlq_ef_total(const int64_t* tile_meta, int64_t num_tiles);

/* Host: Elias-Fano tile stream -> chunk CSR (offsets [N, nch+1], cols).
 * tile_meta int64 [num_tiles, 2] = (start_bit, m), tiles row-major over the
 * K-padded grid of tile_size x tile_size cells.  Coordinates outside
 * [0,N) x [0,K) are dropped; *nnz_out receives the number written to cols.
 * Replaces decode_ef_to_chunk_csr_cpp (csrc/vllm_binding.cpp:94-196). */
int wlq_ef_decode_chunk_csr(const int64_t* tile_meta, int64_t num_tiles, const uint32_t* bitstream,
                            int64_t stream_words, int64_t N, int64_t K, int64_t tile_size, int64_t chunk_m,
                            int32_t* offsets, uint16_t* cols, int64_t cols_capacity, int64_t* nnz_out);

#ifdef __cplusplus
}
#endif

#endif /* WLQ_ABI_H */
