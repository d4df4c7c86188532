// Internal (C++) launch interface between the C ABI layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace wlq {

// One quantized layer as the kernels see it (all device pointers).
struct Layer {
  const uint32_t* q;        // [N * wpr] row-aligned codes
  const uint16_t* lut;      // fp16 bits [N, ng, 2^bits]
  const int32_t* offsets;   // [N, nch + 1] or nullptr (no outliers)
  const uint16_t* cols;     // [nnz]
  const uint8_t* vals;      // [nnz] e5m2 bytes
  int N, K, bits, wpr;
  int group_size;           // 0: one LUT per row
  int ng;                   // LUT groups per row
  int nch, chunk;           // outlier chunks per row and chunk width
};

// DoRA epilogue operands: y = (acc + scale * H[i,:] . B[n,:]) * gamma[n].
// H is given by the caller, or computed from A as fp16(x . A^T) when H is null.
struct Dora {
  const uint16_t* B;        // fp16 [N, r]
  const float* H;           // fp32 [M, r] or nullptr
  const uint16_t* gamma;    // fp16 [N]
  const uint16_t* A;        // fp16 [r, K] (lora_A) or nullptr
  float scale;
  int r;                    // 0 disables the epilogue
};

struct SplitPlan {
  int splits;               // blocks along K
  int slabs_per_split;      // K range per block, in slabs
  int seg_slabs;            // activation staging segment, in slabs
  size_t workspace_bytes;   // fp32 partials (0 when splits == 1) + aux_bytes
  size_t aux_bytes;         // GEMM: prepared outlier entries after the partials (0: not used)
};

// The first kSyncBytes of a caller's workspace hold arrival counters of the decode
// kernel (one 32-bit word per 64-row block).  They must be zero before the first call
// on a workspace and every call leaves them zero.  Products, H and partials use the
// bytes after them.
constexpr size_t kSyncBytes = 16384;
constexpr int kSyncWords = (int)(kSyncBytes / 4);
// The area's last 128-byte line holds the sticky error word (the counters use the words
// before it).  A kernel that detects a failed hand-off ORs one of the kErr* bits into it
// and writes the rows concerned as fp16 NaN; later calls on the workspace see the word
// and write NaN too, until wlq_workspace_reset clears the area.
constexpr int kSyncErrorWord = kSyncWords - 32;
constexpr int kMaxSyncRowBlocks = kSyncErrorWord;
// Counter words of the streaming kernels (decode and wide), all zero between calls:
constexpr int kSyncDora = 0;      // DoRA blocks arrived (reset by the last of them)
constexpr int kSyncSlot0 = 64;    // H ready slots: word 0 = H published, word 1 = consumers counted
constexpr int kSlotWords = 16;    // one 64-byte line per slot
constexpr int kMaxSlots = 128;    // tile block tb uses slot tb % min(TB, kMaxSlots)
constexpr int kSyncTile = kSyncSlot0 + kSlotWords * kMaxSlots;  // [TB] split arrivals per tile block
constexpr uint32_t kErrHTimeout = 1u;   // a wait for the DoRA H ran out of polls
constexpr uint32_t kErrArrivals = 2u;   // an arrival count exceeded what one call makes
constexpr uint32_t kDefaultSpinLimit = 1u << 24;  // ~1 s of polls

// Polls of a ready slot before a wait gives up (default kDefaultSpinLimit), and the
// test hook that keeps the DoRA finisher from raising its ready slots.  Both come from
// the environment only when WLQ_TEST_HOOKS=1 was set when the library first ran a
// product (WLQ_SPIN_LIMIT, WLQ_TEST_WITHHOLD_H, read on every call then).
uint32_t spin_limit();
bool withhold_h();
// Test hook (WLQ_TEST_FORCE_PREFILL=1 with the hooks on): M > 128 products on a prepared layer take
// the prefill kernel wherever it can run, not only where it is the faster choice.
bool force_prefill();

int slab_cols(int bits);             // columns one 16-row wave tile covers per step
int skinny_max_m();
int skinny_max_fused_rank();         // largest DoRA rank whose H the decode kernel computes itself
// fused_rank > 0: H will be computed from lora_A inside the decode product.
SplitPlan plan_skinny(const Layer& L, int M, int cu_count, size_t workspace_bytes, int fused_rank);
// sync: the workspace's arrival counters, or nullptr (a finalize kernel then finishes).
hipError_t launch_skinny(const Layer& L, const Dora& D, const uint16_t* x, uint16_t* out, int M,
                         const SplitPlan& plan, float* workspace, uint32_t* sync, hipStream_t stream);

// A layer's prepared buffer as the GEMM reads it: codes and LUT planes (per 16-row tile and
// 128-column slab) in place of the row-layout tensors, and the outlier patch lists in place of
// per-call outlier records.
struct PatchLists {
  const uint32_t* codes;    // u32x4 [T][S][64]
  const uint32_t* planes;   // u32x4 [T][ng][2][16]
  const uint32_t* wpidx;    // [T * S + 1] list starts
  const uint32_t* wpatch;   // [nnz] patches
  int64_t nnz;
  int T, S, ng;
};
// lists: the GEMM takes the layer's outliers from prepared patch lists (no per-call records)
SplitPlan plan_gemm(const Layer& L, int M, int cu_count, size_t workspace_bytes, bool lists = false);
hipError_t launch_gemm(const Layer& L, const Dora& D, const uint16_t* X, uint16_t* out, int M,
                       const SplitPlan& plan, float* workspace, hipStream_t stream,
                       const PatchLists* lists = nullptr);

hipError_t launch_dequant(const Layer& L, uint16_t* W, hipStream_t stream);

// Prepared (tile-contiguous) layout of a 4-bit or 3-bit layer for the streaming decode kernel
// (wlq_stream.hip): byte offsets of its four parts inside one buffer.
struct PreparedLayout {
  int T, S, ng;             // row tiles of 16, slabs of 128 columns, LUT groups per row
  size_t codes_off, planes_off, gcol_off, delta_off, wpidx_off, wpatch_off, bytes;
};
bool prepared_supported(int N, int K, int bits, int group_size);
PreparedLayout prepared_layout(int N, int K, int group_size, int64_t nnz);
hipError_t launch_prepare(const Layer& L, int64_t nnz, void* prepared, hipStream_t stream);

struct StreamPlan {
  int tpb;                  // row tiles per block (1, 2 or 4)
  int TB, splits, cps;      // tile blocks, K splits, outlier chunks per split
  int h_blocks;             // DoRA blocks when H is computed in the kernel
  size_t hfin_off, hpart_off, partial_off, workspace_bytes;
  bool ok;
};
int stream_max_m();
int stream_max_rank();
StreamPlan plan_stream(int N, int K, int M, int cu_count, int fused_rank, int chunk);  // chunk: outlier chunk width
hipError_t launch_stream(const Layer& L, const void* prepared, int64_t nnz, const Dora& D, const uint16_t* x,
                         uint16_t* out, int M, const StreamPlan& plan, float* workspace, uint32_t* sync,
                         hipStream_t stream);

// Product for 8 < M <= wide_max_m() on the prepared layout (wlq_wide.hip): activations streamed
// through LDS slab by slab, outliers overwritten in the dequantized words.
struct WidePlan {
  int tpw;                  // 16-row W tiles per compute wave (1, or 2 at 128 activation rows)
  int TB, splits, sps;      // tile blocks (64 tpw rows), K splits, 128-column slabs per split
  int h_blocks;             // DoRA blocks (each a share of the columns, all activation rows)
  size_t hfin_off, hpart_off, partial_off, workspace_bytes;
  size_t lds;               // dynamic LDS bytes per block
  bool ok;
};
int wide_max_m();
// rank: DoRA rank of the epilogue (0: none); fused_rank: rank when H is computed in the kernel.
WidePlan plan_wide(int N, int K, int M, int cu_count, int rank, int fused_rank, int chunk, bool csr);
hipError_t launch_wide(const Layer& L, const void* prepared, int64_t nnz, const Dora& D, const uint16_t* x,
                       uint16_t* out, int M, const WidePlan& plan, float* workspace, uint32_t* sync,
                       hipStream_t stream);

// Product for M >= prefill_min_m() on the prepared layout (wlq_prefill.hip): W dequantized in
// registers into 32x32x16 MFMA operands, activations double-buffered through LDS, block tiles of
// 128 activation rows x 256 W rows.  Per-row LUTs or LUT groups of 128 << g columns.
struct PrefillPlan {
  int nblk, mblk, tiles;    // W blocks (256 rows), activation blocks (128 rows), output tiles
  int splits, sps;          // K splits, 128-column slabs per split
  int hk, h_blocks;         // DoRA shares per activation block, DoRA blocks
  int per_xcd, grid;        // tile blocks per XCD, grid size
  size_t hfin_off, hpart_off, partial_off, workspace_bytes;
  size_t lds;
  bool ok;                  // the kernel can run the product
  bool preferred;           // ... and is the faster choice (measured; otherwise the MFMA GEMM)
};
int prefill_min_m();
PrefillPlan plan_prefill(int N, int K, int M, int group_size, int cu_count, int rank, int fused_rank, int chunk);
hipError_t launch_prefill(const Layer& L, const void* prepared, int64_t nnz, const Dora& D, const uint16_t* x,
                          uint16_t* out, int M, const PrefillPlan& plan, float* workspace, uint32_t* sync,
                          hipStream_t stream);

// out = fp16_rn(sum of fp32 split-K partials [splits, M, N]) (epilogue already applied).
hipError_t launch_splitk_sum(const float* partial, int splits, int M, int N, uint16_t* out, hipStream_t stream);

// Decode finish: sum split partials, round the DoRA H (from hpart partial sums
// over h_blocks column blocks, or D.H) and apply the epilogue.
hipError_t launch_finalize(const float* partial, int splits, int M, int N, const Dora& D, const float* hpart,
                           int h_blocks, uint16_t* out, hipStream_t stream);

// H[M, r] = fp32(fp16(X . A^T)) (the reference's F.linear in fp16, then .float()).
// H = fp32(fp16(X A^T)); part: room for K-chunk parts (lora_h_part_bytes), or null
size_t lora_h_part_bytes(int M, int K, int r, int cu_count);
hipError_t launch_lora_h(const uint16_t* X, const uint16_t* A, int M, int K, int r, float* H, float* part,
                         size_t part_bytes, int cu_count, hipStream_t stream);

// In-place epilogue on an fp16 output (the reference's separate pass).
hipError_t launch_dora_epilogue(uint16_t* out, int M, int N, const Dora& D, hipStream_t stream);

}  // namespace wlq
