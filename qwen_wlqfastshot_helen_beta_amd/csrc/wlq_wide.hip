// Product for M = 9..128 activation rows on the prepared (tile-contiguous) layout.
//
// Reference behaviour replaced: the M >= 16 branch of gemm_forward
// (csrc/vllm_binding.cpp:355-393: dequant into a workspace, at::mm_out, fused DoRA
// epilogue) and gemm_metalog_dora_kernel for 9 <= M < 16 (csrc/gemm_kernel.cu:32-294).
// Same arithmetic: W0 expanded through the LUTs with outliers overwritten by
// fp16(e5m2 << 8) (csrc/gemm_kernel.cu:204-228), y = fp16((x.W0^T + s * H.B^T) * gamma)
// rounded once (the reference rounds x.W0^T to fp16 first for M >= 16; both are within
// the tolerance of the tests).
//
// Why a second streaming kernel.  The decode kernel (wlq_stream.hip) stages a block's
// activations for its whole K range up front; at M = 16..32 that staging limits a K
// split to one or two outlier chunks, so blocks do little work per byte of activation.
// Here the activations stream through LDS one 128-column slab at a time, so every
// block covers a long K range whatever M is.
//
// Block = 4 compute waves + 1 loader wave (320 threads).
//  * Compute wave w owns 16-row W tile t = 4 tb + w: its slabs stream from the
//    prepared layout into registers kPF slabs ahead (one 1 KB load of codes and the
//    LUT planes per slab), are dequantized (dequant_word4s) and feed
//    V_MFMA_F32_16X16X32_F16 for every 16-row group of activations (B = W rows,
//    A = activation rows read from the slab's LDS buffer).
//  * The loader wave copies activation slabs into 3..6 LDS buffers with
//    buffer_load_dwordx4 ... lds, 2..5 slabs ahead; rows >= M and columns >= K read as
//    zeros through the buffer range check.  Its loads are in its own wait counter,
//    so the compute waves' in-order waits only ever cover W.  Each slab buffer's
//    16-byte units are XOR-swizzled by row (unit u of row i at u ^ (i % 16)) so the 16
//    rows of an MFMA fragment read hit distinct banks.
//  * Outliers (W0 overwritten): the prepared layout holds them as patch lists per
//    (16-row tile, slab) -- (operand lane, column of the lane's 32, e5m2 byte) -- and
//    the loader wave copies the four tiles' lists of each slab into LDS next to the
//    activations.  A compute wave stores its dequantized words to a wave-private LDS
//    scratch, each of its lanes applies one patch of the list (a 2-byte store into the
//    target lane's words), and the words are read back as the MFMA operand: two LDS
//    round trips per slab with outliers, independent of M.
//  * One s_barrier (without a memory fence: the compute waves' W loads stay in flight)
//    per slab hands the activation buffer and the patch lists over; the loader waits
//    for its own copies (vmcnt) and header stores (lgkmcnt) before it.
//
// Completion, DoRA H and failure handling follow the decode kernel: K splits hand fp32
// partials to the block that counts the last arrival on its tile block; H is computed
// by DoRA blocks (x.A^T partials per 512 columns and 32 activation rows) at the front of
// the grid, published through the ready slots; a failed hand-off sets the workspace's
// sticky error word and the rows are written as NaN.
#include <algorithm>

#include "wlq_device.h"
#include "wlq_internal.h"

namespace wlq {
namespace {

constexpr int kCW = 4;                     // compute waves per block
constexpr int kThreads = 64 * (kCW + 1);   // + the loader wave
constexpr int kPF = 4;                     // W slabs in flight per compute wave
constexpr int kPatchCap = 64;              // patches per (slab buffer, compute wave) in LDS
constexpr int kEpiStride = 72;             // fp16 per LDS row of the epilogue (64 + 8: rows 36 banks apart)
constexpr int kSc1 = 16;                   // buffer cache-policy bit sc1: device-coherent (as agent-scope atomics)
// activation slab buffers by activation rows (the loader runs one fewer slabs ahead)
constexpr int xbufs(int MB) { return MB <= 16 ? 6 : MB <= 32 ? 4 : 3; }
constexpr int kMaxSlabs = 127;             // slabs per K split (patch-list starts held in two lane registers)
constexpr int kMaxDoraBlocks = 16;        // DoRA blocks (x.A^T shares) per call
constexpr int kMaxRank = 64;
constexpr uint16_t kHalfNaN = 0x7E00u;
constexpr uint32_t kOutOfRange = 0x80000000u;  // past every buffer resource (sizes < 2^31 bytes)
constexpr int kRsrcWord3 = 0x00020000;         // raw buffer, 32-bit data format

struct WideArgs {
  const u32x4_t* codes;
  const u32x4_t* planes;
  const uint32_t* wpidx;    // patch-list starts per (tile, slab), T * S + 1
  const uint32_t* wpatch;   // patches (null with no outliers)
  uint32_t patch_bytes;     // size of wpatch (the buffer range of the list copies)
  const uint16_t* X;
  uint16_t* out;
  const uint16_t* B;
  const float* H;           // caller's H, or null (DoRA blocks compute it when A is set)
  const uint16_t* gamma;
  const uint16_t* A;
  float scale;
  int r;
  int M, N, K, S, ng, T, TB;
  uint32_t g_magic;
  int gshift;
  int splits, sps;          // K splits, slabs per split
  int h_blocks;             // DoRA blocks (x.A^T shares over strided 32-column steps)
  float* partial;           // [splits][TB][kCW][tiles per wave][MB / 16][64] x 4 fp32 (register layout)
  uint32_t partial_bytes;
  int out_vec;              // 16-byte output stores (N % 8 == 0, out 16-byte aligned)
  float* hpart;             // [h_blocks, M, r]
  float* hfin;              // [M, r]
  uint32_t* sync;
  uint32_t spin_limit;
  int withhold_h;
};

__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_dev(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void raise_error(uint32_t* sync, uint32_t bit) {
  __hip_atomic_fetch_or(sync + kSyncErrorWord, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }
// A workgroup barrier without the memory fence __syncthreads() carries (which would wait for
// every load in flight); LDS ordering is made explicit with lgkmcnt waits where needed.
__device__ __forceinline__ void raw_barrier() {
  compiler_fence();
  __builtin_amdgcn_s_barrier();
  compiler_fence();
}
__device__ __forceinline__ int group_of(int col, uint32_t magic) { return (int)__umulhi((uint32_t)col, magic); }

// s_waitcnt vmcnt(n) for a runtime n (the count is an immediate of the instruction).
__device__ __forceinline__ void wait_vm(int n) {
#define WLQ_VM(k) \
  case k:         \
    asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); \
    break;
  switch (n < 0 ? 0 : n > 63 ? 63 : n) {
    WLQ_VM(0) WLQ_VM(1) WLQ_VM(2) WLQ_VM(3) WLQ_VM(4) WLQ_VM(5) WLQ_VM(6) WLQ_VM(7)
    WLQ_VM(8) WLQ_VM(9) WLQ_VM(10) WLQ_VM(11) WLQ_VM(12) WLQ_VM(13) WLQ_VM(14) WLQ_VM(15)
    WLQ_VM(16) WLQ_VM(17) WLQ_VM(18) WLQ_VM(19) WLQ_VM(20) WLQ_VM(21) WLQ_VM(22) WLQ_VM(23)
    WLQ_VM(24) WLQ_VM(25) WLQ_VM(26) WLQ_VM(27) WLQ_VM(28) WLQ_VM(29) WLQ_VM(30) WLQ_VM(31)
    WLQ_VM(32) WLQ_VM(33) WLQ_VM(34) WLQ_VM(35) WLQ_VM(36) WLQ_VM(37) WLQ_VM(38) WLQ_VM(39)
    WLQ_VM(40) WLQ_VM(41) WLQ_VM(42) WLQ_VM(43) WLQ_VM(44) WLQ_VM(45) WLQ_VM(46) WLQ_VM(47)
    WLQ_VM(48) WLQ_VM(49) WLQ_VM(50) WLQ_VM(51) WLQ_VM(52) WLQ_VM(53) WLQ_VM(54) WLQ_VM(55)
    WLQ_VM(56) WLQ_VM(57) WLQ_VM(58) WLQ_VM(59) WLQ_VM(60) WLQ_VM(61) WLQ_VM(62)
    default:
      asm volatile("s_waitcnt vmcnt(63)" ::: "memory");
  }
#undef WLQ_VM
}

// s_waitcnt vmcnt(C * m) for a runtime 0 <= m < MAXM (C, MAXM compile-time; m above
// MAXM - 1 waits for everything).
template <int C, int MAXM>
__device__ __forceinline__ void wait_copies(int m) {
  static_assert(C * (MAXM - 1) <= 63, "vmcnt holds 6 bits");
#define WLQ_WC(k)                                                       \
  if constexpr (k < MAXM) {                                             \
    if (m == k) {                                                       \
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(C * k) : "memory");       \
      return;                                                           \
    }                                                                   \
  }
  WLQ_WC(1) WLQ_WC(2) WLQ_WC(3) WLQ_WC(4) WLQ_WC(5)
#undef WLQ_WC
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// LDS layout of a tile block (bytes), kTiles = kCW x tiles per wave row tiles of 16 rows.
// Main loop:
//   [0, XB * MB * 256)           activation slab buffers (MB rows x 16 swizzled units)
//   lists: [XB][kTiles][kPatchCap] u32 patches, headers [XB][64] u32: {start, end} of the
//          tiles' lists, then zeros (outliers only; one 64-lane copy each)
//   scratch: [kTiles][4 words][64 lanes][8] fp16 dequantized words (outliers only)
// Epilogue (reuses the front): H as fp16 high / low parts, B rows, gamma, the output tile.
// TPW: W row tiles per compute wave; with two, each activation fragment read from LDS feeds
// two MFMAs (half the LDS traffic per weight) on half as many blocks.
template <int MB, bool CSR, int TPW_>
struct WideLds {
  static constexpr int NA = MB / 16;
  static constexpr int TPW = TPW_;
  static constexpr int kTiles = kCW * TPW;
  static constexpr int kBlockRows = 16 * kTiles;
  static constexpr int XB = xbufs(MB);
  static constexpr int kXBytes = XB * MB * 256;
  static constexpr int kListOff = kXBytes;
  static constexpr int kListBytes = XB * kTiles * kPatchCap * 4;
  static constexpr int kHdrOff = kListOff + kListBytes;
  static constexpr int kScratchOff = kHdrOff + XB * 256;
  static constexpr int kMainBytes = CSR ? kScratchOff + kTiles * 64 * 64 : kXBytes;
  // epilogue: H high / low parts [MB][kEpiStride] fp16, B rows [kBlockRows][kEpiStride],
  // gamma [kBlockRows], output tile [MB][kOutStride] fp16 (rows 4 banks apart)
  static constexpr int kOutStride = kBlockRows + 8;
  static constexpr int kEpiHi = 0;
  static constexpr int kEpiLo = kEpiHi + MB * kEpiStride * 2;
  static constexpr int kEpiB = kEpiLo + MB * kEpiStride * 2;
  static constexpr int kEpiG = kEpiB + kBlockRows * kEpiStride * 2;
  static constexpr int kEpiOut = kEpiG + kBlockRows * 2;
  static constexpr int kEpiBytes = kEpiOut + MB * kOutStride * 2;
  static_assert(2 * kTiles <= 64, "one 64-lane copy holds the header");
};

// ------------------------------------------------------------------ DoRA blocks
// hpart[d, i, j] = DoRA block d's share of x[i, :] . A[j, :] for every activation row (NA row
// groups of 16): wave w takes the 32-column steps d kCW + w, + h_blocks kCW, ... (MFMA
// 16x16x32), the four wave sums are added through LDS.  The block that arrives last sums the
// blocks' shares in block order (all of a value's loads in flight at once), rounds
// H = fp16(sum) and raises the ready slots.  At most kMaxDoraBlocks: while one runs it holds a
// CU's LDS like a tile block.
template <int NA>
__device__ void wide_dora_block(const WideArgs& a, int d, float* red) {
  constexpr int JT = kMaxRank / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int jt_n = (a.r + 15) >> 4;
  if (wave < kCW) {
    float4_t acc[NA][JT];
#pragma unroll
    for (int g = 0; g < NA; ++g)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) acc[g][jt] = float4_t{0.f, 0.f, 0.f, 0.f};
    const int nks = (a.K + 31) / 32;
    for (int ks = d * kCW + wave; ks < nks; ks += a.h_blocks * kCW) {
      const int k = 32 * ks + 8 * kq;
      const bool kin = k < a.K;  // K % 8 == 0
      u32x4_t xa[NA];
#pragma unroll
      for (int g = 0; g < NA; ++g) {
        const int i = 16 * g + r16;
        xa[g] = u32x4_t{0u, 0u, 0u, 0u};
        if (i < a.M && kin) xa[g] = *reinterpret_cast<const u32x4_t*>(a.X + (size_t)i * a.K + k);
      }
      u32x4_t ab[JT];
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const int j = 16 * jt + r16;
        ab[jt] = u32x4_t{0u, 0u, 0u, 0u};
        if (jt < jt_n && j < a.r && kin) ab[jt] = *reinterpret_cast<const u32x4_t*>(a.A + (size_t)j * a.K + k);
      }
#pragma unroll
      for (int g = 0; g < NA; ++g)
#pragma unroll
        for (int jt = 0; jt < JT; ++jt)
          if (jt < jt_n) acc[g][jt] = mfma16x16x32(xa[g], ab[jt], acc[g][jt]);
    }
#pragma unroll
    for (int g = 0; g < NA; ++g)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
        if (jt < jt_n)
#pragma unroll
          for (int e = 0; e < 4; ++e) red[(((wave * NA + g) * JT + jt) * 4 + e) * 64 + lane] = acc[g][jt][e];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < NA * jt_n * 256; idx += blockDim.x) {
    const int ln = idx & 63;
    const int e = (idx >> 6) & 3;
    const int jt = (idx >> 8) % jt_n;
    const int g = (idx >> 8) / jt_n;
    const int i = 16 * g + 4 * (ln >> 4) + e;
    const int j = 16 * jt + (ln & 15);
    if (i < a.M && j < a.r) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kCW; ++w) v += red[(((w * NA + g) * JT + jt) * 4 + e) * 64 + ln];
      store_dev(a.hpart + ((size_t)d * a.M + i) * a.r + j, v);
    }
  }
  stores_done();
  __syncthreads();
  __shared__ int s_last;
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(a.sync + kSyncDora, 1u);
    if (old >= (uint32_t)a.h_blocks) raise_error(a.sync, kErrArrivals);
    s_last = old == (uint32_t)(a.h_blocks - 1);
  }
  __syncthreads();
  if (!s_last) return;
  compiler_fence();
  const size_t pstride = (size_t)a.M * a.r;
  for (int idx = threadIdx.x; idx < a.M * a.r; idx += blockDim.x) {
    float t[kMaxDoraBlocks];
#pragma unroll
    for (int u = 0; u < kMaxDoraBlocks; ++u) t[u] = load_dev(a.hpart + (size_t)min(u, a.h_blocks - 1) * pstride + idx);
    float v = 0.f;
#pragma unroll
    for (int u = 0; u < kMaxDoraBlocks; ++u)
      if (u < a.h_blocks) v += t[u];
    store_dev(a.hfin + idx, h2f(f2h_rn(v)));  // the reference's F.linear output is fp16
  }
  stores_done();
  __syncthreads();
  const int slots = min(a.TB, kMaxSlots);
  if (!a.withhold_h)
    for (int g = threadIdx.x; g < slots; g += blockDim.x) store_dev(a.sync + kSyncSlot0 + kSlotWords * g, 1u);
  if (threadIdx.x == 0) store_dev(a.sync + kSyncDora, 0u);
}

// --------------------------------------------------------------- tile blocks

struct Slab {
  u32x4_t codes;
  u32x4_t lo, hi;
};

template <int LM, int MB, bool CSR, int TPW_>
__global__ __launch_bounds__(kThreads) void wide_kernel(const WideArgs a) {
  using Lds = WideLds<MB, CSR, TPW_>;
  constexpr int NA = Lds::NA;
  constexpr int kDma = MB / 4;  // loader copies per activation slab (1 KB = 4 rows each)
  constexpr int XB = Lds::XB;    // activation slab buffers
  constexpr int XA = XB - 1;     // slabs the loader runs ahead
  constexpr int TPW = Lds::TPW;  // row tiles per compute wave
  constexpr int kTiles = Lds::kTiles;
  constexpr int kBlockRows = Lds::kBlockRows;
  extern __shared__ __align__(16) unsigned char smem[];

  int bid = blockIdx.x;
  if (bid < a.h_blocks) {
    wide_dora_block<NA>(a, bid, reinterpret_cast<float*>(smem));
    return;
  }
  bid -= a.h_blocks;
  const int tb = bid / a.splits;
  const int split = bid - tb * a.splits;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool loader = wave == kCW;
  const int r = lane & 15;
  const int kq = lane >> 4;
  const int s0 = a.sps * split;
  const int nsl = min(a.S, s0 + a.sps) - s0;  // slabs of this block: 1..kMaxSlabs (block-uniform)

  unsigned char* xbase = smem;
  uint32_t* lists = reinterpret_cast<uint32_t*>(smem + Lds::kListOff);
  uint32_t* hdr = reinterpret_cast<uint32_t*>(smem + Lds::kHdrOff);
  uint16_t* scratch = reinterpret_cast<uint16_t*>(smem + Lds::kScratchOff);

  __shared__ int s_err;  // poison: a failed hand-off (this call or the sticky error word)
  if (threadIdx.x == 0) s_err = 0;  // (ordered before its uses by the first barrier)

  float4_t acc[TPW][NA];  // compute wave w, tile jt: D rows 16 g + 4 kq + e, column 16 (w TPW + jt) + r
#pragma unroll
  for (int jt = 0; jt < TPW; ++jt)
#pragma unroll
    for (int g = 0; g < NA; ++g) acc[jt][g] = float4_t{0.f, 0.f, 0.f, 0.f};

  // The loader and the compute waves run separate loops with the same number of barriers
  // (one per slab): neither's wait-count bookkeeping sees the other's loads.
  if (loader) {
    // ------------------------------------------------------------------ loader wave
    // Patch-list starts of the block's tiles for slabs s0 .. s0 + nsl: tile w's start of
    // slab s0 + j is lane j of pa[w] (j < 64) or pb[w] (j >= 64).
    uint32_t pa[kTiles], pb[kTiles];
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.X), (short)0, (int)((size_t)a.M * a.K * 2), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(a.wpatch), (short)0, (int)a.patch_bytes, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t ir = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(a.wpidx), (short)0, CSR ? (int)(((size_t)a.T * a.S + 1) * 4) : 0, kRsrcWord3);
    // slab s0 + j -> buffer j % XB: the activations ...
    auto issue_x = [&](int j) __attribute__((always_inline)) {
      const int s = s0 + j;
      unsigned char* buf = xbase + (j % XB) * (MB * 256);
#pragma unroll
      for (int k = 0; k < kDma; ++k) {
        const int i = 4 * k + (lane >> 4);
        const int u = (lane & 15) ^ (i & 15);
        const int col = 128 * s + 8 * u;
        const uint32_t off = (i < a.M && col < a.K) ? (uint32_t)(((size_t)i * a.K + col) * 2) : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, buf + 1024 * k, 16, off, 0, 0, 0);
      }
    };
    // ... and, with outliers, the header (each tile's list start and end, copied from wpidx)
    // and the 4 tiles' lists (first kPatchCap).  Every slab takes the same number of copies,
    // kCopies (a copy of an empty list reads zeros), so a wait for a slab is a constant count
    // of younger copies; and the loader writes LDS only through copies.
    auto issue_lists = [&](int j) __attribute__((always_inline)) {
      const int b = j % XB;
      {
        const int w = lane >> 1;
        const uint32_t off = (lane < 2 * kTiles && tb * kTiles + w < a.T)
                                 ? (uint32_t)((((size_t)(tb * kTiles + w) * a.S + s0 + j + (lane & 1))) * 4)
                                 : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ir, hdr + 64 * b, 4, off, 0, 0, 0);
      }
#pragma unroll
      for (int w = 0; w < kTiles; ++w) {
        const uint32_t st = (uint32_t)__builtin_amdgcn_readlane((int)(j < 64 ? pa[w] : pb[w]), j & 63);
        const uint32_t en = (uint32_t)__builtin_amdgcn_readlane((int)(j + 1 < 64 ? pa[w] : pb[w]), (j + 1) & 63);
        const int n = tb * kTiles + w < a.T ? (int)(en - st) : 0;
        const uint32_t off = lane < n ? (st + (uint32_t)lane) * 4u : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(pr, lists + (b * kTiles + w) * kPatchCap, 4, off, 0, 0, 0);
      }
    };
    constexpr int kCopies = kDma + (CSR ? kTiles + 1 : 0);
    const int npre = min(XA, nsl);
    for (int j = 0; j < npre; ++j) issue_x(j);
    if constexpr (CSR) {
#pragma unroll
      for (int w = 0; w < kTiles; ++w) {
        const size_t base = (size_t)min(tb * kTiles + w, a.T - 1) * a.S + s0;  // + j <= T * S
        pa[w] = a.wpidx[base + min(lane, nsl)];
        pb[w] = a.wpidx[base + min(64 + lane, nsl)];
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (and every activation copy issued so far)
#pragma unroll
      for (int w = 0; w < kTiles; ++w) {  // plain registers from here on (no load pending on them)
        asm volatile("v_mov_b32 %0, %1" : "=v"(pa[w]) : "v"(pa[w]));
        asm volatile("v_mov_b32 %0, %1" : "=v"(pb[w]) : "v"(pb[w]));
      }
      for (int j = 0; j < npre; ++j) issue_lists(j);
      wait_copies<kTiles + 1, XA>(npre - 1);  // slab 0's lists in LDS (the later slabs' may be in flight)
    } else {
      wait_copies<kCopies, XA>(npre - 1);  // slab 0 in LDS
    }
    raw_barrier();
    for (int j = 0; j < nsl; ++j) {
      const int jf = j + XA;
      if (jf < nsl) {
        issue_x(jf);
        if constexpr (CSR) issue_lists(jf);
      }
      // slab j + 1 in LDS: the copies of slabs j + 2 .. min(jf, nsl - 1), all issued after
      // its own, may stay in flight (this wave issues nothing else)
      if (j + 1 < nsl) wait_copies<kCopies, XA>(min(jf, nsl - 1) - (j + 1));
      raw_barrier();
    }
  } else {
    // ------------------------------------------------------------------ compute waves
    // row tiles wt = w TPW + jt of the block (t = tb kTiles + wt), kPFW slabs of each in flight
    constexpr int kPFW = kPF / TPW;
    const u32x4_t* qb[TPW];
    const u32x4_t* lb[TPW];
#pragma unroll
    for (int jt = 0; jt < TPW; ++jt) {
      const int t = min(tb * kTiles + wave * TPW + jt, a.T - 1);
      qb[jt] = a.codes + (size_t)t * a.S * 64 + lane;
      lb[jt] = a.planes + (size_t)t * a.ng * 32 + r;
    }
    auto ld = [](const u32x4_t* p) __attribute__((always_inline)) { return __builtin_nontemporal_load(p); };
    auto load_slab = [&](Slab* sl, int s) __attribute__((always_inline)) {  // sl[TPW]
#pragma unroll
      for (int jt = 0; jt < TPW; ++jt) {
        sl[jt].codes = ld(qb[jt] + (size_t)s * 64);
        if constexpr (LM == 2) {
          const int g = s >> a.gshift;
          sl[jt].lo = ld(lb[jt] + g * 32);
          sl[jt].hi = ld(lb[jt] + g * 32 + 16);
        } else if constexpr (LM == 1) {
          const int g = min(group_of(128 * s + 32 * kq, a.g_magic), a.ng - 1);
          sl[jt].lo = ld(lb[jt] + g * 32);
          sl[jt].hi = ld(lb[jt] + g * 32 + 16);
        }
      }
    };
    LutPlanes<4> pl[TPW];
    if constexpr (LM == 0) {
#pragma unroll
      for (int jt = 0; jt < TPW; ++jt) {
        const u32x4_t lo = lb[jt][0];
        const u32x4_t hi = lb[jt][16];
        pl[jt].lo[0] = lo.x; pl[jt].lo[1] = lo.y; pl[jt].lo[2] = lo.z; pl[jt].lo[3] = lo.w;
        pl[jt].hi[0] = hi.x; pl[jt].hi[1] = hi.y; pl[jt].hi[2] = hi.z; pl[jt].hi[3] = hi.w;
      }
    }
    Slab buf[kPFW][TPW];
#pragma unroll
    for (int u = 0; u < kPFW; ++u) load_slab(buf[u], s0 + min(u, nsl - 1));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // s_err initialised
    raw_barrier();

    auto consume = [&](const Slab* sl, int j) __attribute__((always_inline)) {  // sl[TPW]
      const int b = j % XB;
      u32x4_t bq[TPW][4];
#pragma unroll
      for (int jt = 0; jt < TPW; ++jt) {
        LutPlanes<4> t4;
        if constexpr (LM == 0) {
          t4 = pl[jt];
        } else {
          t4.lo[0] = sl[jt].lo.x; t4.lo[1] = sl[jt].lo.y; t4.lo[2] = sl[jt].lo.z; t4.lo[3] = sl[jt].lo.w;
          t4.hi[0] = sl[jt].hi.x; t4.hi[1] = sl[jt].hi.y; t4.hi[2] = sl[jt].hi.z; t4.hi[3] = sl[jt].hi.w;
        }
        const uint32_t w[4] = {sl[jt].codes.x, sl[jt].codes.y, sl[jt].codes.z, sl[jt].codes.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t bv[4];
          dequant_word4s(w[q], t4, bv);
          bq[jt][q] = u32x4_t{bv[0], bv[1], bv[2], bv[3]};
        }
        if constexpr (CSR) {
          // outliers: dequantized words to the tile's scratch [word q][lane][8 fp16] (consecutive
          // lanes at consecutive 16-byte units), the slab's patches (one per lane), words back
          // (one wave's LDS operations complete in order)
          const int wt = wave * TPW + jt;
          const uint32_t st = hdr[64 * b + 2 * wt];
          const int n = (int)(hdr[64 * b + 2 * wt + 1] - st);
          if (n > 0) {
            uint16_t* scr = scratch + wt * 2048;
#pragma unroll
            for (int q = 0; q < 4; ++q) *reinterpret_cast<u32x4_t*>(scr + (q * 64 + lane) * 8) = bq[jt][q];
            auto apply = [&](uint32_t p) __attribute__((always_inline)) {  // element e of lane l: word e / 8
              const uint32_t e = (p >> 6) & 31u;
              scr[((e >> 3) * 64 + (p & 63u)) * 8 + (e & 7u)] = (uint16_t)((p >> 24) << 8);
            };
            if (lane < n) apply(lists[(b * kTiles + wt) * kPatchCap + lane]);
            if (n > kPatchCap) {  // the rest from global memory (rare: > 64 outliers in 16 x 128 weights)
              const uint32_t np = a.patch_bytes >> 2;
              for (int e = kPatchCap + lane; e < n; e += 64)
                if (st + (uint32_t)e < np) apply(a.wpatch[st + e]);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) bq[jt][q] = *reinterpret_cast<const u32x4_t*>(scr + (q * 64 + lane) * 8);
          }
        }
      }
      const unsigned char* xb = xbase + b * (MB * 256);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int v = ((4 * kq + q) ^ r) << 4;  // lane (r, kq) word q: columns 32 kq + 8 q .. +7
#pragma unroll
        for (int g = 0; g < NA; ++g) {
          const u32x4_t av = *reinterpret_cast<const u32x4_t*>(xb + (16 * g + r) * 256 + v);
#pragma unroll
          for (int jt = 0; jt < TPW; ++jt) acc[jt][g] = mfma16x16x32(av, bq[jt][q], acc[jt][g]);
        }
      }
      // this slab's LDS reads are complete before the barrier lets the loader refill the buffer
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      raw_barrier();
    };

    // Steady state: every slot consumed is reloaded kPFW slabs ahead; then one round with
    // conditional reloads and a last round without (nsl is block-uniform).
    int j0 = 0;
    for (; j0 + 2 * kPFW <= nsl; j0 += kPFW) {
#pragma unroll
      for (int u = 0; u < kPFW; ++u) {
        consume(buf[u], j0 + u);
        load_slab(buf[u], s0 + j0 + u + kPFW);
        __builtin_amdgcn_sched_barrier(0);  // keep each reload right behind its slot's use
      }
    }
    if (j0 < nsl) {
#pragma unroll
      for (int u = 0; u < kPFW; ++u) {
        if (j0 + u < nsl) {
          consume(buf[u], j0 + u);
          if (j0 + u + kPFW < nsl) load_slab(buf[u], s0 + j0 + u + kPFW);
        }
      }
      j0 += kPFW;
#pragma unroll
      for (int u = 0; u < kPFW; ++u)
        if (j0 + u < nsl) consume(buf[u], j0 + u);
    }
  }

  // ---------------------------------------------------------------- completion
  // Compute wave w holds D[i = 16 g + 4 kq + e][block column 16 (w TPW + jt) + r] in
  // acc[jt][g][e]; the epilogue works on that register layout (the main loop's LDS is reused).
  __syncthreads();
  const int slots = min(a.TB, kMaxSlots);
  uint32_t* slot = a.sync + kSyncSlot0 + kSlotWords * (tb % slots);
  const bool h_fused = a.r > 0 && a.h_blocks > 0;
  uint32_t err = 0u;
  if (a.splits > 1) {
    // Split partials in the register layout, [split][tile block][wave][jt][g][lane] x 4 fp32,
    // with 16-byte device-coherent (sc1) stores and loads.
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(a.partial, (short)0, (int)a.partial_bytes,
                                                                         kRsrcWord3);
    auto poff = [&](int sp, int jt, int g) __attribute__((always_inline)) {
      return (int)(((((((size_t)sp * a.TB + tb) * kCW + wave) * TPW + jt) * NA + g) * 64 + lane) * 16);
    };
    if (!loader) {
#pragma unroll
      for (int jt = 0; jt < TPW; ++jt)
#pragma unroll
        for (int g = 0; g < NA; ++g)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc[jt][g]), prs, poff(split, jt, g), 0,
                                                 kSc1);
    }
    stores_done();
    __syncthreads();
    __shared__ int s_last;
    if (threadIdx.x == 0) {
      const uint32_t old = atomicAdd(a.sync + kSyncTile + tb, 1u);
      if (old >= (uint32_t)a.splits) {
        raise_error(a.sync, kErrArrivals);
        s_err = 1;
      }
      s_last = old == (uint32_t)(a.splits - 1) || old >= (uint32_t)a.splits;
    }
    __syncthreads();
    if (!s_last) return;
    compiler_fence();
    if (threadIdx.x == 0) {
      err = load_dev(a.sync + kSyncErrorWord);
      store_dev(a.sync + kSyncTile + tb, 0u);
    }
    if (!loader) {
      // the splits' partials summed in split order (the same sum whichever block is last),
      // kU splits' loads in flight at a time
      constexpr int kNV = TPW * NA;
      constexpr int kU = kNV >= 8 ? 2 : kNV >= 4 ? 4 : 8;
#pragma unroll
      for (int jt = 0; jt < TPW; ++jt)
#pragma unroll
        for (int g = 0; g < NA; ++g) acc[jt][g] = float4_t{0.f, 0.f, 0.f, 0.f};
      for (int sp0 = 0; sp0 < a.splits; sp0 += kU) {
        u32x4_t v[kU][TPW][NA];
#pragma unroll
        for (int u = 0; u < kU; ++u)
#pragma unroll
          for (int jt = 0; jt < TPW; ++jt)
#pragma unroll
            for (int g = 0; g < NA; ++g)
              v[u][jt][g] =
                  __builtin_amdgcn_raw_buffer_load_b128(prs, poff(min(sp0 + u, a.splits - 1), jt, g), 0, kSc1);
#pragma unroll
        for (int u = 0; u < kU; ++u)
          if (sp0 + u < a.splits)
#pragma unroll
            for (int jt = 0; jt < TPW; ++jt)
#pragma unroll
              for (int g = 0; g < NA; ++g) acc[jt][g] += __builtin_bit_cast(float4_t, v[u][jt][g]);
      }
    }
  }

  // DoRA: s * H.B^T as MFMAs onto the accumulator layout.  H is staged in LDS as fp16 high
  // and low parts of 2^-sh H (sh > 0 only for blocks of H beyond the fp16 range), so the
  // products match fp32 H * fp16 B to ~2^-22; B rows and gamma of the block's columns.
  uint16_t* h_hi = reinterpret_cast<uint16_t*>(smem + Lds::kEpiHi);
  uint16_t* h_lo = reinterpret_cast<uint16_t*>(smem + Lds::kEpiLo);
  uint16_t* b_s = reinterpret_cast<uint16_t*>(smem + Lds::kEpiB);
  uint16_t* g_s = reinterpret_cast<uint16_t*>(smem + Lds::kEpiG);
  uint16_t* o_s = reinterpret_cast<uint16_t*>(smem + Lds::kEpiOut);
  __shared__ uint32_t s_hmax;
  uint32_t cons_old = 0u;
  bool counted = false;
  const int rp = a.r <= 32 ? 32 : 64;  // rank padded to the MFMA depth
  if (a.r > 0) {
    if (h_fused && lane == 0) {  // every wave reads H below: each polls the ready slot first
      uint32_t ready = load_dev(slot);
      for (uint32_t spins = 0; ready == 0u && spins < a.spin_limit; ++spins) {
        __builtin_amdgcn_s_sleep(2);
        ready = load_dev(slot);
      }
      if (ready == 0u) {
        s_err = 1;
        raise_error(a.sync, kErrHTimeout);
      }
    }
    compiler_fence();
    if (h_fused && threadIdx.x == 0 && a.splits == 1) err = load_dev(a.sync + kSyncErrorWord);
    if (threadIdx.x == 0) s_hmax = 0u;
    const float* hsrc = h_fused ? a.hfin : a.H;
    __syncthreads();
    uint32_t hmax = 0u;
    for (int idx = threadIdx.x; idx < a.M * a.r; idx += kThreads)
      hmax = max(hmax, __float_as_uint(hsrc[idx]) & 0x7FFFFFFFu);  // (NaN bit patterns order above inf)
    if (hmax != 0u) atomicMax(&s_hmax, hmax);
    for (int u = threadIdx.x; u < kBlockRows * (rp / 8); u += kThreads) {  // B rows, zero beyond rank r
      const int row = u / (rp / 8);
      const int c8 = 8 * (u % (rp / 8));
      const int n = min(tb * kBlockRows + row, a.N - 1);
      u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
      if (c8 < a.r) v = *reinterpret_cast<const u32x4_t*>(a.B + (size_t)n * a.r + c8);
      *reinterpret_cast<u32x4_t*>(b_s + row * kEpiStride + c8) = v;
    }
    if (threadIdx.x < kBlockRows) g_s[threadIdx.x] = a.gamma[min(tb * kBlockRows + (int)threadIdx.x, a.N - 1)];
    __syncthreads();
    const int hex = (int)((s_hmax >> 23) & 0xFFu) - 127;  // max |H| < 2^(hex + 1)
    const int sh = max(0, hex - 14);                     // 2^-sh max |H| < 2^15
    for (int idx = threadIdx.x; idx < MB * rp; idx += kThreads) {
      const int i = idx / rp;
      const int j = idx - i * rp;
      const float v = (i < a.M && j < a.r) ? ldexpf(hsrc[i * a.r + j], -sh) : 0.f;
      const uint16_t hi = f2h_rn(v);
      h_hi[i * kEpiStride + j] = hi;
      h_lo[i * kEpiStride + j] = f2h_rn(v - h2f(hi));
    }
    __syncthreads();
    if (!loader) {
      const float sc = ldexpf(a.scale, sh);
#pragma unroll
      for (int jt = 0; jt < TPW; ++jt) {
        const int col = 16 * (wave * TPW + jt) + r;  // block column of this lane's outputs
        float4_t dd[NA];
#pragma unroll
        for (int g = 0; g < NA; ++g) dd[g] = float4_t{0.f, 0.f, 0.f, 0.f};
        for (int kk = 0; kk < rp; kk += 32) {
          const u32x4_t bb = *reinterpret_cast<const u32x4_t*>(b_s + col * kEpiStride + kk + 8 * kq);
#pragma unroll
          for (int g = 0; g < NA; ++g) {
            const int ro = (16 * g + r) * kEpiStride + kk + 8 * kq;
            dd[g] = mfma16x16x32(*reinterpret_cast<const u32x4_t*>(h_hi + ro), bb, dd[g]);
            dd[g] = mfma16x16x32(*reinterpret_cast<const u32x4_t*>(h_lo + ro), bb, dd[g]);
          }
        }
        const float gam = h2f(g_s[col]);
#pragma unroll
        for (int g = 0; g < NA; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[jt][g][e] = (acc[jt][g][e] + sc * dd[g][e]) * gam;
      }
    }
  }
  if (err != 0u) s_err = 1;
  __syncthreads();
  if (h_fused && threadIdx.x == 0) {  // every poll of the block is done (the barrier above)
    cons_old = atomicAdd(slot + 1, 1u);
    counted = true;
  }
  // outputs: fp16 through LDS ([MB][kOutStride]), then rows of kBlockRows columns in 16-byte stores
  const bool poisoned = s_err != 0;
  if (!loader) {
#pragma unroll
    for (int jt = 0; jt < TPW; ++jt)
#pragma unroll
      for (int g = 0; g < NA; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o_s[(16 * g + 4 * kq + e) * Lds::kOutStride + 16 * (wave * TPW + jt) + r] =
              poisoned ? kHalfNaN : f2h_rn(acc[jt][g][e]);
  }
  __syncthreads();
  constexpr int kUnits = kBlockRows / 8;  // 16-byte units per output row of the block
  for (int idx = threadIdx.x; idx < a.M * kUnits; idx += kThreads) {
    const int i = idx / kUnits;
    const int c8 = 8 * (idx - i * kUnits);
    const int n0 = tb * kBlockRows + c8;
    const uint16_t* src = o_s + i * Lds::kOutStride + c8;
    uint16_t* dst = a.out + (size_t)i * a.N + n0;
    if (a.out_vec && n0 + 8 <= a.N) {
      *reinterpret_cast<u32x4_t*>(dst) = *reinterpret_cast<const u32x4_t*>(src);
    } else {
      for (int c = 0; c < 8; ++c)
        if (n0 + c < a.N) dst[c] = src[c];
    }
  }
  if (counted) {  // the slot's last consumer lowers it for the next call
    const int g = tb % slots;
    const uint32_t members = (uint32_t)(a.TB / slots + (g < a.TB % slots ? 1 : 0));
    if (cons_old >= members) raise_error(a.sync, kErrArrivals);
    if (cons_old == members - 1u) {
      store_dev(slot + 1, 0u);
      store_dev(slot, 0u);
    }
  }
}

template <int LM, int MB, bool CSR, int TPW>
hipError_t launch_wide_tpl(const WideArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((wide_kernel<LM, MB, CSR, TPW>), grid, dim3(kThreads), lds, stream, a);
  return hipGetLastError();
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

int wide_mb(int M) { return M <= 16 ? 16 : M <= 32 ? 32 : M <= 64 ? 64 : 128; }

template <int MB, int TPW>
size_t wide_lds_bytes(bool csr) {
  const size_t main =
      csr ? (size_t)WideLds<MB, true, TPW>::kMainBytes : (size_t)WideLds<MB, false, TPW>::kMainBytes;
  return std::max(main, (size_t)WideLds<MB, true, TPW>::kEpiBytes);
}

size_t wide_lds(int M, bool csr, int tpw) {
  switch (wide_mb(M)) {
    case 16: return wide_lds_bytes<16, 1>(csr);
    case 32: return wide_lds_bytes<32, 1>(csr);
    case 64: return wide_lds_bytes<64, 1>(csr);
    default: return tpw == 2 ? wide_lds_bytes<128, 2>(csr) : wide_lds_bytes<128, 1>(csr);
  }
}

}  // namespace

int wide_max_m() { return 128; }

WidePlan plan_wide(int N, int K, int M, int cu_count, int rank, int fused_rank, int chunk, bool csr) {
  WidePlan p{};
  const int T = (N + 15) / 16;
  const int S = (K + 127) / 128;
  // two row tiles per compute wave at 128 activation rows on layers wide enough to keep the CUs
  // busy with half the blocks or long enough in K to split (measured: gate 18944x3584 at M = 128
  // 106 -> 67 us, down 3584x18944 73 -> 66 us; q/k/v and every M <= 64 slower)
  const int cus = std::max(1, cu_count);
  p.tpw = (wide_mb(M) == 128 && ((T + 2 * kCW - 1) / (2 * kCW) >= cus / 2 || S >= 64)) ? 2 : 1;
  const int tiles = kCW * p.tpw;  // row tiles per block
  p.TB = (T + tiles - 1) / tiles;
  p.lds = wide_lds(M, csr, p.tpw);
  if (fused_rank > 0)  // the DoRA blocks' wave sums, [kCW][row groups][kMaxRank / 16][4][64] fp32
    p.lds = std::max<size_t>(p.lds, (size_t)kCW * (wide_mb(M) / 16) * (kMaxRank / 16) * 4 * 64 * 4);
  p.ok = M > 8 && M <= wide_max_m() && (chunk == 512 || chunk == 640) && rank % 8 == 0 && rank <= kMaxRank &&
         fused_rank % 8 == 0 && fused_rank <= kMaxRank && p.lds <= 160 * 1024;
  if (!p.ok) return p;
  // K splits.  Measured on MI355X (Qwen2.5-7B shapes, M = 16..128): extra blocks pay while
  // they add latency hiding (up to ~2.5 per CU at M <= 16, ~2 up to M = 64) and cost once
  // the MFMA and LDS work per slab fills the CU (M = 128: one block per CU); a split
  // shorter than ~7 slabs spends more in its prologue and hand-off than it gains, except
  // on layers too narrow to occupy a quarter of the CUs (k/v: 8 tile blocks), where 4
  // slabs per split measured best.
  // The DoRA blocks are dispatched first and hold CU slots too: a tile block past the cap waits
  // for a second round (down 3584x18944 at M = 128: 8 splits 62 us, 9 splits 75 us).
  const int min_slabs = p.TB < cus / 4 ? 4 : 7;
  const int cap = (M <= 16 ? cus * 5 / 2 : M <= 64 ? 2 * cus : cus) -
                  (fused_rank > 0 ? std::min(kMaxDoraBlocks, (K + 511) / 512) : 0);
  const int smin = (S + kMaxSlabs - 1) / kMaxSlabs;
  int splits = std::max(smin, std::min(cap / p.TB, S / min_slabs));
  const int sps = (S + splits - 1) / splits;
  splits = (S + sps - 1) / sps;
  p.splits = splits;
  p.sps = sps;
  p.h_blocks = fused_rank > 0 ? std::min(kMaxDoraBlocks, (K + 511) / 512) : 0;
  const size_t hf = fused_rank > 0 ? align256((size_t)M * fused_rank * 4) : 0;
  const size_t hp = fused_rank > 0 ? align256((size_t)p.h_blocks * M * fused_rank * 4) : 0;
  const size_t part = splits > 1 ? (size_t)splits * p.TB * 16 * tiles * wide_mb(M) * 4 : 0;
  p.hfin_off = 0;
  p.hpart_off = hf;
  p.partial_off = hf + hp;
  p.workspace_bytes = hf + hp + part;
  p.ok = sps <= kMaxSlabs && (splits == 1 || p.TB <= kSyncErrorWord - kSyncTile) && part < ((size_t)1 << 31);
  return p;
}

hipError_t launch_wide(const Layer& L, const void* prepared, int64_t nnz, const Dora& D, const uint16_t* x,
                       uint16_t* out, int M, const WidePlan& plan, float* workspace, uint32_t* sync,
                       hipStream_t stream) {
  const PreparedLayout lay = prepared_layout(L.N, L.K, L.group_size, nnz);
  const char* base = reinterpret_cast<const char*>(prepared);
  WideArgs a{};
  a.codes = reinterpret_cast<const u32x4_t*>(base + lay.codes_off);
  a.planes = reinterpret_cast<const u32x4_t*>(base + lay.planes_off);
  const bool csr = L.offsets != nullptr && nnz > 0;
  a.wpidx = csr ? reinterpret_cast<const uint32_t*>(base + lay.wpidx_off) : nullptr;
  a.wpatch = csr ? reinterpret_cast<const uint32_t*>(base + lay.wpatch_off) : nullptr;
  a.patch_bytes = csr ? (uint32_t)((size_t)nnz * 4) : 0u;
  a.X = x;
  a.out = out;
  a.B = D.B;
  a.H = D.H;
  a.gamma = D.gamma;
  a.A = D.A;
  a.scale = D.scale;
  a.r = D.r;
  a.M = M;
  a.N = L.N;
  a.K = L.K;
  a.S = lay.S;
  a.ng = lay.ng;
  a.T = lay.T;
  a.TB = plan.TB;
  a.g_magic = L.group_size > 0 ? (uint32_t)((0x100000000ull / (uint64_t)L.group_size) + 1ull) : 0u;
  a.splits = plan.splits;
  a.sps = plan.sps;
  const bool fused_h = D.r > 0 && D.H == nullptr;
  a.h_blocks = fused_h ? plan.h_blocks : 0;
  char* ws = reinterpret_cast<char*>(workspace);
  a.hfin = reinterpret_cast<float*>(ws + plan.hfin_off);
  a.hpart = reinterpret_cast<float*>(ws + plan.hpart_off);
  a.partial = reinterpret_cast<float*>(ws + plan.partial_off);
  a.partial_bytes = (uint32_t)(plan.workspace_bytes - plan.partial_off);
  a.out_vec = L.N % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  a.sync = sync;
  a.spin_limit = spin_limit();
  a.withhold_h = withhold_h() ? 1 : 0;
  const bool per_row = L.group_size <= 0 || lay.ng == 1;
  if (per_row) a.ng = 1;
  int gshift = 0;
  while (gshift < 5 && (128 << gshift) < L.group_size) ++gshift;
  const bool slab_groups = !per_row && L.group_size == (128 << gshift);
  a.gshift = gshift;
  const dim3 grid(a.h_blocks + plan.TB * plan.splits);
  const size_t lds = plan.lds;
  const int mb = wide_mb(M);
#define WLQ_WIDE_MB(LMV, CSRV)                                                                  \
  switch (mb) {                                                                                \
    case 16: return launch_wide_tpl<LMV, 16, CSRV, 1>(a, grid, lds, stream);                   \
    case 32: return launch_wide_tpl<LMV, 32, CSRV, 1>(a, grid, lds, stream);                   \
    case 64: return launch_wide_tpl<LMV, 64, CSRV, 1>(a, grid, lds, stream);                   \
    default:                                                                                   \
      return plan.tpw == 2 ? launch_wide_tpl<LMV, 128, CSRV, 2>(a, grid, lds, stream)          \
                           : launch_wide_tpl<LMV, 128, CSRV, 1>(a, grid, lds, stream);         \
  }
#define WLQ_WIDE_LM(LMV) \
  if (csr) {             \
    WLQ_WIDE_MB(LMV, true) \
  } else {               \
    WLQ_WIDE_MB(LMV, false) \
  }
  if (per_row) {
    WLQ_WIDE_LM(0)
  } else if (slab_groups) {
    WLQ_WIDE_LM(2)
  } else {
    WLQ_WIDE_LM(1)
  }
#undef WLQ_WIDE_LM
#undef WLQ_WIDE_MB
}

}  // namespace wlq
