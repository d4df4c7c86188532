// Decode product on the prepared (tile-contiguous) layout: M = 1..32 activation
// rows, 4-bit or 3-bit codes (3-bit codes are stored as 4-bit nibbles against
// their 8-entry LUTs padded to 16), per-row LUTs or LUT groups of a multiple of
// 32 columns.
//
// Reference behaviour replaced: gemv_chunk_csr_kernel + launch_gemv_chunk_csr
// (csrc/gemv_kernel.cu:86-320, :396-457) and the split-K reduce
// (csrc/gemv_kernel.cu:322-353) for M == 1, gemm_metalog_dora_kernel
// (csrc/gemm_kernel.cu:32-294) for 2 <= M < 16, and the dequant -> GEMM -> DoRA
// epilogue sequence (csrc/vllm_binding.cpp:355-393) for 16 <= M <= 32.  Same arithmetic: W0 rows
// expanded through their LUTs, the delta-form outlier correction
// (w_true - lut[code]) * x (csrc/gemv_kernel.cu:262-288), the DoRA epilogue
// fp16_rn((acc + s * h.B) * gamma) (csrc/gemv_kernel.cu:305-319).
//
// Prepared layout (built once per layer by the prepare kernels below, from the
// reference's row-aligned codes, LUTs and chunk CSR):
//   codes  u32x4 [T][S][64]     T = ceil(N/16) row tiles, S = ceil(K/128) slabs;
//                               lane l = r + 16*kq holds the 32 codes of row 16t + r,
//                               columns 128s + 32kq .. +31 (4 words, 8 columns each in
//                               the selector-ready encoding of wlq_device.h), so one
//                               wave load is 1 KB contiguous and lands in the MFMA
//                               B-operand lane order.
//   planes u32x4 [T][ng][2][16] the low and the high bytes of the 16 fp16 LUT
//                               entries of row 16t + r, group g (the V_PERM_B32
//                               byte planes, wlq_device.h).
//   gcol   u16 [nnz]            the outlier's column (chunk base + chunk column).
//   delta  f32 [nnz]            fp32(fp16(e5m2 << 8)) - fp32(lut[code]): the
//                               reference's delta_w, computed once.
//   wpidx  u32 [T*S + 1]        start of each (tile, slab)'s patch list in wpatch
//                               (exclusive prefix sums; the last entry is the total).
//   wpatch u32 [nnz]            the outliers as patches of the dequantized operand of
//                               the M = 9..128 kernel (wlq_wide.hip), grouped by
//                               (tile, slab) in storage order: lane | (column % 32) << 6
//                               | e5m2 byte << 24, lane = row % 16 + 16 ((column % 128) / 32)
//                               -- the MFMA B-operand lane holding that column.  Entries
//                               with column >= K are dropped, and so is an entry whose
//                               column a later entry of the row overwrites (the last
//                               write wins, as in the dense overwrite).
// The reference's chunk offsets are used as they are.
//
// Work decomposition.  The grid is the DoRA blocks (x.A^T partial sums over 512
// columns, when H is computed here) followed by tile blocks x K splits.  A tile
// block is 4 waves on TPB row tiles (16 rows each); the WPT = 4 / TPB waves of a
// tile take its slabs round-robin.  Blocks are small (tens of KB of weights) and
// many (~4 per CU or more), so the hardware dispatcher balances them.  Per slab a
// lane dequantizes its 4 code words through its row's byte planes and feeds four
// V_MFMA_F32_16X16X32_F16 (A = activation rows from LDS, B = W rows); slabs are
// prefetched kPF ahead into registers.  After the slabs, the block's threads walk
// its rows' outlier entries (col, delta) and the wave partials are summed in a
// fixed order.  One K split: the block applies the epilogue.  Several: fp32
// partials go to the workspace and the block that counts the last arrival on its
// tile block sums them in split order and applies the epilogue.
//
// DoRA H: the DoRA blocks have the lowest block indices, so they are dispatched
// before every tile block.  The last of them rounds H to fp16 and raises a ready
// flag; a block that needs H waits for the flag (normally long set by then).  The
// last block to finish resets the flag and the counters, so every call leaves
// them zero.
//
// Failures of the hand-off are loud, not silent.  A wait for H that runs out of
// polls, or an arrival count that exceeds the number of arrivals a call can make
// (the counters were not zero at entry: a workspace shared by unordered calls,
// or never zero-filled), sets a bit in the workspace's error word and the rows
// concerned are written as fp16 NaN.  The error word is sticky: every later call
// on that workspace writes NaN rows too, until the host reads it
// (wlq_workspace_status) and clears the counter area (wlq_workspace_reset).
#include <algorithm>

#include "wlq_device.h"
#include "wlq_internal.h"

namespace wlq {
namespace {

#ifndef WLQ_STREAM_PF
#define WLQ_STREAM_PF 4
#endif
#ifndef WLQ_STREAM_BLOCKS_PER_CU
#define WLQ_STREAM_BLOCKS_PER_CU 4
#endif
#ifndef WLQ_STREAM_CUS_PER_BLOCK_M2
#define WLQ_STREAM_CUS_PER_BLOCK_M2 2  // M <= 2 (one tile per block): split K only below CUs / 2 tile blocks
#endif
#ifndef WLQ_STREAM_WAVES_PER_EU
#define WLQ_STREAM_WAVES_PER_EU 5
#endif
constexpr int kPF = WLQ_STREAM_PF;  // slabs in flight per wave
// Outlier entries per thread fetched during the slab loop: 3 where a block covers one or two row
// tiles (8-16 threads per row; -1-3% at M <= 2), 2 with four tiles (4 threads per row, M > 2).
template <int TPB> constexpr int outlier_prefetch() { return TPB <= 2 ? 3 : 2; }
constexpr int kXR = 4;          // 16-byte activation units per thread (the planner bounds the staging)
constexpr int kHCols = 512;     // columns per DoRA block
constexpr int kMaxRank = 64;
constexpr int kXBudget = 16384; // activation staging bytes per block
constexpr int kBlocksPerCU = WLQ_STREAM_BLOCKS_PER_CU;  // tile-block target per CU
// Sync words in the workspace's counter area (layout in wlq_internal.h; all zero between calls).
constexpr int kSyncErr = kSyncErrorWord;  // sticky error bits (own 128-byte line)

struct StreamArgs {
  const u32x4_t* codes;
  const u32x4_t* planes;
  const uint16_t* gcol;
  const float* delta;
  const int32_t* offsets;  // [N, nch + 1] (null: no outliers)
  const uint16_t* x;
  uint16_t* out;
  const uint16_t* B;
  const float* H;          // caller's H, or null (DoRA blocks compute it when A is set)
  const uint16_t* gamma;
  const uint16_t* A;
  float scale;
  int r;
  int M, N, K, S, ng, nch, T, TB;
  uint32_t g_magic;        // floor(c / G) == umulhi(c, g_magic) for c < 2^20
  int gshift;              // G == 128 << gshift (the kernel's LM == 2 case)
  int splits, cps;         // K splits per tile block, outlier chunks per split
  int spc;                 // slabs per outlier chunk (4; 5 for 3-bit's 640-column chunks)
  int xstride;             // halves per staged activation row
  int h_blocks;
  float* partial;          // [splits, M, N]
  float* hpart;            // [h_blocks, M, r]
  float* hfin;             // [M, r]
  uint32_t* sync;
  uint32_t spin_limit;     // polls of a ready slot before the wait gives up
  int withhold_h;          // test hook: the DoRA finisher never raises the ready slots
};

// Error word: bits from wlq_internal.h (kErr*), set with a device-scope atomic OR.
__device__ __forceinline__ void raise_error(uint32_t* sync, uint32_t bit) {
  __hip_atomic_fetch_or(sync + kSyncErr, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr uint16_t kHalfNaN = 0x7E00u;

__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_dev(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Stores are device-scope (coherent across the XCDs' L2s); waiting for them to
// complete orders them before a following arrival count.
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ int group_of(int col, uint32_t magic) { return (int)__umulhi((uint32_t)col, magic); }

// ------------------------------------------------------------------ DoRA blocks

// hpart[hb, i, j] = sum over columns [512 hb, +512) of x[i, k] * A[j, k]; wave w
// covers 128 columns with MFMA 16x16x32 (A = 16 activation rows per group, NA
// groups; B = lora_A rows; both in natural column order); the four wave sums are
// added through LDS.  The block that arrives last rounds H = fp16(sum over hb) and
// publishes it.
template <int NA>
__device__ void dora_block(const StreamArgs& a, int hb, float* red) {
  constexpr int JT = kMaxRank / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int jt_n = (a.r + 15) >> 4;
  float4_t acc[NA][JT];
#pragma unroll
  for (int g = 0; g < NA; ++g)
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) acc[g][jt] = float4_t{0.f, 0.f, 0.f, 0.f};
  const int kbase = hb * kHCols + wave * 128;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int k = kbase + 32 * ks + 8 * kq;
    const bool kin = k < a.K;  // K % 8 == 0: an 8-column unit is all inside or all outside
    u32x4_t xa[NA];
#pragma unroll
    for (int g = 0; g < NA; ++g) {
      const int i = 16 * g + r16;
      xa[g] = u32x4_t{0u, 0u, 0u, 0u};
      if (i < a.M && kin) xa[g] = *reinterpret_cast<const u32x4_t*>(a.x + (size_t)i * a.K + k);
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
  // red[wave][g][jt][e][lane]
#pragma unroll
  for (int g = 0; g < NA; ++g)
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
      if (jt < jt_n)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[(((wave * NA + g) * JT + jt) * 4 + e) * 64 + lane] = acc[g][jt][e];
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
      for (int w = 0; w < 4; ++w) v += red[(((w * NA + g) * JT + jt) * 4 + e) * 64 + ln];
      store_dev(a.hpart + ((size_t)hb * a.M + i) * a.r + j, v);
    }
  }
  stores_done();
  __syncthreads();
  __shared__ int s_last;
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(a.sync + kSyncDora, 1u);
    if (old >= (uint32_t)a.h_blocks) raise_error(a.sync, kErrArrivals);  // no finisher: the H waits run out
    s_last = old == (uint32_t)(a.h_blocks - 1);
  }
  __syncthreads();
  if (!s_last) return;
  compiler_fence();
  // sums in block order, 8 blocks' partials in flight at once (clamped; only b < h_blocks added)
  for (int idx = threadIdx.x; idx < a.M * a.r; idx += blockDim.x) {
    float v = 0.f;
    for (int b0 = 0; b0 < a.h_blocks; b0 += 8) {
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = load_dev(a.hpart + (size_t)min(b0 + u, a.h_blocks - 1) * a.M * a.r + idx);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (b0 + u < a.h_blocks) v += t[u];
    }
    store_dev(a.hfin + idx, h2f(f2h_rn(v)));  // the reference's F.linear output is fp16
  }
  stores_done();
  __syncthreads();
  // H is visible: raise every ready slot, then reset the arrival count for the next call
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

// LM: 0 = one LUT per row; 1 = LUT groups of a multiple of 32 columns; 2 = groups of 128 << gshift
// columns, so a slab's group is s >> gshift for all its lanes (no per-lane group arithmetic).
template <int LM, int TPB, int MB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MB > 16 ? 4 : WLQ_STREAM_WAVES_PER_EU)))
void stream4_kernel(const StreamArgs a) {
  constexpr int WPT = 4 / TPB;       // waves per row tile
  constexpr int ROWS = 16 * TPB;     // output rows per block
  constexpr int TPR = 256 / ROWS;    // threads per row in the outlier pass
  constexpr int NA = (MB + 15) / 16; // 16-row activation groups (MFMA A operands)
  constexpr int XR = MB > 16 ? 2 * kXR : kXR;  // 16-byte activation units per thread
  extern __shared__ __align__(16) uint16_t smem[];

  int bid = blockIdx.x;
  if (bid < a.h_blocks) {
    dora_block<NA>(a, bid, reinterpret_cast<float*>(smem));
    return;
  }
  bid -= a.h_blocks;
  const int tb = bid / a.splits;
  const int split = bid - tb * a.splits;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: slab indices live in SGPRs
  const int r = lane & 15;
  const int kq = lane >> 4;
  const int t = min(tb * TPB + wave / WPT, a.T - 1);
  const int ph = wave % WPT;
  const int c0 = split * a.cps;
  const int c1 = min(a.nch, c0 + a.cps);
  const int s0 = a.spc * c0;
  const int s1 = min(a.S, a.spc * c1);
  const int nw = (s1 - s0 - ph + WPT - 1) / WPT;  // this wave's slabs (may be 0)
  const int s_last = min(s0 + ph + WPT * max(nw - 1, 0), s1 - 1);  // prefetch clamp (in range)

  // LDS: [x: M rows x xstride halves][64 B zeros][red: 4 x NA x 256 f32]
  //      [B rows: ROWS x r halves][gamma: ROWS halves]; H (M x r f32) reuses the x rows
  //      once the outlier pass has read them.
  uint16_t* xs = smem;
  const int xbytes = ((a.M * a.xstride * 2) + 15) & ~15;
  uint16_t* zline = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(smem) + xbytes);
  float* red = reinterpret_cast<float*>(reinterpret_cast<char*>(zline) + 64);
  float* hs = reinterpret_cast<float*>(smem);
  uint16_t* bs = reinterpret_cast<uint16_t*>(red + 4 * NA * 256);
  uint16_t* gs = bs + ROWS * a.r;

  // Poison flag: this call's own hand-off failure (an H wait that ran out, an arrival count
  // beyond one call's) or the workspace's sticky error word, which a block reads together with
  // its first cross-block load (H or the split partials), so the read adds no round trip.
  // Blocks that hand nothing over have no counters that could be stale.
  __shared__ int s_err;
  if (threadIdx.x == 0) s_err = 0;

  // Outlier pass mapping: thread (rho, j) walks entries j, j + TPR, ... of block row rho.
  const int rho = threadIdx.x / TPR;
  const int jr = threadIdx.x - rho * TPR;
  const int n_out = tb * ROWS + rho;
  const bool csr = a.offsets != nullptr;
  int e0 = 0, e1 = 0;
  if (csr && n_out < a.N) {
    const int32_t* offr = a.offsets + (size_t)n_out * (a.nch + 1);
    e0 = offr[c0];
    e1 = offr[c1];
  }

  // Activations [s0*128, s1*128) of the M rows: loads now, LDS stores after the prefetch is issued.
  const int upr = (s1 - s0) * 16;  // 8-column units per row
  const int total = a.M * upr;
  u32x4_t xv[XR];
#pragma unroll
  for (int k = 0; k < XR; ++k) {
    const int u = min((int)threadIdx.x + 256 * k, max(total - 1, 0));
    const int i = u / upr;
    const int col = min(s0 * 128 + ((u - i * upr) << 3), a.K - 8);
    xv[k] = *reinterpret_cast<const u32x4_t*>(a.x + (size_t)i * a.K + col);
  }

  // DoRA B rows and gamma of the block's rows (16-byte units; r % 8 == 0, checked by the host).
  const int bupr = a.r >> 3;
  const int btotal = ROWS * bupr;
  u32x4_t bv[2];
  uint16_t gv = 0;
  if (a.r > 0) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int u = min((int)threadIdx.x + 256 * k, btotal - 1);
      const int row = min(tb * ROWS + u / bupr, a.N - 1);
      bv[k] = *reinterpret_cast<const u32x4_t*>(a.B + (size_t)row * a.r + 8 * (u % bupr));
    }
    gv = a.gamma[min(tb * ROWS + (int)(threadIdx.x % ROWS), a.N - 1)];
  }

  // Slab prefetch.
  const u32x4_t* qb = a.codes + (size_t)t * a.S * 64 + lane;
  const u32x4_t* lb = a.planes + (size_t)t * a.ng * 32 + r;
  // Codes and LUT planes are read once per call: non-temporal loads keep them from displacing the
  // activations and DoRA operands that every block re-reads (o_proj at M = 1 8.7 -> 7.9 us).
  auto ld = [](const u32x4_t* p) __attribute__((always_inline)) { return __builtin_nontemporal_load(p); };
  auto load_slab = [&](Slab& sl, int s) __attribute__((always_inline)) {
    sl.codes = ld(qb + (size_t)s * 64);
    if constexpr (LM == 2) {
      const int g = s >> a.gshift;
      sl.lo = ld(lb + g * 32);
      sl.hi = ld(lb + g * 32 + 16);
    } else if constexpr (LM == 1) {
      const int g = min(group_of(128 * s + 32 * kq, a.g_magic), a.ng - 1);
      sl.lo = ld(lb + g * 32);
      sl.hi = ld(lb + g * 32 + 16);
    }
  };
  LutPlanes<4> pl;
  if constexpr (LM == 0) {
    const u32x4_t lo = lb[0];
    const u32x4_t hi = lb[16];
    pl.lo[0] = lo.x; pl.lo[1] = lo.y; pl.lo[2] = lo.z; pl.lo[3] = lo.w;
    pl.hi[0] = hi.x; pl.hi[1] = hi.y; pl.hi[2] = hi.z; pl.hi[3] = hi.w;
  }
  Slab buf[kPF];
#pragma unroll
  for (int u = 0; u < kPF; ++u) load_slab(buf[u], min(s0 + ph + WPT * u, s_last));

#pragma unroll
  for (int k = 0; k < XR; ++k) {
    const int u = (int)threadIdx.x + 256 * k;
    if (u < total) {
      const int i = u / upr;
      const int c8 = u - i * upr;
      const bool inside = s0 * 128 + (c8 << 3) < a.K;  // K % 8 == 0
      *reinterpret_cast<u32x4_t*>(xs + i * a.xstride + (c8 << 3)) = inside ? xv[k] : u32x4_t{0u, 0u, 0u, 0u};
    }
  }
  if (threadIdx.x < 16) reinterpret_cast<uint32_t*>(zline)[threadIdx.x] = 0u;
  if (a.r > 0) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int u = (int)threadIdx.x + 256 * k;
      if (u < btotal) *reinterpret_cast<u32x4_t*>(bs + 8 * u) = bv[k];
    }
    if (threadIdx.x < ROWS) gs[threadIdx.x] = gv;
  }

  // Outlier entries, fetched while the slabs stream (clamped, so the loads are unconditional).
  constexpr int kEB = outlier_prefetch<TPB>();
  uint32_t ecol[kEB];
  float edel[kEB];
  if (csr) {
#pragma unroll
    for (int u = 0; u < kEB; ++u) {
      const int e = min(e0 + jr + TPR * u, max(e1 - 1, 0));
      ecol[u] = a.gcol[e];
      edel[u] = a.delta[e];
    }
  }
  __syncthreads();

  // Slab loop.  acc[g]: activation rows 16 g .. 16 g + 15.
  float4_t acc[NA];
#pragma unroll
  for (int g = 0; g < NA; ++g) acc[g] = float4_t{0.f, 0.f, 0.f, 0.f};
  const uint16_t* xrow = (r < a.M) ? xs + r * a.xstride + kq * 32 : nullptr;
  const uint16_t* xrow2 = (NA > 1 && r + 16 < a.M) ? xs + (r + 16) * a.xstride + kq * 32 : nullptr;
  auto consume = [&](const Slab& sl, int s) __attribute__((always_inline)) {
    LutPlanes<4> t4;
    if constexpr (LM == 0) {
      t4 = pl;
    } else {
      t4.lo[0] = sl.lo.x; t4.lo[1] = sl.lo.y; t4.lo[2] = sl.lo.z; t4.lo[3] = sl.lo.w;
      t4.hi[0] = sl.hi.x; t4.hi[1] = sl.hi.y; t4.hi[2] = sl.hi.z; t4.hi[3] = sl.hi.w;
    }
    const uint16_t* xp = xrow ? xrow + (s - s0) * 128 : zline;
    const uint16_t* xp2 = xrow2 ? xrow2 + (s - s0) * 128 : zline;
    const uint32_t w[4] = {sl.codes.x, sl.codes.y, sl.codes.z, sl.codes.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t b[4];
      dequant_word4s(w[q], t4, b);
      const u32x4_t bv = {b[0], b[1], b[2], b[3]};
      const u32x4_t av = *reinterpret_cast<const u32x4_t*>(xp + (xrow ? 8 * q : 0));
      acc[0] = mfma16x16x32(av, bv, acc[0]);
      if constexpr (NA > 1) {
        const u32x4_t av2 = *reinterpret_cast<const u32x4_t*>(xp2 + (xrow2 ? 8 * q : 0));
        acc[1] = mfma16x16x32(av2, bv, acc[1]);
      }
    }
  };
  // DoRA H into registers, by the threads that own H elements.  A caller's H is loaded
  // directly.  The computed H needs the block's ready slot (raised by the DoRA finisher,
  // normally long before the tile blocks end): lane 0 of each owner wave polls it (after
  // spin_limit polls the wait gives up, raises kErrHTimeout and the block writes NaN rows
  // rather than hang), then the owners load H.  One K split: every tile block loads H after its
  // slab loop, so the loads overlap the outlier pass; several: only the block that finishes the
  // rows does.  A block counts itself on the slot after all its polls (a barrier) and the slot's
  // last consumer lowers it, so no slot is lowered while one of its tile blocks still polls.
  const int slots = min(a.TB, kMaxSlots);
  uint32_t* slot = a.sync + kSyncSlot0 + kSlotWords * (tb % slots);
  constexpr int kHB = (MB * kMaxRank + 255) / 256;  // H words per thread (M * r <= MB * 64)
  float hv[kHB];
  bool h_have = false;               // this thread's H words are in hv
  const bool h_owner = (int)threadIdx.x < a.M * a.r;
  const bool h_fused = a.r > 0 && a.h_blocks > 0;
  // H words of an owner thread once the slot is known raised; thread 0 also reads the
  // workspace's sticky error word, in parallel with H (no extra round trip).
  auto fetch_h = [&]() __attribute__((always_inline)) {
    uint32_t err = 0u;
    if (threadIdx.x == 0) err = load_dev(a.sync + kSyncErr);
    // H is read through the caches: no block touches hfin before it saw the slot raised, and a
    // kernel starts with invalidated caches, so the first read of the line on each XCD brings
    // the published values and later blocks on that XCD hit its L2.
    const float* hf = a.hfin;
#pragma unroll
    for (int u = 0; u < kHB; ++u) hv[u] = hf[min((int)threadIdx.x + 256 * u, a.M * a.r - 1)];
    if (err != 0u) s_err = 1;
    h_have = true;
  };
  // Blocking: only the threads that own H elements load them (store_h and the epilogue go
  // through LDS after a barrier).
  auto load_h = [&]() __attribute__((always_inline)) {
    if (!h_owner || h_have) return;
    if (a.h_blocks > 0) {
      if (lane == 0) {
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
      fetch_h();
    } else {
#pragma unroll
      for (int u = 0; u < kHB; ++u) hv[u] = a.H[min((int)threadIdx.x + 256 * u, a.M * a.r - 1)];
      h_have = true;
    }
  };

  // Outliers: corr[i] = sum over the thread's entries of delta * x[i, col], summed over the
  // TPR threads of the row by a butterfly (each holds the row's sum).
  float corr[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) corr[i] = 0.f;
  auto outlier_pass = [&]() __attribute__((always_inline)) {
    if (!csr) return;
    const int xc0 = s0 * 128;
    auto entry = [&](uint32_t col, float d) __attribute__((always_inline)) {
      const int xi = (int)col - xc0;  // activations are staged in natural column order
#pragma unroll
      for (int i = 0; i < MB; ++i)
        if (i < a.M) corr[i] += d * h2f(xs[i * a.xstride + xi]);
    };
#pragma unroll
    for (int u = 0; u < kEB; ++u)
      if (e0 + jr + TPR * u < e1) entry(ecol[u], edel[u]);
    for (int e = e0 + jr + TPR * kEB; e < e1; e += TPR) entry(a.gcol[e], a.delta[e]);
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if (i < a.M) {
        float v = corr[i];
#pragma unroll
        for (int m = TPR / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m);
        corr[i] = v;
      }
    }
  };

  // Steady state: every slot consumed is reloaded kPF slabs ahead; then one round with
  // conditional reloads and a last round without (nw is wave-uniform).
  int j0 = 0;
  for (; j0 + 2 * kPF <= nw; j0 += kPF) {
#pragma unroll
    for (int u = 0; u < kPF; ++u) {
      consume(buf[u], s0 + ph + WPT * (j0 + u));
      load_slab(buf[u], s0 + ph + WPT * (j0 + u + kPF));
      __builtin_amdgcn_sched_barrier(0);  // keep each reload right behind its slot's use
    }
  }
  if (j0 < nw) {
#pragma unroll
    for (int u = 0; u < kPF; ++u) {
      if (j0 + u < nw) {
        consume(buf[u], s0 + ph + WPT * (j0 + u));
        if (j0 + u + kPF < nw) load_slab(buf[u], s0 + ph + WPT * (j0 + u + kPF));
      }
    }
    j0 += kPF;
#pragma unroll
    for (int u = 0; u < kPF; ++u)
      if (j0 + u < nw) consume(buf[u], s0 + ph + WPT * (j0 + u));
  }

  // Wave partials: red[wave][g][e][lane] = D[i = 16 g + 4 kq + e][row r].
#pragma unroll
  for (int g = 0; g < NA; ++g)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[((wave * NA + g) * 4 + e) * 64 + lane] = acc[g][e];

  auto store_h = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kHB; ++u)
      if ((int)threadIdx.x + 256 * u < a.M * a.r) hs[threadIdx.x + 256 * u] = hv[u];
  };
  // One K split (or H given): this block finishes its rows and needs H now; the loads overlap
  // the outlier pass when it has not run yet.  Several splits: only the last to arrive needs H.
  const bool h_early = a.r > 0 && (a.splits == 1 || a.h_blocks == 0);
  if (h_early) load_h();
  outlier_pass();
  __syncthreads();
  // Count the block as a consumer of its ready slot as soon as every wave's poll is done (the
  // barrier above), so the atomic's round trip overlaps the epilogue; the slot's last
  // consumer lowers it at the end, for the next call.
  uint32_t cons_old = 0u;
  bool counted = false;
  auto count_consumer = [&]() __attribute__((always_inline)) {
    if (h_fused && threadIdx.x == 0) {
      cons_old = atomicAdd(slot + 1, 1u);
      counted = true;
    }
  };
  if (h_early) count_consumer();

  // Wave partial of output (i, row rr) in phase p.
  auto red_at = [&](int i, int rr, int p) __attribute__((always_inline)) -> float& {
    const int ln = (rr & 15) + 16 * ((i & 15) >> 2);
    return red[((((rr >> 4) * WPT + p) * NA + (i >> 4)) * 4 + (i & 3)) * 64 + ln];
  };
  // H over the x rows (read by the outlier pass above, so after its barrier).
  if (h_early) store_h();
  // The outlier sum of (i, rho), which every thread of the row's group holds after the
  // butterfly, is added by thread jr = i % TPR into the last phase's partial.
  if (csr) {
#pragma unroll
    for (int q = 0; q < (MB + TPR - 1) / TPR; ++q) {
      const int i = q * TPR + jr;
      if (i < a.M) {
        float c = 0.f;
#pragma unroll
        for (int u = 0; u < TPR; ++u)
          if (q * TPR + u < MB && u == jr) c = corr[min(q * TPR + u, MB - 1)];
        red_at(i, rho, WPT - 1) += c;
      }
    }
  }
  if (csr || h_early) __syncthreads();

  // Block sums for the outputs (i, rr), o = i * ROWS + rr: wave partials in phase order.
  const int nouts = a.M * ROWS;
  constexpr int kOPT = (MB * ROWS + 255) / 256;  // outputs per thread
  float v[kOPT];
#pragma unroll
  for (int q = 0; q < kOPT; ++q) {
    const int o = (int)threadIdx.x + 256 * q;
    v[q] = 0.f;
    if (o < nouts) {
      const int i = o / ROWS;
      const int rr = o - i * ROWS;
      float s = 0.f;
#pragma unroll
      for (int p = 0; p < WPT; ++p) s += red_at(i, rr, p);
      v[q] = s;
    }
  }

  if (a.splits > 1) {
#pragma unroll
    for (int q = 0; q < kOPT; ++q) {
      const int o = (int)threadIdx.x + 256 * q;
      if (o < nouts) {
        const int i = o / ROWS;
        const int n = tb * ROWS + (o - i * ROWS);
        if (n < a.N) store_dev(a.partial + ((size_t)split * a.M + i) * a.N + n, v[q]);
      }
    }
    stores_done();
    __syncthreads();
    __shared__ int s_last;
    if (threadIdx.x == 0) {
      const uint32_t old = atomicAdd(a.sync + kSyncTile + tb, 1u);
      if (old >= (uint32_t)a.splits) {  // counters not zero at entry: this block writes the rows as NaN
        raise_error(a.sync, kErrArrivals);
        s_err = 1;
      }
      s_last = old == (uint32_t)(a.splits - 1) || old >= (uint32_t)a.splits;
    }
    __syncthreads();
    if (!s_last) return;
    compiler_fence();
    // the sticky error word, read together with the partials
    uint32_t err = 0u;
    if (threadIdx.x == 0) err = load_dev(a.sync + kSyncErr);
    // Sum the split partials in split order, kSumBatch splits of every output in flight at once
    // (clamped addresses; the sums take only splits < a.splits).
    constexpr int kSumBatch = 8;
    size_t base[kOPT];
#pragma unroll
    for (int q = 0; q < kOPT; ++q) {
      const int o = min((int)threadIdx.x + 256 * q, nouts - 1);
      const int i = o / ROWS;
      const int n = min(tb * ROWS + (o - i * ROWS), a.N - 1);
      base[q] = (size_t)i * a.N + n;
      v[q] = 0.f;
    }
    const size_t sstride = (size_t)a.M * a.N;
    for (int sp0 = 0; sp0 < a.splits; sp0 += kSumBatch) {
      float t[kOPT][kSumBatch];
#pragma unroll
      for (int q = 0; q < kOPT; ++q)
#pragma unroll
        for (int u = 0; u < kSumBatch; ++u)
          t[q][u] = load_dev(a.partial + (size_t)min(sp0 + u, a.splits - 1) * sstride + base[q]);
#pragma unroll
      for (int q = 0; q < kOPT; ++q)
#pragma unroll
        for (int u = 0; u < kSumBatch; ++u)
          if (sp0 + u < a.splits) v[q] += t[q][u];
    }
    if (threadIdx.x == 0) {
      store_dev(a.sync + kSyncTile + tb, 0u);
      if (err != 0u) s_err = 1;
    }
    if (a.r > 0 && !h_early) {  // the last split block: computed H now
      load_h();
      store_h();
    }
    __syncthreads();
    if (!h_early) count_consumer();
  }

  // Epilogue: y = fp16_rn((v + s * H[i, :] . B[n, :]) * gamma[n]) with H, B and gamma from LDS;
  // NaN rows when this call or an earlier one on the workspace failed a hand-off.
  const bool poisoned = s_err != 0;
#pragma unroll
  for (int q = 0; q < kOPT; ++q) {
    const int o = (int)threadIdx.x + 256 * q;
    if (o < nouts) {
      const int i = o / ROWS;
      const int rr = o - i * ROWS;
      const int n = tb * ROWS + rr;
      if (n < a.N) {
        float y = v[q];
        if (a.r > 0) {
          float ls = 0.f;
          const float* hi = hs + i * a.r;
          const uint16_t* bb = bs + rr * a.r;
          for (int j = 0; j < a.r; j += 8) {
            const u32x4_t b8 = *reinterpret_cast<const u32x4_t*>(bb + j);
            const uint32_t w4[4] = {b8.x, b8.y, b8.z, b8.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              ls += hi[j + 2 * e] * h2f((uint16_t)(w4[e] & 0xFFFFu));
              ls += hi[j + 2 * e + 1] * h2f((uint16_t)(w4[e] >> 16));
            }
          }
          y = (y + a.scale * ls) * h2f(gs[rr]);
        }
        a.out[(size_t)i * a.N + n] = poisoned ? kHalfNaN : f2h_rn(y);
      }
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

// ---------------------------------------------------------------- preparation

// Every word holds the 8 codes of 8 consecutive columns in the selector-ready encoding of
// wlq_device.h (sel_encode_byte); 4-bit codes come from the row-aligned words (code c at
// bits 4c), 3-bit codes from the ten-per-word layout (values 0..7), columns >= K as code 0.
__global__ __launch_bounds__(256) void prep_codes_kernel(const uint32_t* __restrict__ q, int N, int K, int wpr,
                                                         int bits, int T, int S, u32x4_t* __restrict__ codes) {
  const size_t total = (size_t)T * S * 64;
  for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
    const int l = (int)(idx & 63);
    const size_t ts = idx >> 6;
    const int s = (int)(ts % (size_t)S);
    const int t = (int)(ts / (size_t)S);
    const int n = 16 * t + (l & 15);
    const int w0 = 16 * s + 4 * (l >> 4);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (n < N) {
      const uint32_t* qrow = q + (size_t)n * wpr;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t c[8];
        for (int i = 0; i < 8; ++i) {
          const int col = 8 * (w0 + j) + i;
          uint32_t code = 0u;
          if (col < K) code = bits == 4 ? (qrow[col >> 3] >> (4 * (col & 7))) & 15u : (qrow[col / 10] >> (3 * (col % 10))) & 7u;
          c[i] = code;
        }
        w[j] = sel_encode_byte(c, 0) | (sel_encode_byte(c, 1) << 8) | (sel_encode_byte(c, 2) << 16) |
               (sel_encode_byte(c, 3) << 24);
      }
    }
    codes[idx] = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

// nl = LUT entries per (row, group): 16, or 8 for 3-bit (entries 8..15 of the planes stay 0).
__global__ __launch_bounds__(256) void prep_planes_kernel(const uint16_t* __restrict__ lut, int N, int ng, int nl,
                                                          int T, u32x4_t* __restrict__ planes) {
  const size_t total = (size_t)T * ng * 32;
  for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
    const int rr = (int)(idx & 15);
    const int p = (int)((idx >> 4) & 1);
    const size_t tg = idx >> 5;
    const int g = (int)(tg % (size_t)ng);
    const int t = (int)(tg / (size_t)ng);
    const int n = 16 * t + rr;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (n < N) {
      // the row's 16 (or 8) fp16 entries as 16-byte loads (rows of 32 / 16 bytes)
      const uint16_t* e = lut + ((size_t)n * ng + g) * nl;
      uint32_t raw[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
      const u32x4_t a0 = *reinterpret_cast<const u32x4_t*>(e);
      raw[0] = a0.x; raw[1] = a0.y; raw[2] = a0.z; raw[3] = a0.w;
      if (nl == 16) {
        const u32x4_t a1 = *reinterpret_cast<const u32x4_t*>(e + 8);
        raw[4] = a1.x; raw[5] = a1.y; raw[6] = a1.z; raw[7] = a1.w;
      }
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const uint32_t v = (raw[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
        const uint32_t b = p ? (v >> 8) : (v & 0xFFu);
        w[k >> 2] |= b << (8 * (k & 3));
      }
    }
    planes[idx] = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

// One thread per (row, chunk): the chunk's entries get their column and delta.
__global__ __launch_bounds__(256) void prep_outliers_kernel(const uint32_t* __restrict__ q,
                                                            const uint16_t* __restrict__ lut,
                                                            const int32_t* __restrict__ offsets,
                                                            const uint16_t* __restrict__ cols,
                                                            const uint8_t* __restrict__ vals, int N, int K, int wpr,
                                                            int bits, int ng, int G, int nch, int chunk,
                                                            uint16_t* __restrict__ gcol,
                                                            float* __restrict__ delta) {
  const size_t total = (size_t)N * nch;
  for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
    const int n = (int)(idx / (size_t)nch);
    const int c = (int)(idx - (size_t)n * nch);
    const int32_t* offr = offsets + (size_t)n * (nch + 1);
    const int e_lo = offr[c];
    const int e_hi = offr[c + 1];
    const uint32_t* qrow = q + (size_t)n * wpr;
    for (int e = e_lo; e < e_hi; ++e) {
      const int cl = (int)cols[e];
      const int col = c * chunk + cl;
      if (cl < chunk && col < K) {
        const uint32_t code = bits == 4 ? (qrow[col >> 3] >> (4 * (col & 7))) & 15u
                                        : (qrow[col / 10] >> (3 * (col % 10))) & 7u;
        const int g = G > 0 ? min(col / G, ng - 1) : 0;
        const float w_true = h2f((uint16_t)((uint32_t)vals[e] << 8));
        gcol[e] = (uint16_t)col;
        delta[e] = w_true - h2f(lut[(((size_t)n * ng + g) << bits) + code]);
      } else {  // dropped (the reference drops col >= K; a chunk column >= the chunk width is malformed)
        gcol[e] = (uint16_t)(c * chunk);
        delta[e] = 0.f;
      }
    }
  }
}

// Patch lists of the M = 9..128 kernel, one thread per (tile t, slab s): the entries of
// the tile's 16 rows in the chunk holding the slab, kept when they fall in the slab,
// inside K and are not overwritten by a later entry of the row.  COUNT pass: wpidx[ts] =
// number kept; FILL pass (after the scan): the patches at wpidx[ts] onwards.
template <bool FILL>
__global__ __launch_bounds__(256) void prep_wpatch_kernel(const int32_t* __restrict__ offsets,
                                                          const uint16_t* __restrict__ cols,
                                                          const uint8_t* __restrict__ vals, int N, int K, int nch,
                                                          int chunk, int T, int S, uint32_t* __restrict__ wpidx,
                                                          uint32_t* __restrict__ wpatch) {
  const size_t total = (size_t)T * S;
  const int spc = chunk / 128;
  for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
    const int t = (int)(idx / (size_t)S);
    const int s = (int)(idx - (size_t)t * S);
    const int c = s / spc;
    const int sc = s - c * spc;  // slab within the chunk
    uint32_t pos = FILL ? wpidx[idx] : 0u;
    for (int rr = 0; rr < 16; ++rr) {
      const int n = 16 * t + rr;
      if (n >= N) break;
      const int32_t* offr = offsets + (size_t)n * (nch + 1);
      const int e_lo = offr[c];
      const int e_hi = offr[c + 1];
      for (int e = e_lo; e < e_hi; ++e) {
        const int cl = (int)cols[e];
        if (cl >= chunk || c * chunk + cl >= K || (cl >> 7) != sc) continue;
        bool later = false;
        for (int e2 = e + 1; e2 < e_hi && !later; ++e2) later = (int)cols[e2] == cl;
        if (later) continue;
        if (FILL) {
          const uint32_t cs = (uint32_t)cl & 127u;
          wpatch[pos] = ((uint32_t)rr + 16u * (cs >> 5)) | ((cs & 31u) << 6) | ((uint32_t)vals[e] << 24);
        }
        ++pos;
      }
    }
    if (!FILL) wpidx[idx] = pos;
  }
}

// In-place exclusive prefix sums of v[0, n) by one block; v[n] = the total.
__global__ __launch_bounds__(1024) void prep_scan_kernel(uint32_t* __restrict__ v, int n) {
  __shared__ uint32_t part[1024];
  const int per = (n + 1023) / 1024;
  const int b = (int)threadIdx.x * per;
  const int e = min(n, b + per);
  uint32_t sum = 0u;
  for (int i = b; i < e; ++i) sum += v[i];
  part[threadIdx.x] = sum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const uint32_t add = threadIdx.x >= (unsigned)off ? part[threadIdx.x - off] : 0u;
    __syncthreads();
    part[threadIdx.x] += add;
    __syncthreads();
  }
  uint32_t run = part[threadIdx.x] - sum;
  for (int i = b; i < e; ++i) {
    const uint32_t c = v[i];
    v[i] = run;
    run += c;
  }
  if (threadIdx.x == 1023) v[n] = part[1023];
}

template <int LM, int TPB, int MB>
hipError_t launch_tpl(const StreamArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((stream4_kernel<LM, TPB, MB>), grid, dim3(256), lds, stream, a);
  return hipGetLastError();
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

// ------------------------------------------------------------------ host side

bool prepared_supported(int N, int K, int bits, int group_size) {
  if ((bits != 4 && bits != 3) || N <= 0 || K <= 0 || K % 8 != 0 || K > 65535) return false;
  // a group covers whole 32-column lane segments and at least one 3-bit code window (40 columns)
  return group_size == 0 || (group_size % 32 == 0 && group_size >= (bits == 3 ? 40 : 32));
}

PreparedLayout prepared_layout(int N, int K, int group_size, int64_t nnz) {
  PreparedLayout p{};
  p.T = (N + 15) / 16;
  p.S = (K + 127) / 128;
  p.ng = group_size > 0 ? (K + group_size - 1) / group_size : 1;
  p.codes_off = 0;
  p.planes_off = align256((size_t)p.T * p.S * 1024);
  p.gcol_off = p.planes_off + align256((size_t)p.T * p.ng * 512);
  p.delta_off = p.gcol_off + align256((size_t)nnz * 2);
  p.wpidx_off = p.delta_off + align256((size_t)nnz * 4);
  p.wpatch_off = p.wpidx_off + align256(((size_t)p.T * p.S + 1) * 4);
  p.bytes = p.wpatch_off + align256((size_t)nnz * 4);
  return p;
}

hipError_t launch_prepare(const Layer& L, int64_t nnz, void* prepared, hipStream_t stream) {
  const PreparedLayout p = prepared_layout(L.N, L.K, L.group_size, nnz);
  char* base = reinterpret_cast<char*>(prepared);
  auto grid_for = [](size_t total) { return dim3((unsigned)std::min<size_t>((total + 255) / 256, 65535)); };
  const int ng = L.group_size > 0 ? L.ng : 1;
  hipLaunchKernelGGL(prep_codes_kernel, grid_for((size_t)p.T * p.S * 64), dim3(256), 0, stream, L.q, L.N, L.K, L.wpr,
                     L.bits, p.T, p.S, reinterpret_cast<u32x4_t*>(base + p.codes_off));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(prep_planes_kernel, grid_for((size_t)p.T * ng * 32), dim3(256), 0, stream, L.lut, L.N, ng,
                     1 << L.bits, p.T, reinterpret_cast<u32x4_t*>(base + p.planes_off));
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (L.offsets != nullptr && nnz > 0) {
    hipLaunchKernelGGL(prep_outliers_kernel, grid_for((size_t)L.N * L.nch), dim3(256), 0, stream, L.q, L.lut,
                       L.offsets, L.cols, L.vals, L.N, L.K, L.wpr, L.bits, ng, L.group_size, L.nch, L.chunk,
                       reinterpret_cast<uint16_t*>(base + p.gcol_off), reinterpret_cast<float*>(base + p.delta_off));
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    // patch lists: counts per (tile, slab), prefix sums in place, then the patches
    uint32_t* wpidx = reinterpret_cast<uint32_t*>(base + p.wpidx_off);
    uint32_t* wpatch = reinterpret_cast<uint32_t*>(base + p.wpatch_off);
    const size_t ts = (size_t)p.T * p.S;
    hipLaunchKernelGGL(prep_wpatch_kernel<false>, grid_for(ts), dim3(256), 0, stream, L.offsets, L.cols, L.vals, L.N,
                       L.K, L.nch, L.chunk, p.T, p.S, wpidx, wpatch);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(prep_scan_kernel, dim3(1), dim3(1024), 0, stream, wpidx, (int)ts);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(prep_wpatch_kernel<true>, grid_for(ts), dim3(256), 0, stream, L.offsets, L.cols, L.vals, L.N,
                       L.K, L.nch, L.chunk, p.T, p.S, wpidx, wpatch);
    e = hipGetLastError();
  }
  return e;
}

StreamPlan plan_stream(int N, int K, int M, int cu_count, int fused_rank, int chunk) {
  StreamPlan p{};
  const int T = (N + 15) / 16;
  const int nch = (K + chunk - 1) / chunk;
  // M <= 2: a K split costs a partial round trip that outweighs the parallelism it adds unless the
  // layer has very few tiles; larger M: ~4 blocks per CU.
  const int target = M <= 2 ? std::max(1, cu_count / WLQ_STREAM_CUS_PER_BLOCK_M2) : kBlocksPerCU * std::max(1, cu_count);
  // M <= 2: two row tiles per block (14 slabs per wave at K = 3584 instead of 7) halve the
  // per-block overhead (activation staging, completion) wherever that still leaves target blocks
  // (gate_up 33.2 -> 29.2 us); larger M: a tile per wave (two per block measured slower there).
  p.tpb = M > 2 ? 4 : (T / 2 >= target ? 2 : 1);
  const int TB = (T + p.tpb - 1) / p.tpb;
  int splits = std::max(1, std::min(nch, (target + TB - 1) / TB));
  int cps = (nch + splits - 1) / splits;
  const int cps_max = std::max(1, kXBudget / (M * chunk * 2));
  cps = std::min(cps, cps_max);
  splits = (nch + cps - 1) / cps;
  p.splits = splits;
  p.cps = cps;
  p.TB = TB;
  p.h_blocks = fused_rank > 0 ? (K + kHCols - 1) / kHCols : 0;
  const size_t hf = fused_rank > 0 ? align256((size_t)M * fused_rank * 4) : 0;
  const size_t hp = fused_rank > 0 ? align256((size_t)p.h_blocks * M * fused_rank * 4) : 0;
  const size_t part = splits > 1 ? (size_t)splits * M * N * 4 : 0;
  p.hfin_off = 0;
  p.hpart_off = hf;
  p.partial_off = hf + hp;
  p.workspace_bytes = hf + hp + part;
  // the block's threads stage the activations with kXR (M > 16: 2 kXR) 16-byte loads each
  const bool staged = (size_t)M * cps * (chunk / 8) <= (size_t)256 * kXR * (M > 16 ? 2 : 1);
  p.ok = M >= 1 && M <= stream_max_m() && (chunk == 512 || chunk == 640) && staged &&
         (splits == 1 || TB <= kSyncErrorWord - kSyncTile) && fused_rank % 8 == 0 && fused_rank <= kMaxRank;
  return p;
}

int stream_max_m() { return 32; }
int stream_max_rank() { return kMaxRank; }

hipError_t launch_stream(const Layer& L, const void* prepared, int64_t nnz, const Dora& D, const uint16_t* x,
                         uint16_t* out, int M, const StreamPlan& plan, float* workspace, uint32_t* sync,
                         hipStream_t stream) {
  const PreparedLayout lay = prepared_layout(L.N, L.K, L.group_size, nnz);
  const char* base = reinterpret_cast<const char*>(prepared);
  StreamArgs a{};
  a.codes = reinterpret_cast<const u32x4_t*>(base + lay.codes_off);
  a.planes = reinterpret_cast<const u32x4_t*>(base + lay.planes_off);
  const bool csr = L.offsets != nullptr && nnz > 0;
  a.gcol = reinterpret_cast<const uint16_t*>(base + lay.gcol_off);
  a.delta = reinterpret_cast<const float*>(base + lay.delta_off);
  a.offsets = csr ? L.offsets : nullptr;
  a.x = x;
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
  a.nch = (L.K + L.chunk - 1) / L.chunk;
  a.spc = L.chunk / 128;
  a.T = lay.T;
  a.TB = plan.TB;
  a.g_magic = L.group_size > 0 ? (uint32_t)((0x100000000ull / (uint64_t)L.group_size) + 1ull) : 0u;
  a.splits = plan.splits;
  a.cps = plan.cps;
  a.xstride = plan.cps * L.chunk + 8;
  const bool fused_h = D.r > 0 && D.H == nullptr;
  a.h_blocks = fused_h ? plan.h_blocks : 0;
  char* ws = reinterpret_cast<char*>(workspace);
  a.hfin = reinterpret_cast<float*>(ws + plan.hfin_off);
  a.hpart = reinterpret_cast<float*>(ws + plan.hpart_off);
  a.partial = reinterpret_cast<float*>(ws + plan.partial_off);
  a.sync = sync;
  a.spin_limit = spin_limit();
  a.withhold_h = withhold_h() ? 1 : 0;
  const int rows = 16 * plan.tpb;
  const int mb = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : M <= 16 ? 16 : 32;
  const int na = (mb + 15) / 16;
  // the x rows (>= 1040 bytes per activation row) also hold H (<= 256 bytes per row) at the end
  size_t lds = (((size_t)M * a.xstride * 2 + 15) & ~(size_t)15) + 64 + (size_t)4 * na * 256 * 4 +
               (size_t)rows * D.r * 2 + (size_t)rows * 2;
  if (fused_h) lds = std::max(lds, (size_t)4 * na * (kMaxRank / 16) * 4 * 64 * 4);
  const dim3 grid(a.h_blocks + plan.TB * plan.splits);
  const bool per_row = L.group_size <= 0 || lay.ng == 1;
  if (per_row) a.ng = 1;
  int gshift = 0;
  while (gshift < 5 && (128 << gshift) < L.group_size) ++gshift;
  const bool slab_groups = !per_row && L.group_size == (128 << gshift);
  a.gshift = gshift;
#define WLQ_STREAM_DISPATCH(PR)                                                  \
  if (plan.tpb == 2) {                                                          \
    if (mb == 1) return launch_tpl<PR, 2, 1>(a, grid, lds, stream);             \
    return launch_tpl<PR, 2, 2>(a, grid, lds, stream);                          \
  }                                                                             \
  if (plan.tpb == 1) {                                                          \
    if (mb == 1) return launch_tpl<PR, 1, 1>(a, grid, lds, stream);             \
    return launch_tpl<PR, 1, 2>(a, grid, lds, stream);                          \
  }                                                                             \
  if (mb <= 4) return launch_tpl<PR, 4, 4>(a, grid, lds, stream);               \
  if (mb == 8) return launch_tpl<PR, 4, 8>(a, grid, lds, stream);               \
  if (mb == 16) return launch_tpl<PR, 4, 16>(a, grid, lds, stream);             \
  return launch_tpl<PR, 4, 32>(a, grid, lds, stream);
  if (per_row) {
    WLQ_STREAM_DISPATCH(0)
  } else if (slab_groups) {
    WLQ_STREAM_DISPATCH(2)
  } else {
    WLQ_STREAM_DISPATCH(1)
  }
#undef WLQ_STREAM_DISPATCH
}

}  // namespace wlq
