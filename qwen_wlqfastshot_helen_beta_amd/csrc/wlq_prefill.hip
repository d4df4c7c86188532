// Prefill-shaped product (M > 128 activation rows) on the prepared (tile-contiguous) layout.
//
// Reference behaviour replaced: the M >= 16 branch of gemm_forward
// (csrc/vllm_binding.cpp:355-393: full-matrix dequant into a workspace, cuBLAS HGEMM, fused
// DoRA epilogue), with gemm_metalog_dora_kernel's overwrite semantics for outliers
// (csrc/gemm_kernel.cu:204-228): W0 expanded through the LUTs, outlier positions overwritten
// by fp16(e5m2 << 8), y = fp16((X.W0^T + s * H.B^T) * gamma) with H = fp16(X.A^T).
//
// Design.  W never goes through LDS.  Block tile = 128 activation rows x 256 W rows, eight
// waves (two per SIMD), wave w owning W rows 32 w .. 32 w + 31 of the block (one 32-row pair).
// Per 128-column slab a wave loads its pair's codes straight from the prepared layout (each lane
// two 16-byte loads), dequantizes them in registers (dequant_word4s) into the B operands of
// V_MFMA_F32_32X32X16_F16 and multiplies them with the four 32-row groups of the activation
// slab, read from LDS as the A operands: each dequantized W word feeds 4 x 32 activation rows.
// An MFMA holds its own wave's issue for most of its duration, so a wave's lookups and its MFMAs
// serialize; the second wave on the SIMD fills that time (measured: one wave per SIMD with two
// pairs each ran gate_proj at M = 2048 in 372 us, two waves with one pair each in 321 us).
// The dequant of half a slab runs beside the MFMAs of the other half (half-slab pipeline).
//
// Operand order.  The prepared layout holds a 16-row tile's slab in the lane order of the
// 16x16x32 MFMA: lane L = r + 16 kq, word q covers columns 32 kq + 8 q .. +7 of row r.  For
// the 32x32x16 MFMA, lane l = n + 32 kh (n = W row of the pair, kh = K half) takes, for K16
// step j = 4 jj + q, word q of source lane (n % 16) + 16 (kh + 2 jj) of tile n / 16: columns
// 32 (kh + 2 jj) + 8 q .. +7, i.e. activation unit 8 jj + 4 kh + q.  Every (source lane,
// word) is used exactly once per slab; A and B agree on the column of every product.
//
// Activations: double-buffered 128-row slabs in LDS (16-byte units XOR-swizzled by row so the
// 32 rows of a fragment read hit distinct banks), loaded by all 512 threads into registers
// one slab ahead and written at the top of the next iteration; rows >= M and columns >= K
// read as zeros through the buffer range check.  One barrier per slab.
//
// Outliers: the prepared patch lists per (16-row tile, slab).  A wave writes its dequantized
// words to a wave-private LDS scratch in the source-lane order of the prepared layout, applies
// the patches (one per lane and tile; a wave whose lists exceed 64 entries in its split runs a
// loop instance that continues from global memory) and reads the words back as B operands.
//
// DoRA H: DoRA blocks at the front of the grid compute, per 128-row activation block, shares
// of X.A^T over strided 32-column steps; the last share of an activation block sums them in
// share order, rounds H to fp16 and raises that block's ready slot.  The block that finishes
// an output tile polls its slot before the epilogue (normally long raised by then).
//
// K splits only for layers longer than one split holds (> 191 slabs): fp32 partials in the
// accumulator register layout, summed in split order by the last arrival of the tile.  Failures of the hand-offs set the
// workspace's sticky error word and the rows concerned are written as fp16 NaN, as in the
// decode kernel.
//
// Blocks are mapped so that each XCD works through a contiguous range of output tiles in
// groups of 4 W blocks x all activation blocks: the blocks resident on one XCD share W slabs
// and activation slabs in its L2.
#include <algorithm>
#include <type_traits>

#include "wlq_device.h"
#include "wlq_internal.h"

namespace wlq {
namespace {

typedef float float16v_t __attribute__((ext_vector_type(16)));

constexpr int kCW = 8;                   // waves per block, two per SIMD
constexpr int kThreads = 64 * kCW;
constexpr int MB = 128;                  // activation rows per block
constexpr int kMG = MB / 32;             // 32-row activation groups
constexpr int kPairs = 1;                // 32-row W pairs per wave
constexpr int kTilesW = 2 * kPairs;      // 16-row W tiles per wave
constexpr int kTiles = kCW * kTilesW;    // per block
constexpr int kBlockRows = 16 * kTiles;  // 256 W rows per block
constexpr int kPF = 2;                   // W slabs in flight per wave
constexpr int kXU = MB * 16 / kThreads;  // 16-byte activation units per thread and slab
constexpr int kSlabBytes = MB * 256;     // one activation slab in LDS
constexpr int kScratchHalves = 2 * kPairs * 2 * 4 * 32 * 8 + 64;  // per wave: 2 half-slab regions + spare slots
constexpr int kMaxSlabs = 191;           // slabs per K split (patch-list starts in 3 lane registers)
constexpr int kMaxRank = 64;
constexpr int kGroupN = 4;               // W blocks per tile group of the block order
constexpr int kXcds = 8;
constexpr int kEpiStride = 72;           // fp16 per LDS row of H parts and B rows
constexpr int kOutStride = kBlockRows + 8;
constexpr int kSc1 = 16;                 // buffer cache-policy bit sc1: device-coherent
constexpr uint16_t kHalfNaN = 0x7E00u;
constexpr uint32_t kOutOfRange = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;

// LDS (bytes).  Main loop: two activation slabs, then the waves' scratch.  Epilogue (reuses
// the front): H high / low parts [MB][kEpiStride], B rows [kBlockRows][kEpiStride], gamma,
// the output tile [MB][kOutStride].  DoRA blocks: the wave sums.
constexpr int kLdsX = 0;
constexpr int kLdsScratch = 2 * kSlabBytes;
constexpr int kLdsMain = kLdsScratch + kCW * kScratchHalves * 2;
constexpr int kEpiHi = 0;
constexpr int kEpiLo = kEpiHi + MB * kEpiStride * 2;
constexpr int kEpiB = kEpiLo + MB * kEpiStride * 2;
constexpr int kEpiG = kEpiB + kBlockRows * kEpiStride * 2;
constexpr int kEpiOut = kEpiG + kBlockRows * 2;
constexpr int kEpiBytes = kEpiOut + MB * kOutStride * 2;
constexpr int kDW = 4;                   // waves of a DoRA block that compute
constexpr int kDoraRed = kDW * (MB / 16) * (kMaxRank / 16) * 4 * 64 * 4;
constexpr int kLdsBytes = std::max(std::max(kLdsMain, kEpiBytes), kDoraRed);
static_assert(kLdsBytes <= 160 * 1024, "one block per CU");

struct PrefillArgs {
  const u32x4_t* codes;
  const u32x4_t* planes;
  const uint32_t* wpidx;    // patch-list starts per (tile, slab), T * S + 1
  const uint32_t* wpatch;   // patches (null with no outliers)
  uint32_t patch_bytes;
  const uint16_t* X;
  uint16_t* out;
  const uint16_t* B;
  const float* H;           // caller's H, or null (DoRA blocks compute it when A is set)
  const uint16_t* gamma;
  const uint16_t* A;
  float scale;
  int r;
  int M, N, K, S, ng, T;
  int gshift;               // LUT group = slab >> gshift (groups of 128 << gshift columns)
  int nblk, mblk, tiles;    // W blocks, activation blocks, output tiles (nblk * mblk)
  int splits, sps;          // K splits, slabs per split
  int blocks;               // tiles * splits (the grid holds up to kXcds - 1 more, idle)
  int per_xcd;              // ceil(blocks / kXcds)
  int hk, h_blocks;         // DoRA shares per activation block, DoRA blocks (mblk * hk)
  float* partial;           // [splits][tiles][kCW][kPairs][kMG][64] x 16 fp32
  uint32_t partial_bytes;
  int out_vec;
  float* hpart;             // [h_blocks][MB][r]
  float* hfin;              // [M][r]
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
__device__ __forceinline__ void raw_barrier() {
  compiler_fence();
  __builtin_amdgcn_s_barrier();
  compiler_fence();
}

__device__ __forceinline__ float16v_t mfma32x32x16(u32x4_t a, u32x4_t b, float16v_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}

// ------------------------------------------------------------------ DoRA blocks
// hpart[d, i, j] = share d % hk of X[128 (d / hk) + i, :] . A[j, :] over the 32-column steps
// (d % hk) kDW + w + t hk kDW of wave w < kDW (MFMA 16x16x32, natural column order), wave sums added
// through LDS.  The last share of activation block mb to arrive sums the shares in share order,
// rounds H = fp16(sum) and raises the block's ready slot.
__device__ void prefill_dora_block(const PrefillArgs& a, int d, float* red) {
  constexpr int NA = MB / 16;
  constexpr int JT = kMaxRank / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int jt_n = (a.r + 15) >> 4;
  const int mb = d / a.hk;
  const int share = d - mb * a.hk;
  const int row0 = mb * MB;
  float4_t acc[NA][JT];
#pragma unroll
  for (int g = 0; g < NA; ++g)
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) acc[g][jt] = float4_t{0.f, 0.f, 0.f, 0.f};
  const int nks = (a.K + 31) / 32;
  for (int ks = share * kDW + wave; wave < kDW && ks < nks; ks += a.hk * kDW) {
    const int k = 32 * ks + 8 * kq;
    const bool kin = k < a.K;  // K % 8 == 0
    u32x4_t xa[NA];
#pragma unroll
    for (int g = 0; g < NA; ++g) {
      const int i = row0 + 16 * g + r16;
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
  if (wave < kDW)
#pragma unroll
    for (int g = 0; g < NA; ++g)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
        if (jt < jt_n)
#pragma unroll
          for (int e = 0; e < 4; ++e) red[(((wave * NA + g) * JT + jt) * 4 + e) * 64 + lane] = acc[g][jt][e];
  __syncthreads();
  float* hp = a.hpart + (size_t)d * MB * a.r;
  for (int idx = threadIdx.x; idx < NA * jt_n * 256; idx += kThreads) {
    const int ln = idx & 63;
    const int e = (idx >> 6) & 3;
    const int jt = (idx >> 8) % jt_n;
    const int g = (idx >> 8) / jt_n;
    const int i = 16 * g + 4 * (ln >> 4) + e;
    const int j = 16 * jt + (ln & 15);
    if (j < a.r) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kDW; ++w) v += red[(((w * NA + g) * JT + jt) * 4 + e) * 64 + ln];
      store_dev(hp + i * a.r + j, v);
    }
  }
  stores_done();
  __syncthreads();
  __shared__ int s_last;
  uint32_t* cnt = a.sync + kSyncTile + mb;
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(cnt, 1u);
    if (old >= (uint32_t)a.hk) raise_error(a.sync, kErrArrivals);  // no finisher: the H waits run out
    s_last = old == (uint32_t)(a.hk - 1);
  }
  __syncthreads();
  if (!s_last) return;
  compiler_fence();
  const int rows = min(MB, a.M - row0);
  const float* hp0 = a.hpart + (size_t)mb * a.hk * MB * a.r;
  for (int idx = threadIdx.x; idx < rows * a.r; idx += kThreads) {
    float v = 0.f;
    for (int u0 = 0; u0 < a.hk; u0 += 8) {
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = load_dev(hp0 + (size_t)min(u0 + u, a.hk - 1) * MB * a.r + idx);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (u0 + u < a.hk) v += t[u];
    }
    store_dev(a.hfin + (size_t)row0 * a.r + idx, h2f(f2h_rn(v)));  // the reference's F.linear output is fp16
  }
  stores_done();
  __syncthreads();
  if (threadIdx.x == 0) {
    if (!a.withhold_h) store_dev(a.sync + kSyncSlot0 + kSlotWords * mb, 1u);
    store_dev(cnt, 0u);
  }
}

// --------------------------------------------------------------- tile blocks

// One slab of a wave's two pairs as loaded: per pair the lane's two code vectors (source
// lanes (n % 16) + 16 kh and + 32), its row's LUT planes, and per 16-row tile the lane's
// patch of the slab's list.
struct WSlab {
  u32x4_t c[kPairs][2];
  u32x4_t lo[kPairs], hi[kPairs];
  uint32_t pe[kTilesW];
  uint32_t pn;  // list lengths of the slab, 8 bits per tile (clamped to 255)
};

template <int LM, bool CSR>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_kernel(const PrefillArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  int bid = blockIdx.x;
  if (bid < a.h_blocks) {
    prefill_dora_block(a, bid, reinterpret_cast<float*>(smem));
    return;
  }
  bid -= a.h_blocks;
  // XCD-aware order: the blocks of one XCD (bid % kXcds) take a contiguous range of the
  // logical order, which walks groups of kGroupN W blocks x all activation blocks.
  const int logical = (bid % kXcds) * a.per_xcd + bid / kXcds;
  if (logical >= a.blocks) return;
  const int tile = logical / a.splits;
  const int split = logical - tile * a.splits;
  const int group = tile / (kGroupN * a.mblk);
  const int within = tile - group * (kGroupN * a.mblk);
  const int gn = min(kGroupN, a.nblk - group * kGroupN);
  const int nb = group * kGroupN + within % gn;
  const int mb = within / gn;
  const int row0 = mb * MB;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n32 = lane & 31;
  const int kh = lane >> 5;
  const int r = lane & 15;
  const int hsel = n32 >> 4;  // the lane's 16-row tile within its pair
  const int s0 = a.sps * split;
  const int nsl = min(a.S, s0 + a.sps) - s0;  // 1..kMaxSlabs, block-uniform

  unsigned char* xbuf = smem + kLdsX;
  uint16_t* scratch = reinterpret_cast<uint16_t*>(smem + kLdsScratch) + wave * kScratchHalves;

  __shared__ int s_err;
  if (threadIdx.x == 0) s_err = 0;

  float16v_t acc[kPairs][kMG];  // D[i = 32 mg + 8 (v / 4) + 4 kh + v % 4][W row 64 w + 32 p + n32]
#pragma unroll
  for (int p = 0; p < kPairs; ++p)
#pragma unroll
    for (int g = 0; g < kMG; ++g)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[p][g][v] = 0.f;

  // ---- activations: thread t loads units t + kThreads k (row t / 16 + (kThreads / 16) k, unit t % 16)
  // of a slab
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.X, (uint32_t)((size_t)a.M * a.K * 2));
  const int xu = threadIdx.x & 15;
  const int xrow = threadIdx.x >> 4;
  u32x4_t xv[kXU];
  auto load_x = [&](int j) __attribute__((always_inline)) {
    const int col = 128 * (s0 + j) + 8 * xu;
#pragma unroll
    for (int k = 0; k < kXU; ++k) {
      const int i = xrow + (kThreads / 16) * k;
      const uint32_t off = (row0 + i < a.M && col < a.K) ? (uint32_t)(((size_t)(row0 + i) * a.K + col) * 2) : kOutOfRange;
      xv[k] = __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0);
    }
  };
  auto store_x = [&](int j) __attribute__((always_inline)) {
    unsigned char* buf = xbuf + (j & 1) * kSlabBytes;
#pragma unroll
    for (int k = 0; k < kXU; ++k) {
      const int i = xrow + (kThreads / 16) * k;
      *reinterpret_cast<u32x4_t*>(buf + i * 256 + ((xu ^ (i & 15)) << 4)) = xv[k];
    }
  };

  // ---- W: the lane's source tile per pair, code / plane pointers
  const u32x4_t* qb[kPairs];
  const u32x4_t* lb[kPairs];
#pragma unroll
  for (int p = 0; p < kPairs; ++p) {
    const int t = min(nb * kTiles + wave * kTilesW + 2 * p + hsel, a.T - 1);
    qb[p] = a.codes + (size_t)t * a.S * 64 + r + 16 * kh;
    lb[p] = a.planes + (size_t)t * a.ng * 32 + r;
  }
  // patch-list starts of the wave's tiles for slabs s0 .. s0 + nsl: tile ti's start of slab
  // s0 + j is lane j % 64 of pw[ti][j / 64]
  uint32_t pw[kTilesW][3];
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(a.wpatch, a.patch_bytes);
  if constexpr (CSR) {
#pragma unroll
    for (int ti = 0; ti < kTilesW; ++ti) {
      const size_t base = (size_t)min(nb * kTiles + wave * kTilesW + ti, a.T - 1) * a.S + s0;  // + j <= T * S
#pragma unroll
      for (int c = 0; c < 3; ++c) pw[ti][c] = a.wpidx[base + min(64 * c + lane, nsl)];
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int ti = 0; ti < kTilesW; ++ti)
#pragma unroll
      for (int c = 0; c < 3; ++c) asm volatile("v_mov_b32 %0, %1" : "=v"(pw[ti][c]) : "v"(pw[ti][c]));
  }
  auto list_at = [&](int ti, int j) __attribute__((always_inline)) {  // wave-uniform start of slab s0 + j
    const uint32_t v = j < 64 ? pw[ti][0] : j < 128 ? pw[ti][1] : pw[ti][2];
    return (uint32_t)__builtin_amdgcn_readlane((int)v, j & 63);
  };
  auto ld = [](const u32x4_t* p) __attribute__((always_inline)) { return __builtin_nontemporal_load(p); };
  auto load_w = [&](WSlab& w, int j) __attribute__((always_inline)) {
    const int s = s0 + j;
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      w.c[p][0] = ld(qb[p] + (size_t)s * 64);
      w.c[p][1] = ld(qb[p] + (size_t)s * 64 + 32);
      if constexpr (LM == 2) {
        const int g = s >> a.gshift;
        w.lo[p] = ld(lb[p] + g * 32);
        w.hi[p] = ld(lb[p] + g * 32 + 16);
      }
    }
    if constexpr (CSR) {
      uint32_t pn = 0u;
#pragma unroll
      for (int ti = 0; ti < kTilesW; ++ti) {
        const uint32_t st = list_at(ti, j);
        const uint32_t n = list_at(ti, j + 1) - st;
        const uint32_t off = (uint32_t)lane < n ? (st + (uint32_t)lane) * 4u : kOutOfRange;
        w.pe[ti] = __builtin_amdgcn_raw_buffer_load_b32(pr, (int)off, 0, 0);
        pn |= min(n, 255u) << (8 * ti);
      }
      w.pn = pn;
    }
  };
  LutPlanes<4> pl0[kPairs];
  if constexpr (LM == 0) {
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      const u32x4_t lo = lb[p][0];
      const u32x4_t hi = lb[p][16];
      pl0[p].lo[0] = lo.x; pl0[p].lo[1] = lo.y; pl0[p].lo[2] = lo.z; pl0[p].lo[3] = lo.w;
      pl0[p].hi[0] = hi.x; pl0[p].hi[1] = hi.y; pl0[p].hi[2] = hi.z; pl0[p].hi[3] = hi.w;
    }
  }

  // ---- half-slabs.  A slab's K16 steps 4 jj + q split into halves jj = 0, 1 (source lanes
  // with kq = kh + 2 jj).  The B operands of a half are prepared (dequantized; with outliers
  // written to the wave's scratch region jj and patched there) while the MFMAs of the previous
  // half run: prep(j, 1) beside mfma(j, 0), prep(j + 1, 0) beside mfma(j, 1).
  // Scratch region jj: [pair][tile][word q][source lane - 32 jj][8] fp16.
  auto scr_unit = [&](int jj, int p, int ht, int q, int l32) __attribute__((always_inline)) {
    return scratch + (jj * (kPairs * 2 * 4 * 32) + ((p * 2 + ht) * 4 + q) * 32 + l32) * 8;
  };
  u32x4_t breg[2][kPairs][4];  // B operands of halves 0 / 1 (no outliers: registers only)
  auto planes_of = [&](const WSlab& w, int p) __attribute__((always_inline)) {
    LutPlanes<4> t4;
    if constexpr (LM == 0) {
      t4 = pl0[p];
    } else {
      t4.lo[0] = w.lo[p].x; t4.lo[1] = w.lo[p].y; t4.lo[2] = w.lo[p].z; t4.lo[3] = w.lo[p].w;
      t4.hi[0] = w.hi[p].x; t4.hi[1] = w.hi[p].y; t4.hi[2] = w.hi[p].z; t4.hi[3] = w.hi[p].w;
    }
    return t4;
  };
  auto word_of = [](const u32x4_t& c, int q) __attribute__((always_inline)) {
    return q == 0 ? c.x : q == 1 ? c.y : q == 2 ? c.z : c.w;
  };
  // one K16 step q of half jjp's preparation (both pairs)
  auto prep_step = [&](const WSlab& w, int jjp, int q) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      uint32_t bv[4];
      dequant_word4s(word_of(w.c[p][jjp], q), planes_of(w, p), bv);
      const u32x4_t b = u32x4_t{bv[0], bv[1], bv[2], bv[3]};
      if constexpr (CSR) {
        *reinterpret_cast<u32x4_t*>(scr_unit(jjp, p, hsel, q, r + 16 * kh)) = b;
      } else {
        breg[jjp][p][q] = b;
      }
    }
  };
  // patches of half jjp of slab j (after its words are in the scratch): every lane stores one
  // 2-byte value per tile, a lane without a patch of this half to its own spare slot
  auto prep_patches = [&](const WSlab& w, int jjp, int j, auto long_lists) __attribute__((always_inline)) {
    if constexpr (CSR) {
      uint16_t* spare = scratch + 2 * (kPairs * 2 * 4 * 32) * 8 + lane;
#pragma unroll
      for (int ti = 0; ti < kTilesW; ++ti) {
        const uint32_t n = (w.pn >> (8 * ti)) & 255u;
        const uint32_t pv = w.pe[ti];
        const uint32_t e = (pv >> 6) & 31u;
        const bool mine = (uint32_t)lane < n && (int)((pv >> 5) & 1u) == jjp;
        uint16_t* dst = mine ? scr_unit(jjp, ti >> 1, ti & 1, (int)(e >> 3), (int)(pv & 31u)) + (e & 7u) : spare;
        *dst = (uint16_t)((pv >> 24) << 8);
      }
      if (long_lists) {  // rare: more than 64 outliers in 16 x 128 weights; the rest from global memory
        const uint32_t np = a.patch_bytes >> 2;
#pragma unroll
        for (int ti = 0; ti < kTilesW; ++ti) {
          const uint32_t st = list_at(ti, j);
          const uint32_t n = list_at(ti, j + 1) - st;
          for (uint32_t k = 64u + (uint32_t)lane; k < n; k += 64u) {
            if (st + k >= np) break;
            const uint32_t pv = a.wpatch[st + k];
            if ((int)((pv >> 5) & 1u) == jjp) {
              const uint32_t e = (pv >> 6) & 31u;
              scr_unit(jjp, ti >> 1, ti & 1, (int)(e >> 3), (int)(pv & 31u))[e & 7u] = (uint16_t)((pv >> 24) << 8);
            }
          }
        }
      }
    }
  };
  // A fragments of K16 step k = 4 jj + q of activation slab buffer xb (unit 8 jj + 4 kh + q of
  // rows 32 g + n32); the MFMAs of a step use the fragments read one step earlier.
  auto read_a = [&](const unsigned char* xb, int k, u32x4_t* av) __attribute__((always_inline)) {
    const int u = 8 * (k >> 2) + 4 * kh + (k & 3);
#pragma unroll
    for (int g = 0; g < kMG; ++g) {
      const int i = 32 * g + n32;
      av[g] = *reinterpret_cast<const u32x4_t*>(xb + i * 256 + ((u ^ (i & 15)) << 4));
    }
  };
  auto mfma_step = [&](int k, const u32x4_t* av) __attribute__((always_inline)) {
    const int jjm = k >> 2;
    const int q = k & 3;
    u32x4_t bb[kPairs];
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      if constexpr (CSR) {
        bb[p] = *reinterpret_cast<const u32x4_t*>(scr_unit(jjm, p, hsel, q, r + 16 * kh));
      } else {
        bb[p] = breg[jjm][p][q];
      }
    }
#pragma unroll
    for (int g = 0; g < kMG; ++g)
#pragma unroll
      for (int p = 0; p < kPairs; ++p) acc[p][g] = mfma32x32x16(av[g], bb[p], acc[p][g]);
  };
  // Issue order of one K16 step: the MFMAs spread over the step's dequantization (VALU) and
  // the next step's fragment reads, so the reads' latency and the lookups hide behind MFMAs.
  auto step_order = []() __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < kMG * kPairs; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      if (m < kMG) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // VALU
    }
  };

  // ---- the slab loop.  long_lists: some patch list of the wave's tiles in this split is longer
  // than the 64 entries the lanes hold (a rare instance with the global-memory walk; the common
  // one has no branch in its loop body).  Both run the same barriers.
  auto slab_loop = [&](auto long_lists) __attribute__((always_inline)) {
    // prologue: slab 0 in LDS, slab 1 in registers, kPF W slabs in flight, half (0, 0) prepared
    load_x(0);
    WSlab wbuf[kPF];
  #pragma unroll
    for (int u = 0; u < kPF; ++u) load_w(wbuf[u], min(u, nsl - 1));
    store_x(0);
    if (nsl > 1) load_x(1);
  #pragma unroll
    for (int q = 0; q < 4; ++q) prep_step(wbuf[0], 0, q);
    prep_patches(wbuf[0], 0, 0, long_lists);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    raw_barrier();

    // slab j: W(j) in wc, W(j + 1) in wn (next: whether slab j + 1 exists).  Once half 1 of
    // slab j is prepared, wc is free: W(j + kPF) is loaded into it (reload: whether to), a full
    // slab before prep(j + 1, 0) needs it.
    // The flags are std::true_type in the steady state (no branches: the wait counts stay exact
    // through the loop body) and bool in the last rounds.
    auto consume = [&](WSlab& wc, const WSlab& wn, int j, auto next, auto reload, auto x1, auto x2)
                       __attribute__((always_inline)) {
      // the next slab's activations to the other buffer (read by every wave before the last
      // barrier), the one after into registers
      if (x1) store_x(j + 1);
      if (x2) load_x(j + 2);
      const unsigned char* xb = xbuf + (j & 1) * kSlabBytes;
      u32x4_t av[2][kMG];
      read_a(xb, 0, av[0]);
  #pragma unroll
      for (int q = 0; q < 4; ++q) {
        read_a(xb, q + 1, av[(q + 1) & 1]);
        prep_step(wc, 1, q);
        mfma_step(q, av[q & 1]);
        step_order();
      }
      prep_patches(wc, 1, j, long_lists);
      __builtin_amdgcn_sched_barrier(0);
      if (reload) load_w(wc, j + kPF);
      __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (q < 3) read_a(xb, 5 + q, av[(q + 1) & 1]);
        if (next) prep_step(wn, 0, q);
        mfma_step(4 + q, av[q & 1]);
        step_order();
      }
      if (next) prep_patches(wn, 0, j + 1, long_lists);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      raw_barrier();
    };

    const std::true_type yes{};
    int j0 = 0;
    for (; j0 + 2 * kPF <= nsl; j0 += kPF) {
  #pragma unroll
      for (int u = 0; u < kPF; ++u) {
        consume(wbuf[u], wbuf[(u + 1) % kPF], j0 + u, yes, yes, yes, yes);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (j0 < nsl) {
  #pragma unroll
      for (int u = 0; u < kPF; ++u) {
        const int j = j0 + u;
        if (j < nsl) consume(wbuf[u], wbuf[(u + 1) % kPF], j, j + 1 < nsl, j + kPF < nsl, j + 1 < nsl, j + 2 < nsl);
      }
      j0 += kPF;
  #pragma unroll
      for (int u = 0; u < kPF; ++u) {
        const int j = j0 + u;
        if (j < nsl) consume(wbuf[u], wbuf[(u + 1) % kPF], j, j + 1 < nsl, false, j + 1 < nsl, j + 2 < nsl);
      }
    }
  };
  bool long_lists = false;
  if constexpr (CSR) {  // any list of the wave's tiles over slabs s0 .. s0 + nsl longer than 64
#pragma unroll
    for (int ti = 0; ti < kTilesW; ++ti)
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        const uint32_t cur = pw[ti][c];
        uint32_t nxt = (uint32_t)__shfl_down((int)cur, 1);
        if (lane == 63) nxt = c < 2 ? (uint32_t)__builtin_amdgcn_readfirstlane((int)pw[ti][c + 1]) : cur;
        if (64 * c + lane < nsl && nxt - cur > 64u) long_lists = true;
      }
    long_lists = __builtin_amdgcn_ballot_w64(long_lists) != 0;
  }
  if (long_lists) {
    slab_loop(true);
  } else {
    slab_loop(std::false_type{});
  }

  // ---------------------------------------------------------------- completion
  // The completion reloads its arguments from the kernel-argument segment (the opaque copy of
  // the pointer keeps the compiler from holding them in SGPRs across the slab loop).
  const PrefillArgs* kp = (const PrefillArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(kp));
  const PrefillArgs& e = *kp;
  __syncthreads();
  uint32_t* slot = e.sync + kSyncSlot0 + kSlotWords * mb;
  const bool h_fused = e.r > 0 && e.h_blocks > 0;
  uint32_t err = 0u;
  if (e.splits > 1) {
    const __amdgpu_buffer_rsrc_t prs = make_rsrc(e.partial, e.partial_bytes);
    auto poff = [&](int sp, int p, int g, int v4) __attribute__((always_inline)) {
      return (int)((((((((size_t)sp * e.tiles + tile) * kCW + wave) * kPairs + p) * kMG + g) * 64 + lane) * 4 + v4) *
                   16);
    };
#pragma unroll
    for (int p = 0; p < kPairs; ++p)
#pragma unroll
      for (int g = 0; g < kMG; ++g)
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          const u32x4_t v = u32x4_t{__float_as_uint(acc[p][g][4 * v4]), __float_as_uint(acc[p][g][4 * v4 + 1]),
                                    __float_as_uint(acc[p][g][4 * v4 + 2]), __float_as_uint(acc[p][g][4 * v4 + 3])};
          __builtin_amdgcn_raw_buffer_store_b128(v, prs, poff(split, p, g, v4), 0, kSc1);
        }
    stores_done();
    __syncthreads();
    __shared__ int s_last;
    uint32_t* cnt = e.sync + kSyncTile + e.mblk + tile;
    if (threadIdx.x == 0) {
      const uint32_t old = atomicAdd(cnt, 1u);
      if (old >= (uint32_t)e.splits) {
        raise_error(e.sync, kErrArrivals);
        s_err = 1;
      }
      s_last = old == (uint32_t)(e.splits - 1) || old >= (uint32_t)e.splits;
    }
    __syncthreads();
    if (!s_last) return;
    compiler_fence();
    if (threadIdx.x == 0) {
      err = load_dev(e.sync + kSyncErrorWord);
      store_dev(cnt, 0u);
    }
    // the splits' partials summed in split order, 4 splits' loads in flight per (pair, group)
#pragma unroll
    for (int p = 0; p < kPairs; ++p)
#pragma unroll
      for (int g = 0; g < kMG; ++g) {
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[p][g][v] = 0.f;
        for (int sp0 = 0; sp0 < e.splits; sp0 += 4) {
          u32x4_t t[4][4];
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int v4 = 0; v4 < 4; ++v4)
              t[u][v4] = __builtin_amdgcn_raw_buffer_load_b128(prs, poff(min(sp0 + u, e.splits - 1), p, g, v4), 0, kSc1);
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (sp0 + u < e.splits)
#pragma unroll
              for (int v4 = 0; v4 < 4; ++v4)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[p][g][4 * v4 + e] += __uint_as_float(t[u][v4][e]);
        }
      }
  }

  // DoRA: s * H.B^T as MFMAs onto the accumulator layout (H as fp16 high / low parts of
  // 2^-sh H, B rows and gamma of the block's W rows staged in LDS).
  uint16_t* h_hi = reinterpret_cast<uint16_t*>(smem + kEpiHi);
  uint16_t* h_lo = reinterpret_cast<uint16_t*>(smem + kEpiLo);
  uint16_t* b_s = reinterpret_cast<uint16_t*>(smem + kEpiB);
  uint16_t* g_s = reinterpret_cast<uint16_t*>(smem + kEpiG);
  uint16_t* o_s = reinterpret_cast<uint16_t*>(smem + kEpiOut);
  __shared__ uint32_t s_hmax;
  uint32_t cons_old = 0u;
  bool counted = false;
  const int rows = min(MB, e.M - row0);
  const int n0 = nb * kBlockRows;
  if (e.r > 0) {
    const int rp = (e.r + 15) & ~15;  // rank padded to the MFMA depth
    if (h_fused && lane == 0) {
      uint32_t ready = load_dev(slot);
      for (uint32_t spins = 0; ready == 0u && spins < e.spin_limit; ++spins) {
        __builtin_amdgcn_s_sleep(2);
        ready = load_dev(slot);
      }
      if (ready == 0u) {
        s_err = 1;
        raise_error(e.sync, kErrHTimeout);
      }
    }
    compiler_fence();
    if (h_fused && threadIdx.x == 0 && e.splits == 1) err = load_dev(e.sync + kSyncErrorWord);
    if (threadIdx.x == 0) s_hmax = 0u;
    const float* hsrc = (h_fused ? e.hfin : e.H) + (size_t)row0 * e.r;
    __syncthreads();  // every poll of the block is done: H is final
    // All the stage's loads at once: B rows (zero beyond rank r), gamma, and H through the caches
    // (no line of H was read on this CU before its slot was raised in this launch).
    constexpr int kBU = kBlockRows * (kMaxRank / 8) / kThreads;
    constexpr int kHV = MB * kMaxRank / kThreads;
    const int bunits = kBlockRows * (rp / 8);
    u32x4_t bv[kBU];
#pragma unroll
    for (int t = 0; t < kBU; ++t) {
      const int u = (int)threadIdx.x + kThreads * t;
      const int row = u / (rp / 8);
      const int c8 = 8 * (u - row * (rp / 8));
      bv[t] = u32x4_t{0u, 0u, 0u, 0u};
      if (u < bunits && c8 < e.r) bv[t] = *reinterpret_cast<const u32x4_t*>(e.B + (size_t)min(n0 + row, e.N - 1) * e.r + c8);
    }
    const uint16_t gv = threadIdx.x < kBlockRows ? e.gamma[min(n0 + (int)threadIdx.x, e.N - 1)] : (uint16_t)0;
    float hv[kHV];
    uint32_t hmax = 0u;
#pragma unroll
    for (int t = 0; t < kHV; ++t) {
      const int idx = (int)threadIdx.x + kThreads * t;
      const int i = idx / rp;
      const int j = idx - i * rp;
      hv[t] = (idx < MB * rp && i < rows && j < e.r) ? hsrc[i * e.r + j] : 0.f;
      hmax = max(hmax, __float_as_uint(hv[t]) & 0x7FFFFFFFu);  // (NaN bit patterns order above inf)
    }
    if (hmax != 0u) atomicMax(&s_hmax, hmax);
#pragma unroll
    for (int t = 0; t < kBU; ++t) {
      const int u = (int)threadIdx.x + kThreads * t;
      const int row = u / (rp / 8);
      if (u < bunits) *reinterpret_cast<u32x4_t*>(b_s + row * kEpiStride + 8 * (u - row * (rp / 8))) = bv[t];
    }
    if (threadIdx.x < kBlockRows) g_s[threadIdx.x] = gv;
    __syncthreads();
    const int hex = (int)((s_hmax >> 23) & 0xFFu) - 127;
    const int sh = max(0, hex - 14);
#pragma unroll
    for (int t = 0; t < kHV; ++t) {
      const int idx = (int)threadIdx.x + kThreads * t;
      if (idx < MB * rp) {
        const int i = idx / rp;
        const int j = idx - i * rp;
        const float v = ldexpf(hv[t], -sh);
        const uint16_t hi = f2h_rn(v);
        h_hi[i * kEpiStride + j] = hi;
        h_lo[i * kEpiStride + j] = f2h_rn(v - h2f(hi));
      }
    }
    __syncthreads();
    const float sc = ldexpf(e.scale, sh);
#pragma unroll
    for (int p = 0; p < kPairs; ++p) {
      const int col = 32 * kPairs * wave + 32 * p + n32;
      const float gam = h2f(g_s[col]);
#pragma unroll
      for (int g = 0; g < kMG; ++g) {
        float16v_t dd;
#pragma unroll
        for (int v = 0; v < 16; ++v) dd[v] = 0.f;
        for (int kk = 0; kk < rp; kk += 16) {
          const u32x4_t bb = *reinterpret_cast<const u32x4_t*>(b_s + col * kEpiStride + kk + 8 * kh);
          const int ro = (32 * g + n32) * kEpiStride + kk + 8 * kh;
          dd = mfma32x32x16(*reinterpret_cast<const u32x4_t*>(h_hi + ro), bb, dd);
          dd = mfma32x32x16(*reinterpret_cast<const u32x4_t*>(h_lo + ro), bb, dd);
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[p][g][v] = (acc[p][g][v] + sc * dd[v]) * gam;
      }
    }
  }
  if (err != 0u) s_err = 1;
  __syncthreads();
  if (h_fused && threadIdx.x == 0) {
    cons_old = atomicAdd(slot + 1, 1u);
    counted = true;
  }
  const bool poisoned = s_err != 0;
#pragma unroll
  for (int p = 0; p < kPairs; ++p)
#pragma unroll
    for (int g = 0; g < kMG; ++g)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        o_s[(32 * g + 8 * (v >> 2) + 4 * kh + (v & 3)) * kOutStride + 32 * kPairs * wave + 32 * p + n32] =
            poisoned ? kHalfNaN : f2h_rn(acc[p][g][v]);
  __syncthreads();
  constexpr int kUnits = kBlockRows / 8;
  for (int idx = threadIdx.x; idx < rows * kUnits; idx += kThreads) {
    const int i = idx / kUnits;
    const int c8 = 8 * (idx - i * kUnits);
    const int n = n0 + c8;
    const uint16_t* src = o_s + i * kOutStride + c8;
    uint16_t* dst = e.out + (size_t)(row0 + i) * e.N + n;
    if (e.out_vec && n + 8 <= e.N) {
      *reinterpret_cast<u32x4_t*>(dst) = *reinterpret_cast<const u32x4_t*>(src);
    } else {
      for (int c = 0; c < 8; ++c)
        if (n + c < e.N) dst[c] = src[c];
    }
  }
  if (counted) {  // the slot's last consumer (one per W block) lowers it for the next call
    if (cons_old >= (uint32_t)e.nblk) raise_error(e.sync, kErrArrivals);
    if (cons_old == (uint32_t)(e.nblk - 1)) {
      store_dev(slot + 1, 0u);
      store_dev(slot, 0u);
    }
  }
}

template <int LM, bool CSR>
hipError_t launch_prefill_tpl(const PrefillArgs& a, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((prefill_kernel<LM, CSR>), grid, dim3(kThreads), kLdsBytes, stream, a);
  return hipGetLastError();
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

int prefill_min_m() { return 129; }

PrefillPlan plan_prefill(int N, int K, int M, int group_size, int cu_count, int rank, int fused_rank, int chunk) {
  PrefillPlan p{};
  const int S = (K + 127) / 128;
  const int cus = std::max(1, cu_count);
  p.nblk = (N + kBlockRows - 1) / kBlockRows;
  p.mblk = (M + MB - 1) / MB;
  p.tiles = p.nblk * p.mblk;
  // per-row LUTs or LUT groups of 128 << g columns (a slab's group is uniform)
  bool slab_groups = group_size <= 0 || group_size >= K;
  for (int g = 0; g < 6 && !slab_groups; ++g) slab_groups = group_size == (128 << g);
  p.ok = M >= prefill_min_m() && M <= kMaxSlots * MB && slab_groups && (chunk == 512 || chunk == 640) &&
         rank % 8 == 0 && rank <= kMaxRank && fused_rank % 8 == 0 && fused_rank <= kMaxRank &&
         (size_t)M * K * 2 < ((size_t)1 << 31);
  if (!p.ok) return p;
  // K splits only where a split would exceed kMaxSlabs (the partial round trip costs more than
  // the idle CUs of narrow layers; those take the MFMA GEMM)
  int splits = (S + kMaxSlabs - 1) / kMaxSlabs;
  const int sps = (S + splits - 1) / splits;
  splits = (S + sps - 1) / sps;
  p.splits = splits;
  p.sps = sps;
  // DoRA shares per activation block: ~8 slabs each, at most 8, at most 128 DoRA blocks
  p.hk = fused_rank > 0 ? std::max(1, std::min({8, (S + 7) / 8, std::max(1, 128 / p.mblk)})) : 0;
  p.h_blocks = p.mblk * p.hk;
  const int blocks = p.tiles * splits;
  p.per_xcd = (blocks + kXcds - 1) / kXcds;
  p.grid = p.h_blocks + kXcds * p.per_xcd;
  const size_t hf = fused_rank > 0 ? align256((size_t)M * fused_rank * 4) : 0;
  const size_t hp = fused_rank > 0 ? align256((size_t)p.h_blocks * MB * fused_rank * 4) : 0;
  const size_t part = splits > 1 ? (size_t)splits * p.tiles * kCW * kPairs * kMG * 64 * 64 : 0;
  p.hfin_off = 0;
  p.hpart_off = hf;
  p.partial_off = hf + hp;
  p.workspace_bytes = hf + hp + part;
  p.lds = kLdsBytes;
  // Measured on MI355X (Qwen2.5-7B shapes, 4-bit, DoRA r = 16, 0.5% outliers): faster than the MFMA
  // GEMM (256-row tiles) only where M leaves the GEMM's last row tile at most half full, on layers
  // whose output tiles fill at least half the CUs without K splits (gate 18944 x 3584 at M = 384:
  // 90 us against 144; at M = 256 / 512 / 768 / 1024 the GEMM's 77 / 146 / 151 / 220 us beat 83 /
  // 162 / 168 / 246; slower on down 3584 x 18944 and on narrow layers).
  p.preferred = p.tiles >= cus / 2 && S <= 32 && M <= 1024 && (M - 1) % 256 < 128;
  p.ok = sps <= kMaxSlabs && part < ((size_t)1 << 31) &&
         (splits == 1 || kSyncTile + p.mblk + p.tiles <= kSyncErrorWord) && kSyncTile + p.mblk <= kSyncErrorWord;
  return p;
}

hipError_t launch_prefill(const Layer& L, const void* prepared, int64_t nnz, const Dora& D, const uint16_t* x,
                          uint16_t* out, int M, const PrefillPlan& plan, float* workspace, uint32_t* sync,
                          hipStream_t stream) {
  const PreparedLayout lay = prepared_layout(L.N, L.K, L.group_size, nnz);
  const char* base = reinterpret_cast<const char*>(prepared);
  PrefillArgs a{};
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
  a.nblk = plan.nblk;
  a.mblk = plan.mblk;
  a.tiles = plan.tiles;
  a.splits = plan.splits;
  a.sps = plan.sps;
  a.blocks = plan.tiles * plan.splits;
  a.per_xcd = plan.per_xcd;
  const bool fused_h = D.r > 0 && D.H == nullptr;
  a.hk = fused_h ? plan.hk : 0;
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
  a.gshift = gshift;
  const dim3 grid(a.h_blocks + kXcds * plan.per_xcd);
  if (per_row) return csr ? launch_prefill_tpl<0, true>(a, grid, stream) : launch_prefill_tpl<0, false>(a, grid, stream);
  return csr ? launch_prefill_tpl<2, true>(a, grid, stream) : launch_prefill_tpl<2, false>(a, grid, stream);
}

}  // namespace wlq
