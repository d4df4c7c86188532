// Prefill-shaped WLQ product (M > 32): dequantization into LDS feeding MFMA.
//
// Reference behaviour replaced: the M >= 16 path of gemm_forward
// (csrc/vllm_binding.cpp:355-393: full-matrix dequant into a workspace, cuBLAS
// HGEMM, separate DoRA pass) and gemm_metalog_dora_kernel's overwrite semantics
// (csrc/gemm_kernel.cu:204-228).  W is never materialized in HBM.
//
// Block tile 256 (M) x 128 (N), K step 64, 512 threads = 8 waves in a 4x2
// arrangement, each wave a 64x64 sub-tile of V_MFMA_F32_16X16X32_F16.  The W
// tile is dequantized once per block and shared by the 256 activation rows.
//
// Pipeline per K step: the global loads of step k+2 (activations, code
// windows, group LUTs) are issued into registers, the MFMAs of step k read LDS
// buffer k%2, then step k+1's registers are written to the other LDS buffer:
// activations permuted to column order P, codes expanded through their LUT byte
// planes (4 threads per W row, 16 columns each), outliers overwritten (the
// reference's W0 = e5m2 << 8 at outlier positions).  One barrier per step.
// Outlier entries of the block's 128 rows are staged per 512-column chunk
// (640 for 3-bit) into LDS, one chunk ahead, in phases spread over the chunk's
// first steps (offsets, counts, prefix, entries), so no dependent global load
// sits in the loop.
//
// DoRA: with one split, the low-rank term s * H . B^T is added in the
// epilogue with V_MFMA_F32_16X16X4_F32 (fp32 operands, exact products) and
// the block writes fp16((acc + s H B^T) * gamma); with split-K the partials go
// to an fp32 workspace and splitk_reduce_kernel applies the epilogue.
//
// Blocks are mapped so that each XCD works through a contiguous range of
// tiles, N-tile major: consecutive blocks of one XCD share W tiles in its L2.
#include <algorithm>
#include <utility>

#include "wlq_device.h"
#include "wlq_internal.h"

namespace wlq {
namespace {

constexpr int BM = 256;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int NT = 512;
constexpr int LDS_ROW = BK + 8;  // halves per LDS row (16-byte pad)
constexpr int kEntCap = 2048;    // outlier entries of one (N tile, chunk) held in LDS
constexpr int kPosWords = 132;   // row prefix (BN + 1 used), padded to 16 bytes
constexpr int kSlotWords = kPosWords + kEntCap;  // one (N tile, chunk) slot of the prepared entries
constexpr int kMaxSplits = 32;
constexpr int kXcds = 8;

struct GemmArgs {
  const uint32_t* q;
  const uint16_t* lut;
  const uint16_t* X;
  uint16_t* out;
  float* partial;
  const int32_t* offsets;
  const uint16_t* cols;
  const uint8_t* vals;
  const uint16_t* B;
  const float* H;
  const uint16_t* gamma;
  float scale;
  int r;
  int M, N, K, wpr, G, ng, nch, chunk;
  uint32_t g_magic;
  int ksteps_per_split, splits;
  int tiles_m, tiles_n, tiles;
  int has_csr;
  const uint32_t* tent;  // prepared entries [tiles_n * nch] slots, or nullptr (direct CSR reads)
};

struct GemmSmem {
  uint16_t a[2][BM * LDS_ROW];
  uint16_t b[2][BN * LDS_ROW];
  uint32_t ent[2][kEntCap];   // col | val << 16, the tile's rows in order
  int pos[2][kPosWords];      // row start inside ent (exclusive prefix), pos[BN] = total
};

__device__ __forceinline__ int group_of(int col, uint32_t magic) { return (int)__umulhi((uint32_t)col, magic); }

// 16-column code piece starting at column c16 (c16 % 16 == 0) of a packed row:
// the words that hold it (clamped inside the row; columns past K meet zero
// activations) and its two 8-column blocks expanded to fp16 pairs in order P.
template <int BITS>
__device__ __forceinline__ void load_piece16(const uint32_t* __restrict__ qrow, int c16, int wpr, uint32_t w[3]) {
  if constexpr (BITS == 4) {
    const u32x2_t v = *reinterpret_cast<const u32x2_t*>(qrow + min(c16 >> 3, wpr - 2));
    w[0] = v.x; w[1] = v.y; w[2] = 0u;
  } else if constexpr (BITS == 2) {
    w[0] = qrow[min(c16 >> 4, wpr - 1)]; w[1] = 0u; w[2] = 0u;
  } else if constexpr (BITS == 1) {
    w[0] = qrow[min(c16 >> 5, wpr - 1)]; w[1] = 0u; w[2] = 0u;
  } else {
    const int wi = c16 / 10;
#pragma unroll
    for (int j = 0; j < 3; ++j) w[j] = qrow[min(wi + j, wpr - 1)];
  }
}

template <int BITS, int BLK>
__device__ __forceinline__ void dequant_piece16(const uint32_t w[3], int c16, const LutPlanes<BITS>& t,
                                                uint32_t out[4]) {
  if constexpr (BITS == 4) {
    dequant_word4(w[BLK], t, out);
  } else {
    uint32_t code[8];
    if constexpr (BITS == 2) {
#pragma unroll
      for (int j = 0; j < 8; ++j) code[j] = (w[0] >> (2 * (8 * BLK + j))) & 3u;
    } else if constexpr (BITS == 1) {
      const uint32_t v = w[0] >> ((c16 & 31) + 8 * BLK);
#pragma unroll
      for (int j = 0; j < 8; ++j) code[j] = (v >> j) & 1u;
    } else {  // 3-bit: slot s0 = c16 % 10 of word c16 / 10; codes up to slot s0 + 15 < 25
      const int s0 = c16 - (c16 / 10) * 10;
      // the 25 slots of three words as two 64-bit windows (values only: no indexed access)
      const uint64_t lo = (uint64_t)w[0] | ((uint64_t)w[1] << 30);   // slots 0..19 at 3 bits each
      const uint64_t hi = (uint64_t)w[1] | ((uint64_t)w[2] << 30);   // slots 10..29
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int idx = s0 + 8 * BLK + j;
        const uint64_t src = idx < 20 ? lo : hi;
        const int sh = 3 * (idx < 20 ? idx : idx - 10);
        code[j] = (uint32_t)(src >> sh) & 7u;
      }
    }
    const uint32_t se = code[0] | (code[2] << 8) | (code[4] << 16) | (code[6] << 24);
    const uint32_t so = code[1] | (code[3] << 8) | (code[5] << 16) | (code[7] << 24);
    dequant_sel8<BITS>(se, so, t, out);
  }
}

// ------------------------------------------------------------------ kernel

// Registers carrying one K step from global memory to LDS.
template <int BITS>
struct StepRegs {
  u32x4_t x[4];      // activation 16-byte units u = tid + NT * j
  uint32_t cw[3];    // words holding this thread's 16 code columns
  LutRaw<BITS> lr;   // LUT entries of the piece's group (group LUTs)
};

template <int BITS, bool PER_ROW, bool HAS_CSR, bool X_VEC>
__global__ __launch_bounds__(NT, 2) void gemm_kernel(const GemmArgs a) {
  constexpr int NCB = 1 << BITS;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  GemmSmem& sm = *reinterpret_cast<GemmSmem*>(smem_raw);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;  // 0..3: 64-row slice of the M tile
  const int wn = wave & 1;   // 0..1: 64-column slice of the N tile
  const int r = lane & 15;
  const int kq = lane >> 4;

  // tile of this block: XCD-contiguous ranges, N-tile major
  const int split = blockIdx.x / a.tiles;
  int t = blockIdx.x - split * a.tiles;
  if (a.tiles % kXcds == 0) {
    const int per = a.tiles / kXcds;
    t = (t % kXcds) * per + t / kXcds;
  }
  const int tn = t / a.tiles_m;
  const int m0 = (t - tn * a.tiles_m) * BM;
  const int n0 = tn * BN;

  const int ksteps_total = (a.K + BK - 1) / BK;
  const int kt_begin = split * a.ksteps_per_split;  // whole chunks (the planner aligns splits)
  const int kt_end = min(ksteps_total, kt_begin + a.ksteps_per_split);
  const int kt_last = max(kt_end - 1, kt_begin);

  // W producer role: row nl of the tile, 16 columns [16 qq, 16 qq + 16) of each step
  const int nl = tid >> 2;
  const int qq = tid & 3;
  const int nb = n0 + nl;
  const bool brow_ok = nb < a.N;
  const int nbc = brow_ok ? nb : (a.N - 1);
  const uint32_t* qrow = a.q + (size_t)nbc * a.wpr;
  const uint16_t* lrow = a.lut + (size_t)nbc * a.ng * NCB;

  LutPlanes<BITS> pl_row;
  if constexpr (PER_ROW) {
    LutRaw<BITS> raw;
    lut_load<BITS>(raw, lrow);
    pl_row = lut_planes<BITS>(raw);
  }

  auto load_step = [&](StepRegs<BITS>& S, int kt) __attribute__((always_inline)) {
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = tid + NT * j;
      const int row = u >> 3;
      const int col = k0 + 8 * (u & 7);
      if constexpr (X_VEC) {  // clamped, unconditional; out-of-range units are zeroed when stored
        const int m = min(m0 + row, a.M - 1);
        S.x[j] = *reinterpret_cast<const u32x4_t*>(a.X + (size_t)m * a.K + min(col, a.K - 8));
      } else {
        const int m = m0 + row;
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (m < a.M) {
          const uint16_t* src = a.X + (size_t)m * a.K + col;
          uint32_t e[8];
#pragma unroll
          for (int q2 = 0; q2 < 8; ++q2) e[q2] = (col + q2 < a.K) ? (uint32_t)src[q2] : 0u;
          v.x = e[0] | (e[1] << 16);
          v.y = e[2] | (e[3] << 16);
          v.z = e[4] | (e[5] << 16);
          v.w = e[6] | (e[7] << 16);
        }
        S.x[j] = v;
      }
    }
    const int c16 = k0 + 16 * qq;
    load_piece16<BITS>(qrow, c16, a.wpr, S.cw);
    if constexpr (!PER_ROW) {
      const int g = min(group_of(c16, a.g_magic), a.ng - 1);
      lut_load<BITS>(S.lr, lrow + g * NCB);
    }
  };

  // running position in the row's staged entries (entries are sorted by column)
  int p_run = 0;

  auto store_step = [&](const StepRegs<BITS>& S, int kt, int buf, auto prep) __attribute__((always_inline)) {
    constexpr bool kPrep = decltype(prep)::value;
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = tid + NT * j;
      const int row = u >> 3;
      const int c8 = u & 7;
      const bool ok = m0 + row < a.M && k0 + 8 * c8 < a.K;
      const u32x4_t v = ok ? permute_p(S.x[j]) : u32x4_t{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4_t*>(&sm.a[buf][row * LDS_ROW + 8 * c8]) = v;
    }
    LutPlanes<BITS> pl;
    if constexpr (PER_ROW) pl = pl_row;
    else pl = lut_planes<BITS>(S.lr);
    const int c16 = k0 + 16 * qq;
    uint16_t* brow = &sm.b[buf][nl * LDS_ROW + 16 * qq];
    {
      uint32_t o[4];
      dequant_piece16<BITS, 0>(S.cw, c16, pl, o);
      *reinterpret_cast<u32x4_t*>(brow) = u32x4_t{o[0], o[1], o[2], o[3]};
      dequant_piece16<BITS, 1>(S.cw, c16, pl, o);
      *reinterpret_cast<u32x4_t*>(brow + 8) = u32x4_t{o[0], o[1], o[2], o[3]};
    }
    if constexpr (HAS_CSR) {
      const int ck = k0 / a.chunk;
      const int cb = ck & 1;
      const int kin = k0 - ck * a.chunk;     // step start inside the chunk
      const int lo = kin + 16 * qq;          // my 16 columns inside the chunk
      if (brow_ok) {
        if constexpr (kPrep) {
          if (kin == 0) p_run = sm.pos[cb][nl];
          const int pend = sm.pos[cb][nl + 1];
          while (p_run < pend) {
            const uint32_t e = sm.ent[cb][p_run];
            const int col = (int)(e & 0xFFFFu);
            if (col >= lo + 16) break;
            if (col >= lo) {
              const int cs = col - lo;
              brow[8 * (cs >> 3) + p_slot(cs & 7)] = (uint16_t)((e >> 16) << 8);
            }
            ++p_run;
          }
        } else {  // no prepared list (or a chunk beyond its capacity): read the row's chunk directly
          const int32_t* offr = a.offsets + (size_t)nb * (a.nch + 1);
          const int s1 = offr[ck + 1];
          for (int e = offr[ck]; e < s1; ++e) {
            const int cs = (int)a.cols[e] - lo;
            if (cs >= 0 && cs < 16) brow[8 * (cs >> 3) + p_slot(cs & 7)] = (uint16_t)((uint32_t)a.vals[e] << 8);
          }
        }
      }
    }
  };

  // Prepared outlier entries of a chunk (slot of this N tile): loaded into registers
  // two iterations before the chunk's first step is staged, written to ent/pos[ck & 1]
  // at the end of the next iteration (after that iteration's readers of the other buffer).
  u32x4_t ent_r = {0u, 0u, 0u, 0u}, pos_r = {0u, 0u, 0u, 0u};
  auto ent_load = [&](int ck) __attribute__((always_inline)) {
    const uint32_t* slot = a.tent + ((size_t)tn * a.nch + ck) * kSlotWords;
    ent_r = *reinterpret_cast<const u32x4_t*>(slot + kPosWords + 4 * tid);
    pos_r = *reinterpret_cast<const u32x4_t*>(slot + 4 * min(tid, kPosWords / 4 - 1));
  };
  auto ent_store = [&](int ck) __attribute__((always_inline)) {
    const int cb = ck & 1;
    *reinterpret_cast<u32x4_t*>(&sm.ent[cb][4 * tid]) = ent_r;
    if (tid < kPosWords / 4) *reinterpret_cast<u32x4_t*>(&sm.pos[cb][4 * tid]) = pos_r;
  };

  float4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto mfma_step = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4_t af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const u32x4_t*>(&sm.a[buf][(64 * wm + 16 * i + r) * LDS_ROW + 32 * ks + 8 * kq]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = *reinterpret_cast<const u32x4_t*>(&sm.b[buf][(64 * wn + 16 * j + r) * LDS_ROW + 32 * ks + 8 * kq]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(af[i], bf[j], acc[i][j]);
    }
  };

  // Prepared outlier lists are used when every chunk of this block's range fits its
  // slot; otherwise the block reads the CSR arrays directly (a separate loop, so the
  // hot loop carries no data-dependent loads).
  __shared__ int s_direct;
  const int ck_begin = (kt_begin * BK) / a.chunk;
  const int ck_end = (max(kt_end, kt_begin + 1) * BK + a.chunk - 1) / a.chunk;
  bool prepared = false;
  if constexpr (HAS_CSR) {
    if (a.tent != nullptr) {
      if (tid == 0) s_direct = 0;
      __syncthreads();
      if (tid < ck_end - ck_begin &&
          (int)a.tent[((size_t)tn * a.nch + ck_begin + tid) * kSlotWords + BN] > kEntCap)
        s_direct = 1;
      __syncthreads();
      prepared = s_direct == 0;
    }
  }

  auto run = [&](auto prep) __attribute__((always_inline)) {
    constexpr bool kPrep = decltype(prep)::value;
    StepRegs<BITS> s0, s1;
    if constexpr (kPrep) ent_load(ck_begin);
    load_step(s0, kt_begin);
    load_step(s1, min(kt_begin + 1, kt_last));
    if constexpr (kPrep) {
      ent_store(ck_begin);
      __syncthreads();
      p_run = sm.pos[ck_begin & 1][nl];
    }
    store_step(s0, kt_begin, 0, prep);
    if constexpr (kPrep) ent_load((min(kt_begin + 2, kt_last) * BK) / a.chunk);
    // drain the prologue's loads once: the loop then starts from the same wait state as
    // its back edge, and the compiler does not add first-iteration waits to every trip
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt unconstrained (gfx9 encoding)
    __syncthreads();

    // One K step: loads of step kt+2 (clamped), MFMAs of step kt, LDS stores of step
    // kt+1, the entries of step kt+2's chunk stored when it starts a chunk, the entries
    // of step kt+3's chunk loaded (every step, so the wait counts never depend on data),
    // barrier.
    auto iter = [&](int kt, StepRegs<BITS>& sload, const StepRegs<BITS>& sstore) __attribute__((always_inline)) {
      const int buf = (kt - kt_begin) & 1;
      load_step(sload, min(kt + 2, kt_last));
      // keep the loads ahead of the MFMAs: the scheduler would otherwise sink them
      // past the matrix work (shrinking the prefetch distance to nothing)
      __builtin_amdgcn_sched_barrier(0);
      mfma_step(buf);
      // unconditional (the last trip stores a duplicate of the last step into the idle
      // buffer) so that every trip leaves the same loads pending
      store_step(sstore, min(kt + 1, kt_last), buf ^ 1, prep);
      if constexpr (kPrep) {
        const int k2 = (kt + 2) * BK;
        if (kt + 2 < kt_end && k2 % a.chunk == 0) ent_store(k2 / a.chunk);
        ent_load((min(kt + 3, kt_last) * BK) / a.chunk);
      }
      __syncthreads();
    };
    int kt = kt_begin;
    for (; kt + 1 < kt_end; kt += 2) {  // two steps per trip: the register sets alternate
      iter(kt, s0, s1);
      iter(kt + 1, s1, s0);
    }
    if (kt < kt_end) iter(kt, s0, s1);
  };
  if (kt_begin < kt_end) {
    if (prepared)
      run(std::integral_constant<bool, true>{});
    else
      run(std::integral_constant<bool, false>{});
  }

  // Epilogue.  Lane holds D[4*kq + e][r] of every 16x16 tile (i, j).
  if (a.splits == 1) {
    if (a.r > 0) {
      // acc += s * H . B^T on the matrix core in fp32 (V_MFMA_F32_16X16X4_F32: A = s*H,
      // lane l holds row l%16, k = l/16; B = B^T, lane l holds k = l/16, column l%16).
      // Sixteen rank columns per round, their loads issued together (clamped, zero-selected).
      for (int kr = 0; kr < a.r; kr += 16) {
        float hv[4][4], bv[4][4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const int k = kr + 4 * kk + kq;
          const int kc = min(k, a.r - 1);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int ma = m0 + 64 * wm + 16 * i + r;
            const float h = a.H[(size_t)min(ma, a.M - 1) * a.r + kc];
            hv[i][kk] = (ma < a.M && k < a.r) ? a.scale * h : 0.f;
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int n = n0 + 64 * wn + 16 * j + r;
            const float b = h2f(a.B[(size_t)min(n, a.N - 1) * a.r + kc]);
            bv[j][kk] = (n < a.N && k < a.r) ? b : 0.f;
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(hv[i][kk], bv[j][kk], acc[i][j], 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 64 * wn + 16 * j + r;
      if (n >= a.N) continue;
      const float g = a.r > 0 ? h2f(a.gamma[n]) : 1.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m0 + 64 * wm + 16 * i + 4 * kq + e;
          if (m < a.M) a.out[(size_t)m * a.N + n] = f2h_rn(a.r > 0 ? acc[i][j][e] * g : acc[i][j][e]);
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + 64 * wn + 16 * j + r;
        if (n >= a.N) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m0 + 64 * wm + 16 * i + 4 * kq + e;
          if (m < a.M) a.partial[((size_t)split * a.M + m) * a.N + n] = acc[i][j][e];
        }
      }
    }
  }
}

// Prepared outlier entries: one slot per (N tile, chunk) with the row prefix of the
// tile's 128 rows and their entries (col | val << 16) in row order; a slot whose
// entries exceed kEntCap keeps only the prefix (the GEMM then reads that chunk's
// entries from the CSR arrays directly).
__global__ __launch_bounds__(BN) void tile_entries_kernel(const int32_t* __restrict__ offsets,
                                                          const uint16_t* __restrict__ cols,
                                                          const uint8_t* __restrict__ vals, int N, int nch,
                                                          uint32_t* __restrict__ tent) {
  __shared__ int part[2];
  const int tn = blockIdx.x / nch;
  const int ck = blockIdx.x - tn * nch;
  const int t = threadIdx.x;
  const int n = tn * BN + t;
  int o1 = 0, o2 = 0;
  if (n < N) {
    o1 = offsets[(size_t)n * (nch + 1) + ck];
    o2 = offsets[(size_t)n * (nch + 1) + ck + 1];
  }
  const int cnt = o2 - o1;
  int incl = cnt;  // inclusive prefix inside the wave, then across the two waves
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(incl, d);
    if ((t & 63) >= d) incl += u;
  }
  if ((t & 63) == 63) part[t >> 6] = incl;
  __syncthreads();
  if (t >= 64) incl += part[0];
  const int total = part[0] + part[1];
  uint32_t* slot = tent + (size_t)blockIdx.x * kSlotWords;
  slot[t] = (uint32_t)(incl - cnt);
  if (t < kPosWords - BN) slot[BN + t] = (uint32_t)total;
  if (total <= kEntCap)
    for (int j = 0; j < cnt; ++j)
      slot[kPosWords + incl - cnt + j] = (uint32_t)cols[o1 + j] | ((uint32_t)vals[o1 + j] << 16);
}

template <int BITS, bool PER_ROW, bool HAS_CSR, bool X_VEC>
hipError_t launch_variant(const GemmArgs& a, dim3 grid, hipStream_t stream) {
  auto* fn = gemm_kernel<BITS, PER_ROW, HAS_CSR, X_VEC>;
  static bool attr_set = false;  // > 64 KiB of LDS must be requested once per kernel
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(GemmSmem));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(fn, grid, dim3(NT), sizeof(GemmSmem), stream, a);
  return hipGetLastError();
}

template <int BITS, bool X_VEC>
hipError_t launch_bits(const GemmArgs& a, bool per_row, dim3 grid, hipStream_t stream) {
  if (per_row)
    return a.has_csr ? launch_variant<BITS, true, true, X_VEC>(a, grid, stream)
                     : launch_variant<BITS, true, false, X_VEC>(a, grid, stream);
  return a.has_csr ? launch_variant<BITS, false, true, X_VEC>(a, grid, stream)
                   : launch_variant<BITS, false, false, X_VEC>(a, grid, stream);
}

template <bool X_VEC>
hipError_t launch_any(const GemmArgs& a, int bits, bool per_row, dim3 grid, hipStream_t stream) {
  switch (bits) {
    case 1: return launch_bits<1, X_VEC>(a, per_row, grid, stream);
    case 2: return launch_bits<2, X_VEC>(a, per_row, grid, stream);
    case 3: return launch_bits<3, X_VEC>(a, per_row, grid, stream);
    default: return launch_bits<4, X_VEC>(a, per_row, grid, stream);
  }
}

}  // namespace

SplitPlan plan_gemm(const Layer& L, int M, int cu_count, size_t workspace_bytes) {
  SplitPlan p{};
  const int ksteps = std::max(1, (L.K + BK - 1) / BK);
  const int spc = std::max(1, L.chunk / BK);
  const int nchunks = (ksteps + spc - 1) / spc;
  const long tiles = (long)((L.N + BN - 1) / BN) * (long)((M + BM - 1) / BM);
  const int target = std::max(1, cu_count);  // one 512-thread block per CU
  // prepared outlier entries, when the workspace holds them
  const size_t ent_bytes = (L.offsets != nullptr)
                               ? (size_t)((L.N + BN - 1) / BN) * (size_t)L.nch * kSlotWords * sizeof(uint32_t)
                               : 0;
  const size_t ent_room = workspace_bytes >= ent_bytes ? ent_bytes : 0;
  int splits = 1;
  if (tiles < target) splits = (int)std::min<long>((target + tiles - 1) / tiles, kMaxSplits);
  splits = std::min(splits, nchunks);  // splits hold whole outlier chunks
  const size_t per_split = (size_t)M * (size_t)L.N * sizeof(float);
  while (splits > 1 && (size_t)splits * per_split + ent_room > workspace_bytes) --splits;
  const int cps = (nchunks + splits - 1) / splits;  // chunks per split
  const int kps = cps * spc;
  p.splits = (ksteps + kps - 1) / kps;
  p.slabs_per_split = kps;
  p.seg_slabs = 0;
  const size_t part_bytes = p.splits > 1 ? (size_t)p.splits * per_split : 0;
  p.aux_bytes = (part_bytes + ent_bytes <= workspace_bytes) ? ent_bytes : 0;
  p.workspace_bytes = part_bytes + p.aux_bytes;
  return p;
}

hipError_t launch_gemm(const Layer& L, const Dora& D, const uint16_t* X, uint16_t* out, int M,
                       const SplitPlan& plan, float* workspace, hipStream_t stream) {
  GemmArgs a{};
  a.q = L.q;
  a.lut = L.lut;
  a.X = X;
  a.out = out;
  a.partial = workspace;
  a.offsets = L.offsets;
  a.cols = L.cols;
  a.vals = L.vals;
  a.has_csr = (L.offsets && L.cols && L.vals) ? 1 : 0;
  a.B = D.B;
  a.H = D.H;
  a.gamma = D.gamma;
  a.scale = D.scale;
  a.r = D.r;
  a.M = M;
  a.N = L.N;
  a.K = L.K;
  a.wpr = L.wpr;
  a.G = L.group_size;
  a.ng = L.ng;
  a.nch = L.nch;
  a.chunk = L.chunk;
  a.g_magic = L.group_size > 0 ? (uint32_t)((0x100000000ull / (uint64_t)L.group_size) + 1ull) : 0u;
  a.ksteps_per_split = plan.slabs_per_split;
  a.splits = plan.splits;
  a.tiles_m = (M + BM - 1) / BM;
  a.tiles_n = (L.N + BN - 1) / BN;
  a.tiles = a.tiles_m * a.tiles_n;
  const bool x_vec = (reinterpret_cast<uintptr_t>(X) & 15u) == 0 && (L.K % 8) == 0 && L.K >= 8;
  const size_t part_bytes = plan.splits > 1 ? (size_t)plan.splits * M * L.N * sizeof(float) : 0;
  a.tent = nullptr;
  if (a.has_csr && plan.aux_bytes > 0) {
    a.tent = reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(workspace) + part_bytes);
    hipLaunchKernelGGL(tile_entries_kernel, dim3(a.tiles_n * L.nch), dim3(BN), 0, stream, L.offsets, L.cols,
                       L.vals, L.N, L.nch, const_cast<uint32_t*>(a.tent));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const dim3 grid(a.tiles * plan.splits);
  const bool per_row = L.group_size <= 0 || L.ng == 1;
  const hipError_t err = x_vec ? launch_any<true>(a, L.bits, per_row, grid, stream)
                               : launch_any<false>(a, L.bits, per_row, grid, stream);
  if (err != hipSuccess) return err;
  if (plan.splits > 1) return launch_splitk_reduce(workspace, plan.splits, M, L.N, D, out, stream);
  return hipSuccess;
}

}  // namespace wlq
