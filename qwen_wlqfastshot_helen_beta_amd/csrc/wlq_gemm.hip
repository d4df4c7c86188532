// Prefill-shaped WLQ product (M > 32): LDS-staged dequantization feeding MFMA.
//
// Reference behaviour replaced: the M >= 16 path of gemm_forward
// (csrc/vllm_binding.cpp:355-393: full-matrix dequant into a workspace, cuBLAS
// HGEMM, separate DoRA pass) and gemm_metalog_dora_kernel's overwrite semantics
// (csrc/gemm_kernel.cu:204-228).  Here W is never materialized in HBM.
//
// Block tile 128 (M) x 128 (N), K step 64, 256 threads = 4 waves in a 2x2
// arrangement, each wave a 64x64 sub-tile of V_MFMA_F32_16X16X32_F16.  Per K
// step the block stages X[128, 64] (fp16, column order P inside 8-blocks) and
// the dequantized W tile [128, 64] into one of two LDS buffers; thread (row,
// half) expands one 32-column code window of one row through its LUT byte
// planes and then overwrites that window's outliers in LDS (outlier value
// e5m2 << 8, the reference's overwrite).  The entries of the current outlier
// chunk for the block's 128 rows are staged into LDS once per chunk.
// Split-K partials (when the tile grid alone cannot fill the GPU) go to an fp32
// workspace and the split reduction applies the DoRA epilogue.
#include <algorithm>

#include "wlq_device.h"
#include "wlq_internal.h"

namespace wlq {
namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int LDS_ROW = BK + 8;  // halves per LDS row (16-byte pad)
constexpr int kEntCap = 1024;    // staged outlier entries per chunk
constexpr int kMaxSplits = 32;

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
  int x_vec;
  int has_csr;
};

struct GemmSmem {
  uint16_t a[2][BM * LDS_ROW];
  uint16_t b[2][BN * LDS_ROW];
  uint32_t ent[kEntCap];
  int pos[BN + 1];
  int cnt[BN];
};

__device__ __forceinline__ int group_of(int col, uint32_t magic) { return (int)__umulhi((uint32_t)col, magic); }

// Code window of 32 columns starting at column c (c % 32 == 0) of a packed row.
template <int BITS>
__device__ __forceinline__ void load_window32(const uint32_t* __restrict__ qrow, int c, int wpr, bool ok,
                                              uint32_t w[4]) {
  w[0] = w[1] = w[2] = w[3] = 0u;
  if (!ok) return;
  if constexpr (BITS == 4) {
    const int wi = c >> 3;
    if (wi + 4 <= wpr) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(qrow + wi);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
  } else if constexpr (BITS == 2) {
    const int wi = c >> 4;
    if (wi + 2 <= wpr) {
      const u32x2_t v = *reinterpret_cast<const u32x2_t*>(qrow + wi);
      w[0] = v.x; w[1] = v.y;
    }
  } else if constexpr (BITS == 1) {
    const int wi = c >> 5;
    if (wi < wpr) w[0] = qrow[wi];
  } else {
    const int wi = c / 10;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = (wi + j < wpr) ? qrow[wi + j] : 0u;
  }
}

// Selector bytes of 8-column block b of a 32-column window starting at column c.
template <int BITS>
__device__ __forceinline__ void window32_selectors(const uint32_t w[4], int c, int b, uint32_t& se, uint32_t& so) {
  uint32_t code[8];
  if constexpr (BITS == 2) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int idx = 8 * b + j;
      code[j] = (w[idx >> 4] >> (2 * (idx & 15))) & 3u;
    }
  } else if constexpr (BITS == 1) {
#pragma unroll
    for (int j = 0; j < 8; ++j) code[j] = (w[0] >> (8 * b + j)) & 1u;
  } else {  // 3-bit: window starts at slot c % 10 of word c / 10
    const int base = c - (c / 10) * 10;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int idx = base + 8 * b + j;         // < 40
      const int wsel = (idx * 205) >> 11;       // idx / 10 for idx < 1024
      const int slot = idx - wsel * 10;
      const uint32_t word = wsel == 0 ? w[0] : wsel == 1 ? w[1] : wsel == 2 ? w[2] : w[3];
      code[j] = (word >> (3 * slot)) & 7u;
    }
  }
  se = code[0] | (code[2] << 8) | (code[4] << 16) | (code[6] << 24);
  so = code[1] | (code[3] << 8) | (code[5] << 16) | (code[7] << 24);
}

template <int BITS>
__device__ __forceinline__ void dequant_window32(const uint32_t w[4], int c, int b, const LutPlanes<BITS>& t,
                                                 uint32_t out[4]) {
  if constexpr (BITS == 4) {
    dequant_word4(w[b], t, out);
  } else {
    uint32_t se, so;
    window32_selectors<BITS>(w, c, b, se, so);
    dequant_sel8<BITS>(se, so, t, out);
  }
}

// Stage the outlier entries of chunk `c` for the block's rows into LDS.
// Returns true when they fit (block-uniform).
__device__ __forceinline__ bool stage_chunk_entries(const GemmArgs& a, GemmSmem& sm, int n0, int c) {
  const int tid = threadIdx.x;
  if (tid < BN) {
    const int n = n0 + tid;
    int cnt = 0;
    if (n < a.N) {
      const int32_t* offr = a.offsets + (size_t)n * (a.nch + 1);
      cnt = offr[c + 1] - offr[c];
    }
    sm.cnt[tid] = cnt;
  }
  __syncthreads();
  if (tid < 64) {  // exclusive prefix over 128 counts by one wave
    const int v0 = sm.cnt[2 * tid];
    const int v1 = sm.cnt[2 * tid + 1];
    int s = v0 + v1;
    int incl = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int t = __shfl_up(incl, d);
      if (tid >= d) incl += t;
    }
    const int excl = incl - s;
    sm.pos[2 * tid] = excl;
    sm.pos[2 * tid + 1] = excl + v0;
    if (tid == 63) sm.pos[BN] = incl;
  }
  __syncthreads();
  const bool fits = sm.pos[BN] <= kEntCap;
  if (fits) {
    const int nl = tid >> 1;
    const int h = tid & 1;
    const int n = n0 + nl;
    if (n < a.N) {
      const int s0 = a.offsets[(size_t)n * (a.nch + 1) + c];
      const int cnt = sm.cnt[nl];
      const int p = sm.pos[nl];
      for (int j = h; j < cnt; j += 2) {
        const int e = s0 + j;
        sm.ent[p + j] = (uint32_t)a.cols[e] | ((uint32_t)a.vals[e] << 16);
      }
    }
  }
  __syncthreads();
  return fits;
}

template <int BITS, bool PER_ROW>
__global__ __launch_bounds__(256, 2) void gemm_kernel(const GemmArgs a) {
  constexpr int NCB = 1 << BITS;
  __shared__ __align__(16) GemmSmem sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int r = lane & 15;
  const int kq = lane >> 4;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;

  const int ksteps_total = (a.K + BK - 1) / BK;
  const int kt_begin = blockIdx.z * a.ksteps_per_split;
  const int kt_end = min(ksteps_total, kt_begin + a.ksteps_per_split);

  // B-tile producer role: row nl, 32-column half h of each K step.
  const int nl = tid >> 1;
  const int hh = tid & 1;
  const int nb = n0 + nl;
  const bool brow_ok = nb < a.N;
  const int nbc = brow_ok ? nb : (a.N - 1);
  const uint32_t* qrow = a.q + (size_t)nbc * a.wpr;
  const uint16_t* lrow = a.lut + (size_t)nbc * a.ng * NCB;

  LutPlanes<BITS> pl;
  if constexpr (PER_ROW) {
    LutRaw<BITS> raw;
    lut_load<BITS>(raw, lrow);
    pl = lut_planes<BITS>(raw);
  }

  float4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  // Registers carrying one K step from global memory to LDS.
  u32x4_t xa[4];
  uint32_t cw[4];
  LutRaw<BITS> lraw;

  auto load_step = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = tid + 256 * j;
      const int row = u >> 3;
      const int c8 = u & 7;
      const int m = m0 + row;
      const int col = k0 + 8 * c8;
      u32x4_t v = {0u, 0u, 0u, 0u};
      if (m < a.M) {
        const uint16_t* src = a.X + (size_t)m * a.K + col;
        if (a.x_vec && col + 8 <= a.K) {
          v = *reinterpret_cast<const u32x4_t*>(src);
        } else {
          uint32_t e[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) e[q] = (col + q < a.K) ? (uint32_t)src[q] : 0u;
          v.x = e[0] | (e[1] << 16);
          v.y = e[2] | (e[3] << 16);
          v.z = e[4] | (e[5] << 16);
          v.w = e[6] | (e[7] << 16);
        }
      }
      xa[j] = v;
    }
    const int c = k0 + 32 * hh;
    load_window32<BITS>(qrow, c, a.wpr, brow_ok, cw);
    if constexpr (!PER_ROW) {
      const int g = min(group_of(c, a.g_magic), a.ng - 1);
      lut_load<BITS>(lraw, lrow + g * NCB);
    }
  };

  int staged_chunk = -1;
  bool ent_fit = true;

  auto store_step = [&](int kt, int buf) {
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int u = tid + 256 * j;
      const int row = u >> 3;
      const int c8 = u & 7;
      *reinterpret_cast<u32x4_t*>(&sm.a[buf][row * LDS_ROW + 8 * c8]) = permute_p(xa[j]);
    }
    if constexpr (!PER_ROW) pl = lut_planes<BITS>(lraw);
    const int c = k0 + 32 * hh;
    uint16_t* brow = &sm.b[buf][nl * LDS_ROW + 32 * hh];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      uint32_t o[4];
      dequant_window32<BITS>(cw, c, b, pl, o);
      u32x4_t v;
      v.x = o[0]; v.y = o[1]; v.z = o[2]; v.w = o[3];
      *reinterpret_cast<u32x4_t*>(brow + 8 * b) = v;
    }
    if (a.has_csr && brow_ok) {
      const int chunk_idx = k0 / a.chunk;
      const int lo = c - chunk_idx * a.chunk;  // window start inside the chunk
      if (ent_fit) {
        const int p0 = sm.pos[nl];
        const int p1 = sm.pos[nl + 1];
        for (int p = p0; p < p1; ++p) {
          const uint32_t ent = sm.ent[p];
          const int cc = (int)(ent & 0xFFFFu) - lo;
          if (cc >= 0 && cc < 32 && c + cc < a.K) brow[8 * (cc >> 3) + p_slot(cc & 7)] = (uint16_t)((ent >> 16) << 8);
        }
      } else {
        const int32_t* offr = a.offsets + (size_t)nb * (a.nch + 1);
        const int s1 = offr[chunk_idx + 1];
        for (int e = offr[chunk_idx]; e < s1; ++e) {
          const int cc = (int)a.cols[e] - lo;
          if (cc >= 0 && cc < 32 && c + cc < a.K)
            brow[8 * (cc >> 3) + p_slot(cc & 7)] = (uint16_t)((uint32_t)a.vals[e] << 8);
        }
      }
    }
  };

  auto ensure_chunk = [&](int kt) {
    if (!a.has_csr) return;
    const int chunk_idx = (kt * BK) / a.chunk;
    if (chunk_idx != staged_chunk) {
      ent_fit = stage_chunk_entries(a, sm, n0, chunk_idx);
      staged_chunk = chunk_idx;
    }
  };

  if (kt_begin < kt_end) {
    load_step(kt_begin);
    ensure_chunk(kt_begin);
    store_step(kt_begin, 0);
    __syncthreads();
  }
  for (int kt = kt_begin; kt < kt_end; ++kt) {
    const int buf = (kt - kt_begin) & 1;
    const bool more = kt + 1 < kt_end;
    if (more) load_step(kt + 1);
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
    if (more) {
      ensure_chunk(kt + 1);
      store_step(kt + 1, buf ^ 1);
      __syncthreads();
    }
  }

  // Epilogue: lane holds D[4*kq + e][r] of every 16x16 tile.
  const bool fused = a.splits == 1;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 64 * wn + 16 * j + r;
      if (n >= a.N) continue;
      float gam = 1.f;
      if (fused && a.r > 0) gam = h2f(a.gamma[n]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + 64 * wm + 16 * i + 4 * kq + e;
        if (m >= a.M) continue;
        float v = acc[i][j][e];
        if (fused) {
          if (a.r > 0) {
            float ls = 0.f;
            const float* hrow = a.H + (size_t)m * a.r;
            const uint16_t* brw = a.B + (size_t)n * a.r;
            for (int q = 0; q < a.r; ++q) ls += hrow[q] * h2f(brw[q]);
            v = (v + a.scale * ls) * gam;
          }
          a.out[(size_t)m * a.N + n] = f2h_rn(v);
        } else {
          a.partial[((size_t)blockIdx.z * a.M + m) * a.N + n] = v;
        }
      }
    }
  }
}

template <int BITS>
hipError_t launch_bits(const GemmArgs& a, bool per_row, dim3 grid, hipStream_t stream) {
  if (per_row)
    hipLaunchKernelGGL((gemm_kernel<BITS, true>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((gemm_kernel<BITS, false>), grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

SplitPlan plan_gemm(const Layer& L, int M, int cu_count, size_t workspace_bytes) {
  SplitPlan p{};
  const int ksteps = std::max(1, (L.K + BK - 1) / BK);
  const long tiles = (long)((L.N + BN - 1) / BN) * (long)((M + BM - 1) / BM);
  const int target = 2 * std::max(1, cu_count);
  int splits = 1;
  if (tiles < target) splits = (int)std::min<long>((target + tiles - 1) / tiles, kMaxSplits);
  splits = std::min(splits, std::max(1, ksteps / 4));
  const size_t per_split = (size_t)M * (size_t)L.N * sizeof(float);
  while (splits > 1 && (size_t)splits * per_split > workspace_bytes) --splits;
  const int kps = (ksteps + splits - 1) / splits;
  p.splits = (ksteps + kps - 1) / kps;
  p.slabs_per_split = kps;
  p.seg_slabs = 0;
  p.workspace_bytes = p.splits > 1 ? (size_t)p.splits * per_split : 0;
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
  a.x_vec = ((reinterpret_cast<uintptr_t>(X) & 15u) == 0 && (L.K % 8) == 0) ? 1 : 0;
  const dim3 grid((L.N + BN - 1) / BN, (M + BM - 1) / BM, plan.splits);
  const bool per_row = L.group_size <= 0 || L.ng == 1;
  hipError_t err;
  switch (L.bits) {
    case 1: err = launch_bits<1>(a, per_row, grid, stream); break;
    case 2: err = launch_bits<2>(a, per_row, grid, stream); break;
    case 3: err = launch_bits<3>(a, per_row, grid, stream); break;
    default: err = launch_bits<4>(a, per_row, grid, stream); break;
  }
  if (err != hipSuccess) return err;
  if (plan.splits > 1) return launch_splitk_reduce(workspace, plan.splits, M, L.N, D, out, stream);
  return hipSuccess;
}

}  // namespace wlq
