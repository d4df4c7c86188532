// Decode-shaped WLQ product (M = 1..32 activation rows): weight-streaming kernel.
//
// Reference behaviour replaced: gemv_chunk_csr_kernel + launch_gemv_chunk_csr
// (csrc/gemv_kernel.cu:86-320, :396-457) for M == 1 and gemm_metalog_dora_kernel
// (csrc/gemm_kernel.cu:32-294) for 2 <= M < 16, plus the M >= 16 dequant+HGEMM
// path (csrc/vllm_binding.cpp:355-393) for M <= 32.
//
// Work decomposition.  A block is 4 waves; wave w owns a 16-row tile of W, the
// block owns a contiguous range of K "slabs" (4 code windows = 128 columns for
// 4-bit).  Per slab, lane l = r + 16*kq streams one 16-byte code window of row
// r (columns kq*WIN .. +WIN of the slab), dequantizes it through its LUT byte
// planes and feeds V_MFMA_F32_16X16X32_F16 as the B operand; the A operand is the
// activation block (rows 16*mt + r) read from LDS, where it was staged in the
// same column order P.  The 16x16 accumulator keeps the whole K reduction in the
// matrix core; no cross-lane reduction is needed for the dense part.
//
// Outliers use the delta form of the reference GEMV (csrc/gemv_kernel.cu:262-288):
// after the dense loop each lane walks every 4th CSR entry of its row in the
// block's column range and accumulates (w_true - lut[code]) * x[i, col] for all
// activation rows; the four lanes of a row are summed with two xor-shuffles.
// Split-K partials go to an fp32 workspace and a second kernel applies the
// DoRA epilogue; otherwise the epilogue runs here.
#include <algorithm>
#include <utility>

#include "wlq_device.h"
#include "wlq_internal.h"

namespace wlq {
namespace {

constexpr int kWaves = 4;
constexpr int kRowsPerBlock = 16 * kWaves;
constexpr int kXStageBytes = 32768;  // activation staging budget per block
constexpr int kMaxM = 32;
constexpr int kMaxSplits = 64;

struct SkinnyArgs {
  const uint32_t* q;
  const uint16_t* lut;
  const uint16_t* x;
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
  uint32_t g_magic;  // floor(2^32 / G) + 1: floor(c / G) == umulhi(c, g_magic) for c < 2^20, G < 4096
  int slabs_per_split, seg_slabs, xstride, splits;
  int x_vec;         // 16-byte loads of x rows are aligned
  int has_csr;
};

__device__ __forceinline__ int group_of(int col, uint32_t magic) { return (int)__umulhi((uint32_t)col, magic); }

// Stage activations x[0:M, c_a : c_a + ncols) into LDS in column order P
// (zero beyond K).  ncols is a multiple of 8.
__device__ __forceinline__ void stage_x(const SkinnyArgs& a, uint16_t* xs, int c_a, int ncols) {
  const int upr = ncols >> 3;
  const int total = a.M * upr;
  for (int u = threadIdx.x; u < total; u += blockDim.x) {
    const int i = u / upr;
    const int c8 = u - i * upr;
    const int col = c_a + (c8 << 3);
    const uint16_t* src = a.x + (size_t)i * a.K + col;
    u32x4_t v;
    if (a.x_vec && col + 8 <= a.K) {
      v = *reinterpret_cast<const u32x4_t*>(src);
    } else {
      uint32_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = (col + j < a.K) ? (uint32_t)src[j] : 0u;
      v.x = e[0] | (e[1] << 16);
      v.y = e[2] | (e[3] << 16);
      v.z = e[4] | (e[5] << 16);
      v.w = e[6] | (e[7] << 16);
    }
    *reinterpret_cast<u32x4_t*>(xs + i * a.xstride + (c8 << 3)) = permute_p(v);
  }
}

template <int BITS>
struct LaneState {
  LutPlanes<BITS> pl0, pl1;
  int split_col;  // first column served by pl1 (TWO_LUT)
};

// One 8-column block S of the lane window: dequantize and multiply.
template <int BITS, int MT, bool TWO_LUT, int S>
__device__ __forceinline__ void window_block(const uint32_t w[4], const LaneState<BITS>& st, int c0,
                                             const uint16_t* xs, int xstride, int xoff, int r, int M,
                                             float4_t acc[MT]) {
  uint32_t b[4];
  if constexpr (TWO_LUT) {
    const bool hi = (c0 + 8 * S) >= st.split_col;
    LutPlanes<BITS> t;
#pragma unroll
    for (int p = 0; p < LutPlanes<BITS>::kRegs; ++p) {
      t.lo[p] = hi ? st.pl1.lo[p] : st.pl0.lo[p];
      t.hi[p] = hi ? st.pl1.hi[p] : st.pl0.hi[p];
    }
    dequant_block<BITS, S>(w, t, b);
  } else {
    dequant_block<BITS, S>(w, st.pl0, b);
  }
  u32x4_t bv;
  bv.x = b[0]; bv.y = b[1]; bv.z = b[2]; bv.w = b[3];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int xr = 16 * mt + r;
    u32x4_t av = {0u, 0u, 0u, 0u};
    if (xr < M) av = *reinterpret_cast<const u32x4_t*>(xs + xr * xstride + xoff + 8 * S);
    acc[mt] = mfma16x16x32(av, bv, acc[mt]);
  }
}

template <int BITS, int MT, bool TWO_LUT, int... S>
__device__ __forceinline__ void window_all(std::integer_sequence<int, S...>, const uint32_t w[4],
                                           const LaneState<BITS>& st, int c0, const uint16_t* xs, int xstride,
                                           int xoff, int r, int M, float4_t acc[MT]) {
  (window_block<BITS, MT, TWO_LUT, S>(w, st, c0, xs, xstride, xoff, r, M, acc), ...);
}

template <int BITS, int MT, int MB, bool PER_ROW, bool TWO_LUT>
__global__ __launch_bounds__(256) void skinny_kernel(const SkinnyArgs a) {
  constexpr int WIN = CodeGeom<BITS>::kWin;
  constexpr int SLAB = 4 * WIN;
  constexpr int NCB = 1 << BITS;
  extern __shared__ __align__(16) uint16_t xs[];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int kq = lane >> 4;
  const int n = blockIdx.x * kRowsPerBlock + wave * 16 + r;
  const bool row_ok = n < a.N;
  const int nc = row_ok ? n : (a.N - 1);
  const uint32_t* qrow = a.q + (size_t)nc * a.wpr;
  const uint16_t* lrow = a.lut + (size_t)nc * a.ng * NCB;

  const int total_slabs = (a.K + SLAB - 1) / SLAB;
  const int t_begin = blockIdx.y * a.slabs_per_split;
  const int t_end = min(total_slabs, t_begin + a.slabs_per_split);

  float4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = float4_t{0.f, 0.f, 0.f, 0.f};

  LaneState<BITS> st;
  st.split_col = 0x7fffffff;
  if constexpr (PER_ROW) {
    LutRaw<BITS> raw;
    lut_load<BITS>(raw, lrow);
    st.pl0 = lut_planes<BITS>(raw);
    st.pl1 = st.pl0;
  }

  for (int seg = t_begin; seg < t_end; seg += a.seg_slabs) {
    const int seg_end = min(t_end, seg + a.seg_slabs);
    if (seg != t_begin) __syncthreads();
    stage_x(a, xs, seg * SLAB, (seg_end - seg) * SLAB);
    __syncthreads();
    for (int t = seg; t < seg_end; ++t) {
      const int wi = t * 16 + kq * 4;  // 16 words per slab for every width
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      if (row_ok && wi + 4 <= a.wpr) {
        const u32x4_t v = *reinterpret_cast<const u32x4_t*>(qrow + wi);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
      }
      const int c0 = t * SLAB + kq * WIN;
      if constexpr (!PER_ROW) {
        const int g0 = min(group_of(c0, a.g_magic), a.ng - 1);
        LutRaw<BITS> raw;
        lut_load<BITS>(raw, lrow + g0 * NCB);
        st.pl0 = lut_planes<BITS>(raw);
        if constexpr (TWO_LUT) {
          const int g1 = min(group_of(c0 + WIN - 1, a.g_magic), a.ng - 1);
          LutRaw<BITS> raw1;
          lut_load<BITS>(raw1, lrow + g1 * NCB);
          st.pl1 = lut_planes<BITS>(raw1);
          st.split_col = (g1 != g0) ? g1 * a.G : 0x7fffffff;
        }
      }
      const int xoff = (t - seg) * SLAB + kq * WIN;
      window_all<BITS, MT, TWO_LUT>(std::make_integer_sequence<int, WIN / 8>{}, w, st, c0, xs, a.xstride, xoff, r,
                                    a.M, acc);
    }
  }

  if (a.has_csr) {
    float corr[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) corr[i] = 0.f;
    const int k_lo = t_begin * SLAB;
    const int k_hi = min(a.K, t_end * SLAB);
    if (row_ok && k_lo < k_hi) {
      const int c_lo = k_lo / a.chunk;
      const int c_hi = min(a.nch, (k_hi + a.chunk - 1) / a.chunk);
      const int32_t* offr = a.offsets + (size_t)n * (a.nch + 1);
      for (int c = c_lo; c < c_hi; ++c) {
        const int s0 = offr[c];
        const int s1 = offr[c + 1];
        const int cbase = c * a.chunk;
        for (int e = s0 + kq; e < s1; e += 4) {
          const int col = cbase + (int)a.cols[e];
          if (col >= k_lo && col < k_hi) {
            const uint32_t code = code_at<BITS>(qrow, col);
            const int g = PER_ROW ? 0 : min(group_of(col, a.g_magic), a.ng - 1);
            const float d = h2f((uint16_t)((uint32_t)a.vals[e] << 8)) - h2f(lrow[g * NCB + code]);
#pragma unroll
            for (int i = 0; i < MB; ++i)
              if (i < a.M) corr[i] += d * h2f(a.x[(size_t)i * a.K + col]);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if (i < a.M) {
        float v = corr[i];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (kq == ((i >> 2) & 3)) acc[i >> 4][i & 3] += v;
      }
    }
  }

  const bool fused = a.splits == 1;
  const int n_out = n;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * mt + 4 * kq + e;
      if (i < a.M && row_ok) {
        float v = acc[mt][e];
        if (fused) {
          if (a.r > 0) {
            float ls = 0.f;
            const float* h = a.H + (size_t)i * a.r;
            const uint16_t* bb = a.B + (size_t)n_out * a.r;
            for (int j = 0; j < a.r; ++j) ls += h[j] * h2f(bb[j]);
            v = (v + a.scale * ls) * h2f(a.gamma[n_out]);
          }
          a.out[(size_t)i * a.N + n_out] = f2h_rn(v);
        } else {
          a.partial[((size_t)blockIdx.y * a.M + i) * a.N + n_out] = v;
        }
      }
    }
  }
}

template <int BITS, int MT, int MB, bool PER_ROW, bool TWO_LUT>
hipError_t launch_variant(const SkinnyArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  hipLaunchKernelGGL((skinny_kernel<BITS, MT, MB, PER_ROW, TWO_LUT>), grid, dim3(256), lds, stream, a);
  return hipGetLastError();
}

template <int BITS, int MT, int MB>
hipError_t launch_lut_mode(const SkinnyArgs& a, int mode, dim3 grid, size_t lds, hipStream_t stream) {
  switch (mode) {
    case 0: return launch_variant<BITS, MT, MB, true, false>(a, grid, lds, stream);
    case 1: return launch_variant<BITS, MT, MB, false, false>(a, grid, lds, stream);
    default: return launch_variant<BITS, MT, MB, false, true>(a, grid, lds, stream);
  }
}

template <int BITS>
hipError_t launch_bits(const SkinnyArgs& a, int mode, dim3 grid, size_t lds, hipStream_t stream) {
  if (a.M == 1) return launch_lut_mode<BITS, 1, 1>(a, mode, grid, lds, stream);
  if (a.M <= 4) return launch_lut_mode<BITS, 1, 4>(a, mode, grid, lds, stream);
  if (a.M <= 16) return launch_lut_mode<BITS, 1, 16>(a, mode, grid, lds, stream);
  return launch_lut_mode<BITS, 2, 32>(a, mode, grid, lds, stream);
}

int window_cols(int bits) { return bits == 4 ? 32 : bits == 3 ? 40 : bits == 2 ? 64 : 128; }

}  // namespace

int slab_cols(int bits) { return 4 * window_cols(bits); }
int skinny_max_m() { return kMaxM; }

SplitPlan plan_skinny(const Layer& L, int M, int cu_count, size_t workspace_bytes) {
  SplitPlan p{};
  const int slab = slab_cols(L.bits);
  const int total = std::max(1, (L.K + slab - 1) / slab);
  const int row_blocks = (L.N + kRowsPerBlock - 1) / kRowsPerBlock;
  const int target = 2 * std::max(1, cu_count);
  int splits = std::max(1, (target + row_blocks - 1) / row_blocks);
  splits = std::min(splits, std::min(total, kMaxSplits));
  const size_t per_split = (size_t)M * (size_t)L.N * sizeof(float);
  while (splits > 1 && (size_t)splits * per_split > workspace_bytes) --splits;
  int sps = (total + splits - 1) / splits;
  const int spc = std::max(1, L.chunk / slab);
  if (sps >= spc) sps = (sps + spc - 1) / spc * spc;
  splits = (total + sps - 1) / sps;
  p.splits = splits;
  p.slabs_per_split = sps;
  const int seg_cols_max = kXStageBytes / (2 * std::max(1, M));
  p.seg_slabs = std::max(1, std::min(sps, (seg_cols_max - 8) / slab));
  p.workspace_bytes = splits > 1 ? (size_t)splits * per_split : 0;
  return p;
}

hipError_t launch_skinny(const Layer& L, const Dora& D, const uint16_t* x, uint16_t* out, int M,
                         const SplitPlan& plan, float* workspace, hipStream_t stream) {
  SkinnyArgs a{};
  a.q = L.q;
  a.lut = L.lut;
  a.x = x;
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
  a.slabs_per_split = plan.slabs_per_split;
  a.seg_slabs = plan.seg_slabs;
  const int slab = slab_cols(L.bits);
  a.xstride = plan.seg_slabs * slab + 8;
  a.splits = plan.splits;
  a.x_vec = ((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (L.K % 8) == 0) ? 1 : 0;
  const size_t lds = (size_t)M * a.xstride * sizeof(uint16_t);
  const dim3 grid((L.N + kRowsPerBlock - 1) / kRowsPerBlock, plan.splits);
  const bool per_row = L.group_size <= 0 || L.ng == 1;
  const int mode = per_row ? 0 : ((L.group_size % window_cols(L.bits)) == 0 ? 1 : 2);
  hipError_t err;
  switch (L.bits) {
    case 1: err = launch_bits<1>(a, mode, grid, lds, stream); break;
    case 2: err = launch_bits<2>(a, mode, grid, lds, stream); break;
    case 3: err = launch_bits<3>(a, mode, grid, lds, stream); break;
    default: err = launch_bits<4>(a, mode, grid, lds, stream); break;
  }
  if (err != hipSuccess) return err;
  if (plan.splits > 1) return launch_splitk_reduce(workspace, plan.splits, M, L.N, D, out, stream);
  return hipSuccess;
}

}  // namespace wlq
