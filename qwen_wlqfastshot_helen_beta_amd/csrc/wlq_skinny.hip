// Decode-shaped WLQ product (M = 1..32 activation rows): weight-streaming kernel.
//
// Reference behaviour replaced: gemv_chunk_csr_kernel + launch_gemv_chunk_csr
// (csrc/gemv_kernel.cu:86-320, :396-457) for M == 1 and gemm_metalog_dora_kernel
// (csrc/gemm_kernel.cu:32-294) for 2 <= M < 16, plus the M >= 16 dequant+HGEMM
// path (csrc/vllm_binding.cpp:355-393) for M <= 32.
//
// Work decomposition.  The grid is one-dimensional: first the DoRA blocks (one
// per 512 columns, computing partial x.A^T sums with MFMA when the caller did
// not pass H), then row_blocks x splits product blocks.  A product block is 4
// waves; wave w owns a 16-row tile of W and the block owns a contiguous range
// of K "slabs" (4 code windows, 128 columns for 4-bit).  Per slab, lane
// l = r + 16*kq takes one 16-byte code window of row r (columns kq*WIN..+WIN of
// the slab), dequantizes it through its LUT byte planes and feeds
// V_MFMA_F32_16X16X32_F16 as the B operand; the A operand (activation rows
// 16*mt + r) comes from LDS, staged in the same column order P.  The 16x16
// accumulator keeps the K reduction inside the matrix core.
//
// 4-bit fast path, pipelined per 512-column outlier chunk (= 4 slabs): the code
// windows and LUT quarters of the next chunk are loaded while the current one
// is consumed (unconditional loads, so HBM latency overlaps the dequant/MFMA
// work); each of the four lanes of a row loads one quarter (4 entries) of the
// row's group LUT, splits it into byte planes and the lanes exchange planes
// through wave-private LDS, so a 16-entry LUT costs one 8-byte load and two
// perms per lane.  The chunk's code windows and LUT planes stay in LDS tiles,
// and the chunk's outliers are applied right after its four slabs in the delta
// form of the reference GEMV (csrc/gemv_kernel.cu:262-288): each lane takes
// every 4th CSR entry of its row and accumulates (w_true - lut[code]) * x[i, col]
// with code and LUT value read from the tiles; CSR offsets are fetched two
// chunks ahead and entries one chunk ahead.  The four lanes of a row are summed
// with two xor-shuffles at the end.  Other widths (generic kernel) walk the
// block's CSR entries after the dense loop with global loads.
//
// Output: with one split and H supplied by the caller the epilogue
// fp16_rn((acc + s * H.B) * gamma) runs here; otherwise fp32 partials go to
// the workspace and finalize_kernel (wlq_epilogue.hip) sums splits and DoRA
// partials, rounds H to fp16 (the reference's F.linear output type) and applies
// the epilogue.
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
constexpr int kPF = 4;               // slabs in flight per wave (4-bit path)
constexpr int kHCols = 512;          // columns per DoRA block
constexpr int kMaxFusedRank = 64;
constexpr int kMaxFastSlabs = 60;    // slabs per 4-bit block: any start slab then spans <= 16 chunks

struct SkinnyArgs {
  const uint32_t* q;
  const uint16_t* lut;
  const uint16_t* x;
  uint16_t* out;
  float* partial;   // [splits, M, N]
  float* hpart;     // [h_blocks, M, r] (fused DoRA) or nullptr
  const int32_t* offsets;
  const uint16_t* cols;
  const uint8_t* vals;
  const uint16_t* B;
  const float* H;
  const uint16_t* gamma;
  const uint16_t* A;  // lora_A [r, K] for the fused path
  float scale;
  int r;
  int M, N, K, wpr, G, ng, nch, chunk;
  uint32_t g_magic;  // floor(2^32 / G) + 1: floor(c / G) == umulhi(c, g_magic) for c < 2^20, G < 4096
  int slabs_per_split, seg_slabs, xstride, splits, row_blocks, h_blocks;
  int x_vec;         // 16-byte loads of x rows are aligned
  int has_csr;
  int direct_out;    // epilogue in this kernel (one split, H given)
  // In-kernel completion: arrival counters (one per row block, zero between calls);
  // the block that arrives last for a row block sums the partials and applies the
  // epilogue.  Arrivals per row block = splits + h_blocks.
  uint32_t* sync;    // nullptr: a separate finalize kernel finishes
  int arrivals;
};

// Cross-block hand-off without cache maintenance: partials and DoRA partials are
// stored and loaded as device-scope (relaxed) atomics, which are coherent across
// the XCDs' L2 caches; a block waits for its stores to complete before it counts
// its arrival, and the last block loads only after its count returned.  (Full
// device-scope fences would write back / invalidate whole L2 caches instead.)
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void fence_release() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ uint32_t load_dev(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void raise_error(uint32_t* sync, uint32_t bit) {
  __hip_atomic_fetch_or(sync + kSyncErrorWord, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
constexpr uint16_t kHalfNaN = 0x7E00u;
__device__ __forceinline__ void fence_acquire() { asm volatile("" ::: "memory"); }

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

// 16-byte load of 8 fp16 starting at column k of a row of length K (zeros past K).
__device__ __forceinline__ u32x4_t load8(const uint16_t* row, int k, int K, bool vec) {
  u32x4_t v = {0u, 0u, 0u, 0u};
  if (vec && k + 8 <= K) return *reinterpret_cast<const u32x4_t*>(row + k);
  uint32_t e[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) e[j] = (k + j < K) ? (uint32_t)row[k + j] : 0u;
  v.x = e[0] | (e[1] << 16);
  v.y = e[2] | (e[3] << 16);
  v.z = e[4] | (e[5] << 16);
  v.w = e[6] | (e[7] << 16);
  return v;
}

// DoRA block hb: hpart[hb, i, j] = sum over columns [hb*512, +512) of x[i, k] * A[j, k]
// for i < M, j < r, with MFMA 16x16x32 (both operands in natural k order).
// Wave w covers 128 columns; the four wave partials are summed through LDS.
template <int MT>
__device__ __forceinline__ void dora_h_block(const SkinnyArgs& a, int hb, float* red) {
  constexpr int JT = kMaxFusedRank / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int jt_n = (a.r + 15) >> 4;
  const bool vec = a.x_vec != 0;
  const bool avec = ((reinterpret_cast<uintptr_t>(a.A) & 15u) == 0) && (a.K % 8) == 0;
  float4_t acc[MT][JT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) acc[mt][jt] = float4_t{0.f, 0.f, 0.f, 0.f};
  const int kbase = hb * kHCols + wave * 128;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int k = kbase + 32 * ks + 8 * kq;
    u32x4_t xa[MT], ab[JT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int i = 16 * mt + r16;
      xa[mt] = (i < a.M && k < a.K) ? load8(a.x + (size_t)i * a.K, k, a.K, vec) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) {
      const int j = 16 * jt + r16;
      ab[jt] = (jt < jt_n && j < a.r && k < a.K) ? load8(a.A + (size_t)j * a.K, k, a.K, avec)
                                                 : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
        if (jt < jt_n) acc[mt][jt] = mfma16x16x32(xa[mt], ab[jt], acc[mt][jt]);
  }
  // reduce the four waves: red[wave][mt][jt][e][lane]
  constexpr int per_wave = MT * JT * 4 * 64;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave * per_wave + ((mt * JT + jt) * 4 + e) * 64 + lane] = acc[mt][jt][e];
  __syncthreads();
  for (int idx = threadIdx.x; idx < per_wave; idx += blockDim.x) {
    const float v = red[idx] + red[per_wave + idx] + red[2 * per_wave + idx] + red[3 * per_wave + idx];
    const int ln = idx & 63;
    const int e = (idx >> 6) & 3;
    const int t = idx >> 8;
    const int jt = t % JT;
    const int mt = t / JT;
    const int i = 16 * mt + 4 * (ln >> 4) + e;
    const int j = 16 * jt + (ln & 15);
    if (i < a.M && j < a.r) store_dev(a.hpart + ((size_t)hb * a.M + i) * a.r + j, v);
  }
}

// Delta-form outlier correction for the block's column range, added to the
// lane's accumulators (see the file comment).
template <int BITS, int MT, int MB, bool PER_ROW>
__device__ __forceinline__ void outlier_delta(const SkinnyArgs& a, int n, bool row_ok, int kq, int k_lo, int k_hi,
                                              const uint32_t* qrow, const uint16_t* lrow, float4_t acc[MT]) {
  constexpr int NCB = 1 << BITS;
  float corr[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) corr[i] = 0.f;
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

template <int MT>
__device__ __forceinline__ void write_result(const SkinnyArgs& a, int split, int n, bool row_ok, int kq,
                                             const float4_t acc[MT]) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * mt + 4 * kq + e;
      if (i < a.M && row_ok) {
        float v = acc[mt][e];
        if (a.direct_out) {
          if (a.r > 0) {
            float ls = 0.f;
            const float* h = a.H + (size_t)i * a.r;
            const uint16_t* bb = a.B + (size_t)n * a.r;
            for (int j = 0; j < a.r; ++j) ls += h[j] * h2f(bb[j]);
            v = (v + a.scale * ls) * h2f(a.gamma[n]);
          }
          a.out[(size_t)i * a.N + n] = f2h_rn(v);
        } else {
          store_dev(a.partial + ((size_t)split * a.M + i) * a.N + n, v);
        }
      }
    }
  }
}


// Sum of n_terms device-scope loads p[0], p[stride], ... in index order; the loads
// are issued eight at a time so their latencies overlap.
__device__ __forceinline__ float sum_dev(const float* p, size_t stride, int n_terms) {
  float v = 0.f;
  for (int t0 = 0; t0 < n_terms; t0 += 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = load_dev(p + (size_t)min(t0 + u, n_terms - 1) * stride);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (t0 + u < n_terms) v += t[u];
  }
  return v;
}

// Epilogue for the row blocks rbs[0..count) (rb0 when rbs is null), run by the block that arrived last on
// each of them: y[i, n] = fp16_rn((sum_s partial[s, i, n] + scale * h[i, :] . B[n, :]) * gamma[n])
// with h = fp16(sum over DoRA blocks of hpart) (or the caller's H).  Splits and DoRA
// blocks are summed in index order, so the result does not depend on arrival order.
// lds: at least M * r free floats.
__device__ __forceinline__ void finish_rows(const SkinnyArgs& a, int rb0, const int* rbs, int count, float* lds) {
  // NaN rows when a hand-off on this workspace failed (this call or an earlier one): the
  // sticky error word of the counter area
  const bool poisoned = load_dev(a.sync + kSyncErrorWord) != 0u;
  const float* h = a.H;
  if (a.r > 0 && a.hpart != nullptr) {
    for (int idx = threadIdx.x; idx < a.M * a.r; idx += blockDim.x)
      lds[idx] = h2f(f2h_rn(sum_dev(a.hpart + idx, (size_t)a.M * a.r, a.h_blocks)));
    __syncthreads();
    h = lds;
  }
  const size_t plane = (size_t)a.M * a.N;
  const bool bvec = (a.r & 7) == 0 && (reinterpret_cast<uintptr_t>(a.B) & 15u) == 0;
  for (int t = threadIdx.x; t < count * a.M * kRowsPerBlock; t += blockDim.x) {
    const int k = t / (a.M * kRowsPerBlock);
    const int u = t - k * (a.M * kRowsPerBlock);
    const int i = u / kRowsPerBlock;
    const int n = (rbs ? rbs[k] : rb0) * kRowsPerBlock + (u - i * kRowsPerBlock);
    if (n >= a.N) continue;
    const size_t idx = (size_t)i * a.N + n;
    float v = sum_dev(a.partial + idx, plane, a.splits);
    if (a.r > 0) {
      float ls = 0.f;
      const float* hi = h + (size_t)i * a.r;
      const uint16_t* b = a.B + (size_t)n * a.r;
      if (bvec) {
        for (int j = 0; j < a.r; j += 8) {
          const u32x4_t bv = *reinterpret_cast<const u32x4_t*>(b + j);
          const uint32_t w[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            ls += hi[j + 2 * q] * h2f((uint16_t)(w[q] & 0xFFFFu));
            ls += hi[j + 2 * q + 1] * h2f((uint16_t)(w[q] >> 16));
          }
        }
      } else {
        for (int j = 0; j < a.r; ++j) ls += hi[j] * h2f(b[j]);
      }
      v = (v + a.scale * ls) * h2f(a.gamma[n]);
    }
    a.out[idx] = poisoned ? kHalfNaN : f2h_rn(v);
  }
}

// Product block: partials are written; count the arrival and finish the row block
// when this block is the last one.
__device__ __forceinline__ void arrive_product(const SkinnyArgs& a, int rb, float* lds) {
  __shared__ int s_last;
  fence_release();  // this block's partial stores are complete before it counts
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = atomicAdd(a.sync + rb, 1u);
    if (old >= (uint32_t)a.arrivals) raise_error(a.sync, kErrArrivals);  // counters not zero at entry
    s_last = old >= (uint32_t)(a.arrivals - 1);  // an overflowing block finishes too (with NaN rows)
  }
  __syncthreads();
  if (!s_last) return;
  fence_acquire();
  finish_rows(a, rb, nullptr, 1, lds);
  if (threadIdx.x == 0) atomicExch(a.sync + rb, 0u);  // ready for the next call
}

// DoRA block: hpart is written; count one arrival on every row block and finish,
// in one parallel pass, the row blocks for which this block is the last.
// One K split and the DoRA blocks already done (their arrivals fill the row block's count
// but one): nobody else touches the row block in this call, so the block applies the
// epilogue from its accumulators, without the partial round trip, and clears the count.
// Returns false (nothing done) when the DoRA blocks are still running.
template <int MT>
__device__ __forceinline__ bool finish_direct(const SkinnyArgs& a, int rb, int n, bool row_ok, int kq,
                                              const float4_t acc[MT], float* lds) {
  __shared__ int s_ready;
  __syncthreads();  // every wave is past its last use of the activation staging (reused below)
  if (threadIdx.x == 0)
    s_ready = __hip_atomic_load(a.sync + rb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.arrivals - 1);
  __syncthreads();
  if (!s_ready) return false;
  fence_acquire();
  const bool poisoned = load_dev(a.sync + kSyncErrorWord) != 0u;
  for (int idx = threadIdx.x; idx < a.M * a.r; idx += blockDim.x)
    lds[idx] = h2f(f2h_rn(sum_dev(a.hpart + idx, (size_t)a.M * a.r, a.h_blocks)));
  __syncthreads();
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = 16 * mt + 4 * kq + e;
      if (i < a.M && row_ok) {
        float ls = 0.f;
        const float* hi = lds + (size_t)i * a.r;
        const uint16_t* bb = a.B + (size_t)n * a.r;
        for (int j = 0; j < a.r; ++j) ls += hi[j] * h2f(bb[j]);
        a.out[(size_t)i * a.N + n] = poisoned ? kHalfNaN : f2h_rn((acc[mt][e] + a.scale * ls) * h2f(a.gamma[n]));
      }
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(a.sync + rb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

__device__ __forceinline__ void arrive_dora(const SkinnyArgs& a, float* lds) {
  __shared__ int s_list[256];
  __shared__ int s_n;
  fence_release();
  for (int base = 0; base < a.row_blocks; base += blockDim.x) {
    if (threadIdx.x == 0) s_n = 0;
    __syncthreads();
    const int rb = base + (int)threadIdx.x;
    if (rb < a.row_blocks) {
      const uint32_t old = atomicAdd(a.sync + rb, 1u);
      if (old >= (uint32_t)a.arrivals) raise_error(a.sync, kErrArrivals);  // counters not zero at entry
      if (old >= (uint32_t)(a.arrivals - 1)) s_list[atomicAdd(&s_n, 1)] = rb;
    }
    __syncthreads();
    const int cnt = s_n;
    if (cnt > 0) {
      fence_acquire();
      finish_rows(a, 0, s_list, cnt, lds);
      __syncthreads();
      if ((int)threadIdx.x < cnt) atomicExch(a.sync + s_list[threadIdx.x], 0u);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- generic path

template <int BITS>
struct LaneState {
  LutPlanes<BITS> pl0, pl1;
  int split_col;  // first column served by pl1 (TWO_LUT)
};

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
__global__ __launch_bounds__(256) void skinny_generic_kernel(const SkinnyArgs a) {
  constexpr int WIN = CodeGeom<BITS>::kWin;
  constexpr int SLAB = 4 * WIN;
  constexpr int NCB = 1 << BITS;
  extern __shared__ __align__(16) uint16_t xs[];

  int bid = blockIdx.x;
  if (bid < a.h_blocks) {
    dora_h_block<MT>(a, bid, reinterpret_cast<float*>(xs));
    if (a.sync) {
      __syncthreads();
      arrive_dora(a, reinterpret_cast<float*>(xs));
    }
    return;
  }
  bid -= a.h_blocks;
  const int split = bid / a.row_blocks;
  const int rb = bid - split * a.row_blocks;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int kq = lane >> 4;
  const int n = rb * kRowsPerBlock + wave * 16 + r;
  const bool row_ok = n < a.N;
  const int nc = row_ok ? n : (a.N - 1);
  const uint32_t* qrow = a.q + (size_t)nc * a.wpr;
  const uint16_t* lrow = a.lut + (size_t)nc * a.ng * NCB;

  const int total_slabs = (a.K + SLAB - 1) / SLAB;
  const int t_begin = split * a.slabs_per_split;
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

  if (a.has_csr)
    outlier_delta<BITS, MT, MB, PER_ROW>(a, n, row_ok, kq, t_begin * SLAB, min(a.K, t_end * SLAB), qrow, lrow, acc);
  write_result<MT>(a, split, n, row_ok, kq, acc);
  if (a.sync) {
    __syncthreads();  // the activation tile is free from here on
    arrive_product(a, rb, reinterpret_cast<float*>(xs));
  }
}

// -------------------------------------------------------------- 4-bit fast path

// Activation staging in two phases (fast path, 16-byte aligned rows, K % 8 == 0):
// xstage_load issues the loads of the first kXR 8-column units per thread (unit
// indices clamped, so the loads are unconditional), xstage_store writes them to LDS
// in order P and stages any remaining units directly.
constexpr int kXR = 4;
struct XStage {
  u32x4_t v[kXR];
};

__device__ __forceinline__ void xstage_load(const SkinnyArgs& a, XStage& xr, int c_a, int ncols) {
  const int upr = ncols >> 3;
  const int total = a.M * upr;
#pragma unroll
  for (int k = 0; k < kXR; ++k) {
    const int u = min((int)threadIdx.x + k * (int)blockDim.x, max(total - 1, 0));
    const int i = u / upr;
    const int col = min(c_a + ((u - i * upr) << 3), a.K - 8);
    xr.v[k] = *reinterpret_cast<const u32x4_t*>(a.x + (size_t)i * a.K + col);
  }
}

__device__ __forceinline__ void xstage_store(const SkinnyArgs& a, const XStage& xr, uint16_t* xs, int c_a,
                                             int ncols) {
  const int upr = ncols >> 3;
  const int total = a.M * upr;
#pragma unroll
  for (int k = 0; k < kXR; ++k) {
    const int u = (int)threadIdx.x + k * (int)blockDim.x;
    if (u < total) {
      const int i = u / upr;
      const int c8 = u - i * upr;
      const bool inside = c_a + (c8 << 3) < a.K;  // K % 8 == 0: a unit is all inside or all outside
      const u32x4_t v = inside ? permute_p(xr.v[k]) : u32x4_t{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4_t*>(xs + i * a.xstride + (c8 << 3)) = v;
    }
  }
  for (int u = (int)threadIdx.x + kXR * (int)blockDim.x; u < total; u += blockDim.x) {
    const int i = u / upr;
    const int c8 = u - i * upr;
    const int col = c_a + (c8 << 3);
    const u32x4_t v = col < a.K ? permute_p(*reinterpret_cast<const u32x4_t*>(a.x + (size_t)i * a.K + col))
                                : u32x4_t{0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4_t*>(xs + i * a.xstride + (c8 << 3)) = v;
  }
}

constexpr int kEB = 4;  // CSR entries per lane fetched ahead for the next chunk

// One prefetched slab: the lane's code window and its LUT quarters.
template <int NGS>
struct Stage4 {
  u32x4_t codes;
  u32x2_t lq[NGS];  // quarter kq (entries 4kq..4kq+3) of the row's LUT for each group in the slab
};

// Unconditional load of slab t (callers clamp t to a valid slab; windows past the
// row end read the row's last window -- those columns meet zero activations).
template <bool PER_ROW, int NGS>
__device__ __forceinline__ void stage4_load(Stage4<NGS>& s, const SkinnyArgs& a, const uint32_t* qrow,
                                            const uint16_t* lrow, int kq, int t) {
  const int wi = min(t * 16 + kq * 4, a.wpr - 4);
  s.codes = *reinterpret_cast<const u32x4_t*>(qrow + wi);
  if constexpr (!PER_ROW) {
    const int g0 = (NGS > 1) ? t * NGS : group_of(t * 128, a.g_magic);
#pragma unroll
    for (int j = 0; j < NGS; ++j) {
      const int g = min(g0 + j, a.ng - 1);
      s.lq[j] = *reinterpret_cast<const u32x2_t*>(lrow + g * 16 + 4 * kq);
    }
  }
}

template <int MT, int S>
__device__ __forceinline__ void fast_block(const u32x4_t& codes, const LutPlanes<4>& t, const uint16_t* const xp[MT],
                                           float4_t acc[MT]) {
  const uint32_t w = S == 0 ? codes.x : S == 1 ? codes.y : S == 2 ? codes.z : codes.w;
  uint32_t b[4];
  dequant_word4(w, t, b);
  u32x4_t bv;
  bv.x = b[0]; bv.y = b[1]; bv.z = b[2]; bv.w = b[3];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const u32x4_t av = *reinterpret_cast<const u32x4_t*>(xp[mt] + 8 * S);
    acc[mt] = mfma16x16x32(av, bv, acc[mt]);
  }
}

// Wave-private LDS tiles of one outlier chunk (4 slabs x 16 rows):
//   ctile: code windows, [slab][row][window ^ ((row >> 2) & 3)] x 16 B
//   ltile: LUT byte planes, [slab][group][lo|hi][row] x 16 B (the per-row LUT: [lo|hi][row])
// The code windows and LUT quarters are loaded with the four lanes of a row adjacent
// (lane 4 * row + window: coalesced 64-byte and 32-byte row pieces) and exchanged
// through these tiles to the MFMA lane order (lane row + 16 * window); the window
// swizzle keeps both the stores and the reads free of LDS bank conflicts.
template <int NGS>
struct ChunkTiles {
  uint32_t* ctile;
  uint32_t* ltile;
};

// Dword offset of code window `w` of tile row `row` in slab `sl` of a ctile.
__device__ __forceinline__ int ctile_word(int sl, int row, int w) { return ((sl * 16 + row) * 4 + (w ^ ((row >> 2) & 3))) * 4; }

// s was loaded by lane (rl, kl) = (lane / 4, lane % 4); the MFMA lane is (r, kq).
template <bool PER_ROW, int NGS, int MT>
__device__ __forceinline__ void stage4_consume(const Stage4<NGS>& s, int slab_in_chunk, LutPlanes<4>& pl,
                                               const ChunkTiles<NGS>& tl, int r, int kq, int rl, int kl,
                                               const uint16_t* const xp[MT], float4_t acc[MT]) {
  *reinterpret_cast<u32x4_t*>(tl.ctile + ctile_word(slab_in_chunk, rl, kl)) = s.codes;
  if constexpr (!PER_ROW) {
    // split the loaded LUT quarters into planes; the row's lanes exchange them
#pragma unroll
    for (int j = 0; j < NGS; ++j) {
      uint32_t* base = tl.ltile + ((slab_in_chunk * NGS + j) * 2 * 16 + rl) * 4 + kl;
      base[0] = perm_b32(s.lq[j].y, s.lq[j].x, 0x06040200u);
      base[16 * 4] = perm_b32(s.lq[j].y, s.lq[j].x, 0x07050301u);
    }
    const int jown = (NGS == 1) ? 0 : (NGS == 2 ? (kq >> 1) : kq);
    const uint32_t* own = tl.ltile + ((slab_in_chunk * NGS + jown) * 2 * 16 + r) * 4;
    const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(own);
    const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(own + 16 * 4);
    pl.lo[0] = lo.x; pl.lo[1] = lo.y; pl.lo[2] = lo.z; pl.lo[3] = lo.w;
    pl.hi[0] = hi.x; pl.hi[1] = hi.y; pl.hi[2] = hi.z; pl.hi[3] = hi.w;
  }
  const u32x4_t codes = *reinterpret_cast<const u32x4_t*>(tl.ctile + ctile_word(slab_in_chunk, r, kq));
  fast_block<MT, 0>(codes, pl, xp, acc);
  fast_block<MT, 1>(codes, pl, xp, acc);
  fast_block<MT, 2>(codes, pl, xp, acc);
  fast_block<MT, 3>(codes, pl, xp, acc);
}

// CSR entries of one chunk for one lane: entries e0 + kq + 4j, j < kEB.  The
// column and value registers are only combined when used, so the loads stay in
// flight while the next chunk streams.
struct ChunkEntries {
  int e0, e1;          // the row's entry range for the chunk
  uint16_t col[kEB];   // column inside the chunk (kept narrow: widened only where used)
  uint8_t val[kEB];    // e5m2 byte
};

// Loads are unconditional (clamped to entry e1-1, or 0 for an empty range) so that the
// wait counters stay in program order; cols/vals point at any readable buffer when the
// layer has no outliers (every range is then empty).
__device__ __forceinline__ void entries_load(ChunkEntries& E, const uint16_t* cols, const uint8_t* vals, int kq,
                                             int e0, int e1) {
  E.e0 = e0;
  E.e1 = e1;
#pragma unroll
  for (int j = 0; j < kEB; ++j) {
    const int e = min(e0 + kq + 4 * j, max(e1 - 1, 0));
    E.col[j] = cols[e];
    E.val[j] = vals[e];
  }
}

// Delta corrections of one entry (chunk-local column cl, e5m2 value vb) from the LDS tiles;
// x_col0 is the first column of the staged activation segment.
template <int MB, bool PER_ROW, int NGS>
__device__ __forceinline__ void entry_delta(const SkinnyArgs& a, const ChunkTiles<NGS>& tl, const uint16_t* xs,
                                            int r, int c, int cl, uint32_t vb, int k_lo, int k_hi, int x_col0,
                                            float corr[MB]) {
  const int gcol = c * 512 + cl;
  if (gcol < k_lo || gcol >= k_hi) return;
  const int sl = cl >> 7;
  const uint32_t word = tl.ctile[ctile_word(sl, r, (cl >> 5) & 3) + ((cl >> 3) & 3)];
  const uint32_t code = (word >> (4 * (cl & 7))) & 15u;
  const int gi = PER_ROW ? 0 : (NGS == 1 ? 0 : (NGS == 2 ? ((cl >> 6) & 1) : ((cl >> 5) & 3)));
  const unsigned char* planes =
      reinterpret_cast<const unsigned char*>(tl.ltile + ((PER_ROW ? 0 : (sl * NGS + gi) * 2 * 16) + r) * 4);
  const uint32_t lutv = (uint32_t)planes[code] | ((uint32_t)planes[16 * 16 + code] << 8);
  const float d = h2f((uint16_t)(vb << 8)) - h2f((uint16_t)lutv);
  const int xc = gcol - x_col0;  // column inside the staged activation segment
  const int xi = (xc & ~7) + p_slot(xc & 7);
#pragma unroll
  for (int i = 0; i < MB; ++i)
    if (i < a.M) corr[i] += d * h2f(xs[i * a.xstride + xi]);
}

template <int MB, bool PER_ROW, int NGS>
__device__ __forceinline__ void chunk_outliers(const SkinnyArgs& a, const ChunkEntries& E, const ChunkTiles<NGS>& tl,
                                               const uint16_t* xs, int r, int kq, int c, int k_lo, int k_hi,
                                               int x_col0, float corr[MB]) {
#pragma unroll
  for (int j = 0; j < kEB; ++j) {
    const bool have = E.e0 + kq + 4 * j < E.e1;
    if (__ballot(have)) {
      if (have) entry_delta<MB, PER_ROW, NGS>(a, tl, xs, r, c, (int)E.col[j], (uint32_t)E.val[j], k_lo, k_hi, x_col0, corr);
    }
  }
  // rows with more than 4 * kEB entries in the chunk: fetch the rest directly
  for (int e = E.e0 + kq + 4 * kEB; e < E.e1; e += 4)
    entry_delta<MB, PER_ROW, NGS>(a, tl, xs, r, c, (int)a.cols[e], (uint32_t)a.vals[e], k_lo, k_hi, x_col0, corr);
}

constexpr int kOT = 17;  // chunk offsets per row kept in LDS (a block spans at most 16 chunks)

template <int MT, int MB, bool PER_ROW, int NGS>
__global__ __launch_bounds__(256, (NGS >= 4 || MT > 1 || (MB > 4 && NGS > 1)) ? 2 : 3) void skinny4_kernel(const SkinnyArgs a) {
  constexpr int SLAB = 128;
  extern __shared__ __align__(16) uint16_t smem[];
  // LDS: [x staging: M * xstride halves][64 B zeros]
  //      [per wave: ctile 4 KB | ltile (PER_ROW ? 512 B : NGS * 2 KB) | otile 16 x kOT ints]
  uint16_t* xs = smem;

  int bid = blockIdx.x;
  if (bid < a.h_blocks) {
    dora_h_block<MT>(a, bid, reinterpret_cast<float*>(smem));
    if (a.sync) {
      __syncthreads();
      arrive_dora(a, reinterpret_cast<float*>(smem));
    }
    return;
  }
  bid -= a.h_blocks;
  const int split = bid / a.row_blocks;
  const int rb = bid - split * a.row_blocks;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int kq = lane >> 4;
  const int n = rb * kRowsPerBlock + wave * 16 + r;
  const bool row_ok = n < a.N;
  const int nc = row_ok ? n : (a.N - 1);
  const uint16_t* lrow = a.lut + (size_t)nc * a.ng * 16;
  // loads: lane (rl, kl) takes window kl of tile row rl (the row's four lanes adjacent)
  const int rl = lane >> 2;
  const int kl = lane & 3;
  const int nload = min(rb * kRowsPerBlock + wave * 16 + rl, a.N - 1);
  const uint32_t* qrow_ld = a.q + (size_t)nload * a.wpr;
  const uint16_t* lrow_ld = a.lut + (size_t)nload * a.ng * 16;

  const size_t xbytes = ((size_t)a.M * a.xstride * 2 + 15) & ~(size_t)15;
  uint16_t* zpad = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(smem) + xbytes);
  constexpr int kLtWords = PER_ROW ? 16 * 8 : 16 * 4 * NGS * 8;
  constexpr int kWaveWords = 16 * 4 * 4 * 4 + kLtWords + 16 * kOT;
  uint32_t* wave_lds = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(zpad) + 64) + wave * kWaveWords;
  ChunkTiles<NGS> tl{wave_lds, wave_lds + 16 * 4 * 4 * 4};
  int* otile = reinterpret_cast<int*>(wave_lds + 16 * 4 * 4 * 4 + kLtWords) + r * kOT;

  const int total_slabs = (a.K + SLAB - 1) / SLAB;
  const int t_begin = split * a.slabs_per_split;  // any slab: the first chunk may be partial
  const int t_end = min(total_slabs, t_begin + a.slabs_per_split);
  const int k_lo = t_begin * SLAB;
  const int k_hi = min(a.K, t_end * SLAB);
  const int c_begin = t_begin >> 2;
  const int c_end = (t_end + 3) >> 2;
  const int nchunks = c_end - c_begin;  // <= kOT - 1 (the planner bounds the split)
  const bool single = a.seg_slabs >= a.slabs_per_split;
  int seg0 = t_begin;
  int seg_end = single ? t_end : min(t_end, (c_begin + a.seg_slabs / 4) * 4);  // segments end on chunks

  float4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = float4_t{0.f, 0.f, 0.f, 0.f};
  float corr[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) corr[i] = 0.f;
  const bool csr = a.has_csr != 0 && t_begin < t_end;

  // Prologue.  Small loads first (CSR offsets, activations, the per-row LUT), then the
  // code prefetch, then the LDS stores: the stores wait only for the small loads, so
  // the first code windows are in flight while the block stages its tiles.
  int offv[(kOT + 3) / 4];
  {  // without outliers the loads read word 0 of the codes and the values are dropped
    const int32_t* offr = csr ? a.offsets + (size_t)nc * (a.nch + 1) + c_begin : reinterpret_cast<const int32_t*>(a.q);
#pragma unroll
    for (int jj = 0; jj < (kOT + 3) / 4; ++jj) {
      const int v = offr[csr ? min(kq + 4 * jj, nchunks) : 0];
      offv[jj] = csr ? v : 0;
    }
  }
  XStage xr;
  const bool xfast = a.x_vec != 0;
  if (xfast) xstage_load(a, xr, seg0 * SLAB, (seg_end - seg0) * SLAB);
  LutRaw<4> raw;
  if constexpr (PER_ROW) lut_load<4>(raw, lrow);
  Stage4<NGS> st[4];  // slot s holds slab 4c + s of chunk c
  const int t_last = max(t_end - 1, t_begin);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    stage4_load<PER_ROW, NGS>(st[j], a, qrow_ld, lrow_ld, kl, min(max(4 * c_begin + j, t_begin), t_last));
#pragma unroll
  for (int jj = 0; jj < (kOT + 3) / 4; ++jj) otile[min(kq + 4 * jj, nchunks)] = offv[jj];
  if (xfast)
    xstage_store(a, xr, xs, seg0 * SLAB, (seg_end - seg0) * SLAB);
  else
    stage_x(a, xs, seg0 * SLAB, (seg_end - seg0) * SLAB);
  LutPlanes<4> pl;
  if constexpr (PER_ROW) {
    pl = lut_planes<4>(raw);
    if (kq == 0) {
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        tl.ltile[r * 4 + p] = pl.lo[p];
        tl.ltile[(16 + r) * 4 + p] = pl.hi[p];
      }
    }
  }
  if (threadIdx.x < 16) reinterpret_cast<uint32_t*>(zpad)[threadIdx.x] = 0u;
  __syncthreads();
  // A row with entries in the range reads only entries below its last offset; a row
  // without any reads word 0 of its codes instead (the CSR arrays may then be empty).
  const bool any = otile[nchunks] > otile[0];
  const uint16_t* colp = any ? a.cols : reinterpret_cast<const uint16_t*>(a.q);
  const uint8_t* valp = any ? a.vals : reinterpret_cast<const uint8_t*>(a.q);
  ChunkEntries ea, eb;
  entries_load(ea, colp, valp, kq, otile[0], otile[min(1, nchunks)]);

  // One chunk: the entries of the next chunk are requested, the chunk's slabs consumed
  // (each slot re-requested for the next chunk), then the chunk's outliers applied.
  // The last chunk requests nothing, so no load is left in flight at the end.
  auto chunk = [&](int c, const ChunkEntries& cur, ChunkEntries& nxt, auto more) __attribute__((always_inline)) {
    constexpr bool kMore = decltype(more)::value;
    const int lc = c - c_begin;
    if constexpr (kMore)
      entries_load(nxt, colp, valp, kq, otile[min(lc + 1, nchunks)], otile[min(lc + 2, nchunks)]);
    const uint16_t* xp[MT];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int t = 4 * c + s;
      if (t >= t_begin && t < t_end) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          xp[mt] = (16 * mt + r < a.M) ? xs + (16 * mt + r) * a.xstride + (t - seg0) * SLAB + kq * 32 : zpad;
        stage4_consume<PER_ROW, NGS, MT>(st[s], s, pl, tl, r, kq, rl, kl, xp, acc);
      }
      if constexpr (kMore) stage4_load<PER_ROW, NGS>(st[s], a, qrow_ld, lrow_ld, kl, min(t + 4, t_last));
    }
    if (csr && row_ok) chunk_outliers<MB, PER_ROW, NGS>(a, cur, tl, xs, r, kq, c, k_lo, k_hi, seg0 * SLAB, corr);
  };
  using More = std::integral_constant<bool, true>;
  using Last = std::integral_constant<bool, false>;

  if (single) {
    int c = c_begin;
    for (; c + 2 < c_end; c += 2) {  // two chunks per trip: the entry registers alternate
      chunk(c, ea, eb, More{});
      chunk(c + 1, eb, ea, More{});
    }
    if (c + 1 < c_end) {
      chunk(c, ea, eb, More{});
      chunk(c + 1, eb, ea, Last{});
    } else {
      chunk(c, ea, eb, Last{});
    }
  } else {
    auto restage = [&](int c) __attribute__((always_inline)) {
      if (4 * c >= seg_end) {  // next activation segment (whole chunks)
        __syncthreads();
        seg0 = 4 * c;
        seg_end = min(t_end, seg0 + a.seg_slabs);
        stage_x(a, xs, seg0 * SLAB, (seg_end - seg0) * SLAB);
        __syncthreads();
      }
    };
    int c = c_begin;
    for (; c + 2 < c_end; c += 2) {
      restage(c);
      chunk(c, ea, eb, More{});
      restage(c + 1);
      chunk(c + 1, eb, ea, More{});
    }
    if (c + 1 < c_end) {
      restage(c);
      chunk(c, ea, eb, More{});
      restage(c + 1);
      chunk(c + 1, eb, ea, Last{});
    } else {
      restage(c);
      chunk(c, ea, eb, Last{});
    }
  }

  if (a.has_csr) {
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
  if (a.sync && a.splits == 1 && a.h_blocks > 0 &&
      finish_direct<MT>(a, rb, n, row_ok, kq, acc, reinterpret_cast<float*>(smem)))
    return;
  write_result<MT>(a, split, n, row_ok, kq, acc);
  if (a.sync) {
    __syncthreads();
    arrive_product(a, rb, reinterpret_cast<float*>(smem));
  }
}

// ------------------------------------------------------------------- dispatch

template <int MT, int MB>
hipError_t launch_fast(const SkinnyArgs& a, int ngs, dim3 grid, size_t lds, hipStream_t stream) {
  if (a.G <= 0 || a.ng == 1)
    hipLaunchKernelGGL((skinny4_kernel<MT, MB, true, 1>), grid, dim3(256), lds, stream, a);
  else if (ngs == 1)
    hipLaunchKernelGGL((skinny4_kernel<MT, MB, false, 1>), grid, dim3(256), lds, stream, a);
  else if (ngs == 2)
    hipLaunchKernelGGL((skinny4_kernel<MT, MB, false, 2>), grid, dim3(256), lds, stream, a);
  else
    hipLaunchKernelGGL((skinny4_kernel<MT, MB, false, 4>), grid, dim3(256), lds, stream, a);
  return hipGetLastError();
}

template <int BITS, int MT, int MB>
hipError_t launch_generic(const SkinnyArgs& a, int mode, dim3 grid, size_t lds, hipStream_t stream) {
  switch (mode) {
    case 0: hipLaunchKernelGGL((skinny_generic_kernel<BITS, MT, MB, true, false>), grid, dim3(256), lds, stream, a); break;
    case 1: hipLaunchKernelGGL((skinny_generic_kernel<BITS, MT, MB, false, false>), grid, dim3(256), lds, stream, a); break;
    default: hipLaunchKernelGGL((skinny_generic_kernel<BITS, MT, MB, false, true>), grid, dim3(256), lds, stream, a); break;
  }
  return hipGetLastError();
}

template <int MT, int MB>
hipError_t launch_m(const SkinnyArgs& a, int bits, int mode, bool fast, int ngs, dim3 grid, size_t lds,
                    hipStream_t stream) {
  switch (bits) {
    case 1: return launch_generic<1, MT, MB>(a, mode, grid, lds, stream);
    case 2: return launch_generic<2, MT, MB>(a, mode, grid, lds, stream);
    case 3: return launch_generic<3, MT, MB>(a, mode, grid, lds, stream);
    default:
      if (!fast) return launch_generic<4, MT, MB>(a, mode, grid, lds, stream);
      return launch_fast<MT, MB>(a, ngs, grid, lds, stream);
  }
}

int window_cols(int bits) { return bits == 4 ? 32 : bits == 3 ? 40 : bits == 2 ? 64 : 128; }

}  // namespace

int slab_cols(int bits) { return 4 * window_cols(bits); }
int skinny_max_m() { return kMaxM; }
int skinny_max_fused_rank() { return kMaxFusedRank; }

SplitPlan plan_skinny(const Layer& L, int M, int cu_count, size_t workspace_bytes, int fused_rank) {
  SplitPlan p{};
  const int slab = slab_cols(L.bits);
  const int total = std::max(1, (L.K + slab - 1) / slab);
  const int row_blocks = (L.N + kRowsPerBlock - 1) / kRowsPerBlock;
  const int target = 2 * std::max(1, cu_count);  // two blocks per CU (measured flat from 2 to 6)
  int splits = std::max(1, (target + row_blocks - 1) / row_blocks);
  splits = std::min(splits, std::min(total, kMaxSplits));
  const size_t per_split = (size_t)M * (size_t)L.N * sizeof(float);
  const size_t hbytes = fused_rank > 0 ? (size_t)((L.K + kHCols - 1) / kHCols) * M * fused_rank * sizeof(float) : 0;
  const bool need_partials = fused_rank > 0;  // the fused DoRA path always finishes in finalize
  while (splits > 1 && (size_t)splits * per_split + hbytes > workspace_bytes) --splits;
  int sps = (total + splits - 1) / splits;
  if (L.bits == 4) {
    // fast path: whole outlier chunks per block (a partial first chunk is supported but
    // measured slower), at most 16 chunks (their offsets are staged in LDS)
    sps = std::min(std::max(kPF, (sps + kPF - 1) / kPF * kPF), kMaxFastSlabs / kPF * kPF);
  } else {
    const int spc = std::max(1, L.chunk / slab);
    if (sps >= spc) sps = (sps + spc - 1) / spc * spc;
  }
  splits = (total + sps - 1) / sps;
  p.splits = splits;
  p.slabs_per_split = sps;
  // activation staging: for M >= 8 a smaller budget (more restaging, less LDS per block)
  // keeps two blocks per CU resident (measured: gate_proj at M = 8 41.0 -> 32.7 us)
  const int x_budget = M >= 8 ? kXStageBytes / 2 : kXStageBytes;
  const int seg_cols_max = x_budget / (2 * std::max(1, M));
  int seg = std::max(1, std::min(sps, (seg_cols_max - 8) / slab));
  if (L.bits == 4 && seg < sps) seg = std::max(kPF, seg / kPF * kPF);
  p.seg_slabs = seg;
  p.workspace_bytes = (splits > 1 || need_partials) ? (size_t)splits * per_split + hbytes : 0;
  return p;
}

hipError_t launch_skinny(const Layer& L, const Dora& D, const uint16_t* x, uint16_t* out, int M,
                         const SplitPlan& plan, float* workspace, uint32_t* sync, hipStream_t stream) {
  SkinnyArgs a{};
  a.q = L.q;
  a.lut = L.lut;
  a.x = x;
  a.out = out;
  a.offsets = L.offsets;
  a.cols = L.cols;
  a.vals = L.vals;
  a.has_csr = (L.offsets && L.cols && L.vals) ? 1 : 0;
  a.B = D.B;
  a.H = D.H;
  a.A = D.A;
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
  a.row_blocks = (L.N + kRowsPerBlock - 1) / kRowsPerBlock;
  const bool fused_h = D.r > 0 && D.H == nullptr && D.A != nullptr;
  a.h_blocks = fused_h ? (L.K + kHCols - 1) / kHCols : 0;
  a.direct_out = (plan.splits == 1 && !fused_h) ? 1 : 0;
  const bool inline_fin = !a.direct_out && sync != nullptr && a.row_blocks <= kMaxSyncRowBlocks;
  a.sync = inline_fin ? sync : nullptr;
  a.arrivals = plan.splits + a.h_blocks;
  a.partial = workspace;
  a.hpart = fused_h ? workspace + (size_t)plan.splits * M * L.N : nullptr;
  a.x_vec = ((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (L.K % 8) == 0) ? 1 : 0;
  const bool per_row = L.group_size <= 0 || L.ng == 1;
  const int mode = per_row ? 0 : ((L.group_size % window_cols(L.bits)) == 0 ? 1 : 2);
  // 4-bit fast path: a 128-column slab holds 1, 2 or 4 whole groups (or the per-row LUT)
  const bool fast = L.bits == 4 && L.K > 0 &&
                    (per_row || L.group_size == 32 || L.group_size == 64 || L.group_size % 128 == 0);
  const int ngs = (!per_row && L.group_size < 128) ? 128 / L.group_size : 1;
  size_t lds = (size_t)M * a.xstride * sizeof(uint16_t);
  lds = (lds + 15) & ~(size_t)15;
  if (fast) lds += 64 + (size_t)kWaves * (16 * 4 * 64 + (per_row ? 16 * 32 : 16 * 4 * ngs * 32) + 16 * kOT * 4);
  const int mt = M > 16 ? 2 : 1;
  const size_t hred = fused_h ? (size_t)4 * mt * (kMaxFusedRank / 16) * 4 * 64 * sizeof(float) : 0;
  lds = std::max(lds, hred);
  if (inline_fin && D.r > 0) lds = std::max(lds, (size_t)M * D.r * sizeof(float));  // rounded H
  const dim3 grid(a.h_blocks + a.row_blocks * plan.splits);
  hipError_t err;
  if (M == 1)
    err = launch_m<1, 1>(a, L.bits, mode, fast, ngs, grid, lds, stream);
  else if (M <= 4)
    err = launch_m<1, 4>(a, L.bits, mode, fast, ngs, grid, lds, stream);
  else if (M <= 16)
    err = launch_m<1, 16>(a, L.bits, mode, fast, ngs, grid, lds, stream);
  else
    err = launch_m<2, 32>(a, L.bits, mode, fast, ngs, grid, lds, stream);
  if (err != hipSuccess) return err;
  if (!a.direct_out && !inline_fin)
    return launch_finalize(workspace, plan.splits, M, L.N, D, a.hpart, a.h_blocks, out, stream);
  return hipSuccess;
}

}  // namespace wlq
