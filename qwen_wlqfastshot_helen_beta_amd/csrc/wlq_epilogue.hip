// Output epilogues.
//
// * splitk_sum_kernel: y = fp16_rn(sum_s partial[s]) for the prefill GEMM's split-K partials, which
//   already carry the DoRA term and gamma; summed in split order (deterministic).  Reference
//   behaviour: reduce_split_k_dora_kernel (csrc/gemv_kernel.cu:322-353), generalized to M rows.
// * dora_epilogue_kernel: the in-place pass of the reference's M >= 16 path,
//   out = fp16_rn((fp16 out + scale * H.B) * gamma) (csrc/gemm_kernel.cu:447-473).
#include "wlq_device.h"
#include "wlq_internal.h"

namespace wlq {
namespace {

__device__ __forceinline__ float dora_dot(const Dora& D, int i, int n) {
  float ls = 0.f;
  const float* h = D.H + (size_t)i * D.r;
  const uint16_t* b = D.B + (size_t)n * D.r;
  for (int j = 0; j < D.r; ++j) ls += h[j] * h2f(b[j]);
  return ls;
}

// y = fp16_rn(sum_s partial[s]) over M*N values, partials summed in split order.
// VEC: four consecutive values per thread (16-byte partial loads, one 8-byte store).
template <bool VEC>
__global__ __launch_bounds__(256) void splitk_sum_kernel(const float* __restrict__ partial, int splits,
                                                         size_t total, uint16_t* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * 256;
  if (VEC) {
    const size_t quads = total / 4;
    const float4* p4 = reinterpret_cast<const float4*>(partial);
    for (size_t q = (size_t)blockIdx.x * 256 + threadIdx.x; q < quads; q += stride) {
      float4 v = p4[q];
      for (int s = 1; s < splits; ++s) {
        const float4 w = p4[(size_t)s * quads + q];
        v.x += w.x;
        v.y += w.y;
        v.z += w.z;
        v.w += w.w;
      }
      uint2 o;
      o.x = (uint32_t)f2h_rn(v.x) | ((uint32_t)f2h_rn(v.y) << 16);
      o.y = (uint32_t)f2h_rn(v.z) | ((uint32_t)f2h_rn(v.w) << 16);
      reinterpret_cast<uint2*>(out)[q] = o;
    }
  } else {
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += stride) {
      float v = partial[idx];
      for (int s = 1; s < splits; ++s) v += partial[(size_t)s * total + idx];
      out[idx] = f2h_rn(v);
    }
  }
}

__global__ __launch_bounds__(256) void dora_epilogue_kernel(uint16_t* __restrict__ out, int M, int N, const Dora D) {
  const size_t total = (size_t)M * N;
  for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
    const int i = (int)(idx / (size_t)N);
    const int n = (int)(idx - (size_t)i * N);
    const float v = (h2f(out[idx]) + D.scale * dora_dot(D, i, n)) * h2f(D.gamma[n]);
    out[idx] = f2h_rn(v);
  }
}

// One block per (256 outputs of row i): first the block rounds row i of H
// (summing the DoRA column-block partials when the decode kernel computed them),
// then every thread sums its split partials and applies the epilogue.
constexpr int kFinRank = 64;

__global__ __launch_bounds__(256) void finalize_kernel(const float* __restrict__ partial, int splits, int M, int N,
                                                       const Dora D, const float* __restrict__ hpart, int h_blocks,
                                                       uint16_t* __restrict__ out) {
  __shared__ float hs[kFinRank];
  const int i = blockIdx.y;
  const int n = blockIdx.x * 256 + threadIdx.x;
  const bool use_hs = hpart != nullptr && D.r > 0;
  if (use_hs) {
    for (int j = threadIdx.x; j < D.r; j += 256) {
      float s = 0.f;
      for (int hb = 0; hb < h_blocks; ++hb) s += hpart[((size_t)hb * M + i) * D.r + j];
      hs[j] = h2f(f2h_rn(s));
    }
    __syncthreads();
  }
  if (n >= N) return;
  const size_t plane = (size_t)M * N;
  const size_t idx = (size_t)i * N + n;
  float v = 0.f;
#pragma unroll 8
  for (int s = 0; s < splits; ++s) v += partial[(size_t)s * plane + idx];
  if (D.r > 0) {
    float ls = 0.f;
    const uint16_t* b = D.B + (size_t)n * D.r;
    const float* h = use_hs ? hs : D.H + (size_t)i * D.r;
    if ((D.r & 7) == 0 && (reinterpret_cast<uintptr_t>(b) & 15u) == 0) {
      for (int j = 0; j < D.r; j += 8) {  // 16-byte rows of B
        const u32x4_t bv = *reinterpret_cast<const u32x4_t*>(b + j);
        const uint32_t w[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          ls += h[j + 2 * q] * h2f((uint16_t)(w[q] & 0xFFFFu));
          ls += h[j + 2 * q + 1] * h2f((uint16_t)(w[q] >> 16));
        }
      }
    } else {
      for (int j = 0; j < D.r; ++j) ls += h[j] * h2f(b[j]);
    }
    v = (v + D.scale * ls) * h2f(D.gamma[n]);
  }
  out[idx] = f2h_rn(v);
}

__device__ __forceinline__ u32x4_t load8z(const uint16_t* row, int k, int K, bool vec) {
  if (vec && k + 8 <= K) return *reinterpret_cast<const u32x4_t*>(row + k);
  uint32_t e[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) e[j] = (k + j < K) ? (uint32_t)row[k + j] : 0u;
  u32x4_t v;
  v.x = e[0] | (e[1] << 16);
  v.y = e[2] | (e[3] << 16);
  v.z = e[4] | (e[5] << 16);
  v.w = e[6] | (e[7] << 16);
  return v;
}

// H = fp16(X . A^T) for large M: a block owns a 16x16 tile of H (16 rows of X,
// 16 columns of A^T); its 4 waves split K, each accumulating with MFMA
// 16x16x32 (both operands in natural k order), and the partials meet in LDS.
// H[M, r] = fp32(fp16(X . A^T)): one block per 16 x 16 tile of H, its 16 waves on K slices of a
// multiple of 256 columns; each wave issues the 16 loads of 256 columns before their 8 MFMAs, so
// a block needs about K / 4096 load round trips.  Wave sums are added through LDS in wave order.
constexpr int kHWaves = 16;
__global__ __launch_bounds__(1024) void lora_h_kernel(const uint16_t* __restrict__ X, const uint16_t* __restrict__ A,
                                                      int M, int K, int r, float* __restrict__ H, int vec) {
  __shared__ float red[kHWaves][4][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int m0 = blockIdx.x * 16;
  const int j0 = blockIdx.y * 16;
  const int i = m0 + r16;
  const int j = j0 + r16;
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  const uint16_t* xr = X + (size_t)min(i, M - 1) * K;
  const uint16_t* ar = A + (size_t)min(j, r - 1) * K;
  const int kslice = ((K + kHWaves - 1) / kHWaves + 255) / 256 * 256;
  const int kb = wave * kslice;
  const int ke = min(K, kb + kslice);
  for (int k0 = kb; k0 < ke; k0 += 256) {
    u32x4_t xa[8], ab[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int k = k0 + 32 * s + 8 * kq;
      xa[s] = (i < M && k < ke) ? load8z(xr, k, ke, vec != 0) : u32x4_t{0u, 0u, 0u, 0u};
      ab[s] = (j < r && k < ke) ? load8z(ar, k, ke, vec != 0) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = mfma16x16x32(xa[s], ab[s], acc);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) red[wave][e][lane] = acc[e];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kHWaves; ++w) v += red[w][e][lane];
      const int ii = m0 + 4 * kq + e;
      if (ii < M && j < r) H[(size_t)ii * r + j] = h2f(f2h_rn(v));
    }
  }
}

unsigned grid_for(size_t total) {
  const size_t blocks = (total + 255) / 256;
  return (unsigned)(blocks < 65536 ? (blocks ? blocks : 1) : 65536);
}

}  // namespace

hipError_t launch_splitk_sum(const float* partial, int splits, int M, int N, uint16_t* out, hipStream_t stream) {
  if (M <= 0 || N <= 0) return hipSuccess;
  const size_t total = (size_t)M * N;
  const bool vec = (total % 4 == 0) && ((reinterpret_cast<uintptr_t>(partial) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(out) & 7) == 0);
  if (vec)
    hipLaunchKernelGGL(splitk_sum_kernel<true>, dim3(grid_for(total / 4)), dim3(256), 0, stream, partial, splits,
                       total, out);
  else
    hipLaunchKernelGGL(splitk_sum_kernel<false>, dim3(grid_for(total)), dim3(256), 0, stream, partial, splits,
                       total, out);
  return hipGetLastError();
}

hipError_t launch_finalize(const float* partial, int splits, int M, int N, const Dora& D, const float* hpart,
                           int h_blocks, uint16_t* out, hipStream_t stream) {
  if (M <= 0 || N <= 0) return hipSuccess;
  const dim3 grid((N + 255) / 256, M);
  hipLaunchKernelGGL(finalize_kernel, grid, dim3(256), 0, stream, partial, splits, M, N, D, hpart, h_blocks, out);
  return hipGetLastError();
}

hipError_t launch_lora_h(const uint16_t* X, const uint16_t* A, int M, int K, int r, float* H, hipStream_t stream) {
  if (M <= 0 || r <= 0) return hipSuccess;
  const int vec = ((reinterpret_cast<uintptr_t>(X) & 15u) == 0 && (reinterpret_cast<uintptr_t>(A) & 15u) == 0 &&
                   (K % 8) == 0) ? 1 : 0;
  const dim3 grid((M + 15) / 16, (r + 15) / 16);
  hipLaunchKernelGGL(lora_h_kernel, grid, dim3(64 * kHWaves), 0, stream, X, A, M, K, r, H, vec);
  return hipGetLastError();
}

hipError_t launch_dora_epilogue(uint16_t* out, int M, int N, const Dora& D, hipStream_t stream) {
  if (M <= 0 || N <= 0 || D.r <= 0) return hipSuccess;
  const dim3 grid(grid_for((size_t)M * N));
  hipLaunchKernelGGL(dora_epilogue_kernel, grid, dim3(256), 0, stream, out, M, N, D);
  return hipGetLastError();
}

}  // namespace wlq
