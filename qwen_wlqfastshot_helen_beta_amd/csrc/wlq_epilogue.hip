// Output epilogues.
//
// * splitk_sum_kernel: y = fp16_rn(sum_s partial[s]) for the prefill GEMM's split-K partials, which
//   already carry the DoRA term and gamma; summed in split order (deterministic).  Reference
//   behaviour: reduce_split_k_dora_kernel (csrc/gemv_kernel.cu:322-353), generalized to M rows.
// * dora_epilogue_kernel: the in-place pass of the reference's M >= 16 path,
//   out = fp16_rn((fp16 out + scale * H.B) * gamma) (csrc/gemm_kernel.cu:447-473).
#include <algorithm>

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

// H[M, r] = fp32(fp16(X . A^T)) in K chunks: block (16-row tile of X, chunk ks, group z of 16 NT
// ranks) computes the 16 x 16 NT part of its chunk with MFMA 16x16x32 (both operands in natural k
// order); its 4 waves take the chunk's 32-column steps in turn, UNR steps of loads in flight per
// wave, and their sums meet in LDS in wave order.  One chunk: the block rounds and writes H;
// several: it writes its fp32 part and lora_h_sum_kernel adds the parts in chunk order and rounds.
constexpr int kHWaves = 4;
template <int NT, int UNR>
__global__ __launch_bounds__(64 * kHWaves) void lora_h_part_kernel(const uint16_t* __restrict__ X,
                                                                   const uint16_t* __restrict__ A, int M, int K,
                                                                   int r, int kch, float* __restrict__ out, int vec) {
  __shared__ float red[kHWaves][NT][4][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int m0 = blockIdx.x * 16;
  const int ks = blockIdx.y;
  const int i = m0 + r16;
  const int j0 = 16 * NT * blockIdx.z;
  const int jt_n = min(NT, (r - j0 + 15) >> 4);
  const int kb = ks * kch;
  const int ke = min(K, kb + kch);
  float4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
  const uint16_t* xr = X + (size_t)min(i, M - 1) * K;
  for (int k0 = kb + 32 * wave; k0 < ke; k0 += 32 * kHWaves * UNR) {
    u32x4_t xa[UNR], ab[UNR][NT];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int k = k0 + 32 * kHWaves * u + 8 * kq;
      const bool kin = k < ke;
      xa[u] = (i < M && kin) ? load8z(xr, k, ke, vec != 0) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int j = j0 + 16 * t + r16;
        ab[u][t] = (t < jt_n && j < r && kin) ? load8z(A + (size_t)j * K, k, ke, vec != 0) : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (t < jt_n) acc[t] = mfma16x16x32(xa[u], ab[u][t], acc[t]);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][t][e][lane] = acc[t][e];
  __syncthreads();
  const bool final_h = gridDim.y == 1;
  float* part = out + (size_t)ks * M * r;
  for (int idx = threadIdx.x; idx < NT * 256; idx += 64 * kHWaves) {
    const int t = idx >> 8;
    const int e = (idx >> 6) & 3;
    const int ln = idx & 63;
    const int ii = m0 + 4 * (ln >> 4) + e;
    const int j = j0 + 16 * t + (ln & 15);
    if (t < jt_n && ii < M && j < r) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kHWaves; ++w) v += red[w][t][e][ln];
      if (final_h)
        out[(size_t)ii * r + j] = h2f(f2h_rn(v));
      else
        part[(size_t)ii * r + j] = v;
    }
  }
}

// H[i] = fp32(fp16(sum of the chunk parts in chunk order)); the loads of 8 parts are issued
// before their adds.
__global__ __launch_bounds__(256) void lora_h_sum_kernel(const float* __restrict__ part, int chunks, size_t total,
                                                         float* __restrict__ H) {
  for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
    float v = 0.f;
    for (int c0 = 0; c0 < chunks; c0 += 8) {
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = part[(size_t)min(c0 + u, chunks - 1) * total + idx];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (c0 + u < chunks) v += t[u];
    }
    H[idx] = h2f(f2h_rn(v));
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

// K chunks of lora_h_part_kernel: enough blocks for about eight per CU, chunks of at least 512
// columns.
int lora_h_chunks(int M, int K, int cu_count) {
  const int tiles = std::max(1, (M + 15) / 16);
  const int target = 8 * std::max(1, cu_count);
  const int most = std::max(1, (K + 511) / 512);
  return std::max(1, std::min(most, (target + tiles - 1) / tiles));
}

size_t lora_h_part_bytes(int M, int K, int r, int cu_count) {
  const int ks = lora_h_chunks(M, K, cu_count);
  return ks > 1 ? (size_t)ks * (size_t)M * (size_t)r * sizeof(float) : 0;
}

hipError_t launch_lora_h(const uint16_t* X, const uint16_t* A, int M, int K, int r, float* H, float* part,
                         size_t part_bytes, int cu_count, hipStream_t stream) {
  if (M <= 0 || r <= 0) return hipSuccess;
  const int vec = ((reinterpret_cast<uintptr_t>(X) & 15u) == 0 && (reinterpret_cast<uintptr_t>(A) & 15u) == 0 &&
                   (K % 8) == 0) ? 1 : 0;
  int ks = lora_h_chunks(M, K, cu_count);
  const size_t per = (size_t)M * (size_t)r * sizeof(float);
  if (part == nullptr || (size_t)ks * per > part_bytes) ks = 1;  // no room for parts: one chunk
  const int kch = ks > 1 ? ((K + ks - 1) / ks + 31) / 32 * 32 : std::max(K, 1);
  ks = std::max(1, (K + kch - 1) / kch);
  float* dst = ks > 1 ? part : H;
  if (r <= 16) {
    hipLaunchKernelGGL((lora_h_part_kernel<1, 8>), dim3((M + 15) / 16, ks, 1), dim3(64 * kHWaves), 0, stream, X, A,
                       M, K, r, kch, dst, vec);
  } else if (r <= 32) {
    hipLaunchKernelGGL((lora_h_part_kernel<2, 4>), dim3((M + 15) / 16, ks, 1), dim3(64 * kHWaves), 0, stream, X, A,
                       M, K, r, kch, dst, vec);
  } else {
    hipLaunchKernelGGL((lora_h_part_kernel<4, 4>), dim3((M + 15) / 16, ks, (r + 63) / 64), dim3(64 * kHWaves), 0,
                       stream, X, A, M, K, r, kch, dst, vec);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || ks == 1) return e;
  const size_t total = (size_t)M * (size_t)r;
  hipLaunchKernelGGL(lora_h_sum_kernel, dim3(grid_for(total)), dim3(256), 0, stream, part, ks, total, H);
  return hipGetLastError();
}

hipError_t launch_dora_epilogue(uint16_t* out, int M, int N, const Dora& D, hipStream_t stream) {
  if (M <= 0 || N <= 0 || D.r <= 0) return hipSuccess;
  const dim3 grid(grid_for((size_t)M * N));
  hipLaunchKernelGGL(dora_epilogue_kernel, grid, dim3(256), 0, stream, out, M, N, D);
  return hipGetLastError();
}

}  // namespace wlq
