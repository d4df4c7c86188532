// Output epilogues.
//
// * splitk_reduce_kernel: y[i, n] = fp16_rn((sum_s partial[s, i, n] + scale * H[i,:].B[n,:]) * gamma[n]),
//   the partials summed in split order (deterministic).  Reference behaviour:
//   reduce_split_k_dora_kernel (csrc/gemv_kernel.cu:322-353), generalized to M rows.
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

__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partial, int splits, int M,
                                                            int N, const Dora D, uint16_t* __restrict__ out) {
  const size_t total = (size_t)M * N;
  const size_t plane = total;
  for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (size_t)gridDim.x * 256) {
    const int i = (int)(idx / (size_t)N);
    const int n = (int)(idx - (size_t)i * N);
    float v = 0.f;
    for (int s = 0; s < splits; ++s) v += partial[(size_t)s * plane + idx];
    if (D.r > 0) v = (v + D.scale * dora_dot(D, i, n)) * h2f(D.gamma[n]);
    out[idx] = f2h_rn(v);
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

unsigned grid_for(size_t total) {
  const size_t blocks = (total + 255) / 256;
  return (unsigned)(blocks < 65536 ? (blocks ? blocks : 1) : 65536);
}

}  // namespace

hipError_t launch_splitk_reduce(const float* partial, int splits, int M, int N, const Dora& D, uint16_t* out,
                                hipStream_t stream) {
  if (M <= 0 || N <= 0) return hipSuccess;
  const dim3 grid(grid_for((size_t)M * N));
  hipLaunchKernelGGL(splitk_reduce_kernel, grid, dim3(256), 0, stream, partial, splits, M, N, D, out);
  return hipGetLastError();
}

hipError_t launch_dora_epilogue(uint16_t* out, int M, int N, const Dora& D, hipStream_t stream) {
  if (M <= 0 || N <= 0 || D.r <= 0) return hipSuccess;
  const dim3 grid(grid_for((size_t)M * N));
  hipLaunchKernelGGL(dora_epilogue_kernel, grid, dim3(256), 0, stream, out, M, N, D);
  return hipGetLastError();
}

}  // namespace wlq
