// Bit-exact dequantization W[n, k] = lut[n, g(k), code(n, k)], then the CSR
// outliers overwrite W[n, c*chunk + col] = fp16 bits (e5m2 << 8).
//
// Reference behaviour: dequant_patch_metalog_kernel + launch_dequant_patch_metalog
// (csrc/gemm_kernel.cu:322-445, :475-503), served to Python as _C.dequant_w0
// (csrc/vllm_binding.cpp:421-453).  Used at load time for the DoRA magnitude
// calibration; the GEMM kernels never materialize W.
//
// One block per row.  Each thread expands whole code words; 4-bit words become
// one 16-byte store of 8 fp16.  After a block barrier the row's outliers are
// written over the LUT values (same-address stores from one workgroup are
// ordered by the barrier).
#include "wlq_device.h"
#include "wlq_internal.h"

namespace wlq {
namespace {

template <int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(const Layer L, uint16_t* __restrict__ W, int vec_ok) {
  constexpr int spw = CodeGeom<BITS>::kSpw;
  constexpr int NCB = 1 << BITS;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  const int n = blockIdx.x;
  const uint32_t* qrow = L.q + (size_t)n * L.wpr;
  const uint16_t* lrow = L.lut + (size_t)n * L.ng * NCB;
  uint16_t* wrow = W + (size_t)n * L.K;
  const int words = (L.K + spw - 1) / spw;
  for (int wi = threadIdx.x; wi < words; wi += blockDim.x) {
    const uint32_t w = qrow[wi];
    const int col0 = wi * spw;
    if (BITS == 4 && vec_ok && L.group_size <= 0 && col0 + 8 <= L.K) {
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = lrow[(w >> (4 * j)) & 15u];
      u32x4_t v;
      v.x = h[0] | (h[1] << 16);
      v.y = h[2] | (h[3] << 16);
      v.z = h[4] | (h[5] << 16);
      v.w = h[6] | (h[7] << 16);
      *reinterpret_cast<u32x4_t*>(wrow + col0) = v;
    } else {
#pragma unroll
      for (int j = 0; j < spw; ++j) {
        const int col = col0 + j;
        if (col < L.K) {
          const int g = L.group_size > 0 ? min(col / L.group_size, L.ng - 1) : 0;
          wrow[col] = lrow[g * NCB + ((w >> (BITS * j)) & mask)];
        }
      }
    }
  }
  if (L.offsets == nullptr || L.cols == nullptr || L.vals == nullptr) return;
  __syncthreads();
  const int32_t* offr = L.offsets + (size_t)n * (L.nch + 1);
  for (int c = 0; c < L.nch; ++c) {
    const int s0 = offr[c];
    const int s1 = offr[c + 1];
    for (int e = s0 + (int)threadIdx.x; e < s1; e += blockDim.x) {
      const int col = c * L.chunk + (int)L.cols[e];
      if (col < L.K) wrow[col] = (uint16_t)((uint32_t)L.vals[e] << 8);
    }
  }
}

}  // namespace

hipError_t launch_dequant(const Layer& L, uint16_t* W, hipStream_t stream) {
  if (L.N <= 0 || L.K <= 0) return hipSuccess;
  const int vec_ok = ((reinterpret_cast<uintptr_t>(W) & 15u) == 0 && (L.K % 8) == 0) ? 1 : 0;
  const dim3 grid(L.N);
  switch (L.bits) {
    case 1: hipLaunchKernelGGL(dequant_kernel<1>, grid, dim3(256), 0, stream, L, W, vec_ok); break;
    case 2: hipLaunchKernelGGL(dequant_kernel<2>, grid, dim3(256), 0, stream, L, W, vec_ok); break;
    case 3: hipLaunchKernelGGL(dequant_kernel<3>, grid, dim3(256), 0, stream, L, W, vec_ok); break;
    default: hipLaunchKernelGGL(dequant_kernel<4>, grid, dim3(256), 0, stream, L, W, vec_ok); break;
  }
  return hipGetLastError();
}

}  // namespace wlq
