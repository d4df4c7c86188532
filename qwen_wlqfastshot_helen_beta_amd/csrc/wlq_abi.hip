// extern "C" device entry points of libwlq_hip.so (declared in include/wlq_abi.h):
// argument validation, per-device launch planning and kernel dispatch.
//
// Unlike the reference launchers (csrc/gemv_kernel.cu:442-456 has no default
// case for unsupported widths; csrc/gemm_kernel.cu:573-575 only printf's), every
// invalid argument returns a status before anything is launched.  The CU count
// used for split planning is cached per device (the reference caches the first
// device's value for all devices, csrc/gemv_kernel.cu:355-363).
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "wlq_abi.h"
#include "wlq_internal.h"

namespace wlq {
void set_error(const char* fmt, ...);
int window_cols_for(int bits);
}  // namespace wlq

namespace wlq {

namespace {
// 0: not read yet, 1: hooks off, 2: hooks on (WLQ_TEST_HOOKS=1 at the first product)
std::atomic<int> g_hooks{0};

bool hooks_on() {
  int h = g_hooks.load(std::memory_order_relaxed);
  if (h == 0) {
    const char* e = std::getenv("WLQ_TEST_HOOKS");
    h = (e != nullptr && e[0] == '1') ? 2 : 1;
    g_hooks.store(h, std::memory_order_relaxed);
  }
  return h == 2;
}
}  // namespace

uint32_t spin_limit() {
  if (hooks_on()) {
    const char* e = std::getenv("WLQ_SPIN_LIMIT");
    if (e != nullptr && e[0] != 0) return (uint32_t)std::strtoul(e, nullptr, 10);
  }
  return kDefaultSpinLimit;
}

bool withhold_h() {
  if (!hooks_on()) return false;
  const char* e = std::getenv("WLQ_TEST_WITHHOLD_H");
  return e != nullptr && e[0] == '1';
}

bool force_prefill() {
  if (!hooks_on()) return false;
  const char* e = std::getenv("WLQ_TEST_FORCE_PREFILL");
  return e != nullptr && e[0] == '1';
}

}  // namespace wlq

namespace {

// Clears `words` 32-bit words (the counter area) with plain vector stores.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int words) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < words; i += gridDim.x * 256) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
// Prepared-layout products with more activation rows than this run the wide kernel
// (activations streamed through LDS) up to wide_max_m(); up to this many, the decode kernel.
constexpr int64_t kWideMinM = 8;
std::atomic<int> g_cu_count[kMaxDevices];

int cu_count_for(int device) {
  if (device < 0 || device >= kMaxDevices) return 256;
  int v = g_cu_count[device].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    cus = 256;
  }
  g_cu_count[device].store(cus, std::memory_order_relaxed);
  return cus;
}

int current_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    dev = 0;
  }
  return cu_count_for(dev);
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return WLQ_OK;
  wlq::set_error("%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return WLQ_ERR_HIP;
}

// Shared shape/format validation; fills the kernel-side layer description.
int make_layer(const int32_t* q_packed, const void* lut_c, int64_t N, int64_t K, int32_t bits, int64_t wpr_given,
               int32_t group_size, const int32_t* offs, const uint16_t* cols, const uint8_t* vals, const char* fn,
               wlq::Layer* L) {
  if (bits < 1 || bits > 4) {
    wlq::set_error("%s: unsupported bits=%d (supported: 1, 2, 3, 4)", fn, (int)bits);
    return WLQ_ERR_UNSUPPORTED;
  }
  if (N < 0 || K < 0 || N > 0x3fffffff || K > 0x3fffffff) {
    wlq::set_error("%s: bad shape N=%lld K=%lld", fn, (long long)N, (long long)K);
    return WLQ_ERR_BAD_SHAPE;
  }
  const int64_t wpr = wlq_words_per_row(K, bits);
  if (wpr_given >= 0 && wpr_given != wpr) {
    wlq::set_error("%s: words_per_row=%lld does not match K=%lld, bits=%d (expected %lld)", fn,
                   (long long)wpr_given, (long long)K, (int)bits, (long long)wpr);
    return WLQ_ERR_BAD_SHAPE;
  }
  if (N * wpr > ((int64_t)1 << 40)) {
    wlq::set_error("%s: packed weight too large", fn);
    return WLQ_ERR_BAD_SHAPE;
  }
  int ng = 1;
  int gs = group_size;
  if (gs < 0) {
    wlq::set_error("%s: group_size must be >= 0, got %d", fn, (int)gs);
    return WLQ_ERR_UNSUPPORTED;
  }
  if (gs > 0 && gs >= K) gs = 0;  // a single group is the per-row layout
  if (gs > 0) {
    const int win = wlq::window_cols_for(bits);
    if (gs % 32 != 0 || gs < win || gs >= 4096 || K >= (1 << 20)) {
      wlq::set_error("%s: unsupported group_size=%d for bits=%d, K=%lld (need a multiple of 32, >= %d, < 4096, "
                     "and K < 2^20)",
                     fn, (int)group_size, (int)bits, (long long)K, win);
      return WLQ_ERR_UNSUPPORTED;
    }
    ng = (int)((K + gs - 1) / gs);
  }
  if (N > 0 && (lut_c == nullptr || (wpr > 0 && q_packed == nullptr))) {
    wlq::set_error("%s: q_packed and lut_c must be non-null", fn);
    return WLQ_ERR_NULL_POINTER;
  }
  // 16-byte code/LUT loads need aligned bases (row strides keep the alignment).
  if ((reinterpret_cast<uintptr_t>(q_packed) & 15u) != 0 || (reinterpret_cast<uintptr_t>(lut_c) & 15u) != 0) {
    wlq::set_error("%s: q_packed and lut_c must be 16-byte aligned", fn);
    return WLQ_ERR_BAD_SHAPE;
  }
  const bool csr = offs != nullptr && cols != nullptr && vals != nullptr;
  L->q = reinterpret_cast<const uint32_t*>(q_packed);
  L->lut = reinterpret_cast<const uint16_t*>(lut_c);
  L->offsets = csr ? offs : nullptr;
  L->cols = csr ? cols : nullptr;
  L->vals = csr ? vals : nullptr;
  L->N = (int)N;
  L->K = (int)K;
  L->bits = bits;
  L->wpr = (int)wpr;
  L->group_size = gs;
  L->ng = ng;
  L->chunk = wlq_chunk_width(bits);
  L->nch = (int)((K + L->chunk - 1) / L->chunk);
  return WLQ_OK;
}

wlq::Dora make_dora(const void* lora_B, const float* lora_H, const void* dora_gamma, const void* lora_A,
                    float scale, int32_t r) {
  wlq::Dora D{};
  if (lora_B != nullptr && dora_gamma != nullptr && r > 0 && (lora_H != nullptr || lora_A != nullptr)) {
    D.B = reinterpret_cast<const uint16_t*>(lora_B);
    D.H = lora_H;
    D.A = lora_H != nullptr ? nullptr : reinterpret_cast<const uint16_t*>(lora_A);
    D.gamma = reinterpret_cast<const uint16_t*>(dora_gamma);
    D.scale = scale;
    D.r = r;
  }
  return D;
}

size_t round_up(size_t v) { return (v + 255) & ~(size_t)255; }

// lists: the layer's prepared patch lists (the GEMM reads its outliers from them), or nullptr
int run_product(const wlq::Layer& L, wlq::Dora D, const void* X, void* out, int64_t M, void* workspace,
                size_t workspace_bytes, hipStream_t stream, const char* fn,
                const wlq::PatchLists* lists = nullptr) {
  if (M < 0 || M > 0x7fffffff / 4) {
    wlq::set_error("%s: bad M=%lld", fn, (long long)M);
    return WLQ_ERR_BAD_SHAPE;
  }
  if (M == 0 || L.N == 0) return WLQ_OK;
  if (X == nullptr || out == nullptr) {
    wlq::set_error("%s: activation and output pointers must be non-null", fn);
    return WLQ_ERR_NULL_POINTER;
  }
  const int cus = current_cu_count();
  size_t ws = workspace != nullptr ? workspace_bytes : 0;
  char* wbase = reinterpret_cast<char*>(workspace);
  uint32_t* sync = nullptr;  // arrival counters at the front of the workspace
  if (ws >= wlq::kSyncBytes) {
    sync = reinterpret_cast<uint32_t*>(wbase);
    wbase += wlq::kSyncBytes;
    ws -= wlq::kSyncBytes;
  } else {
    ws = 0;
  }
  const uint16_t* x = reinterpret_cast<const uint16_t*>(X);
  uint16_t* y = reinterpret_cast<uint16_t*>(out);
  const bool skinny = M <= wlq::skinny_max_m();
  const bool need_h = D.r > 0 && D.H == nullptr;
  const bool fused_h = need_h && skinny && D.r <= wlq::skinny_max_fused_rank();
  if (need_h && !fused_h) {  // H = fp16(X A^T) computed first into the front of the workspace
    const size_t hb = round_up((size_t)M * D.r * sizeof(float));
    if (ws < hb) {
      wlq::set_error("%s: computing H from lora_A needs a workspace of at least %zu bytes", fn, hb);
      return WLQ_ERR_CAPACITY;
    }
    float* H = reinterpret_cast<float*>(wbase);
    // its K-chunk parts use the bytes after H (the product's part of the workspace, not yet in use)
    float* part = ws > hb ? reinterpret_cast<float*>(wbase + hb) : nullptr;
    int st = hip_status(wlq::launch_lora_h(x, D.A, (int)M, L.K, D.r, H, part, ws - hb, cus, stream), fn);
    if (st != WLQ_OK) return st;
    D.H = H;
    D.A = nullptr;
    wbase += hb;
    ws -= hb;
  }
  float* w = reinterpret_cast<float*>(wbase);
  if (skinny) {
    const wlq::SplitPlan p = wlq::plan_skinny(L, (int)M, cus, ws, fused_h ? D.r : 0);
    if (p.workspace_bytes > ws) {
      wlq::set_error("%s: the fused DoRA path needs a workspace of at least %zu bytes (got %zu)", fn,
                     p.workspace_bytes, ws);
      return WLQ_ERR_CAPACITY;
    }
    return hip_status(wlq::launch_skinny(L, D, x, y, (int)M, p, w, sync, stream), fn);
  }
  const bool use_lists = lists != nullptr && lists->nnz > 0 && L.offsets != nullptr;
  const wlq::SplitPlan p = wlq::plan_gemm(L, (int)M, cus, ws, use_lists);
  return hip_status(wlq::launch_gemm(L, D, x, y, (int)M, p, w, stream, lists), fn);
}

// wlq_gemm_prepared with a workspace of the caller's (strict = false: a stream-kernel plan
// whose workspace does not fit falls back to the row-layout kernels, which adapt their
// splits) or the library's scratch (strict = true: such a call is refused instead).
int gemm_prepared_impl(const void* X, const int32_t* q_packed, const void* lut_c, const void* prepared,
                       size_t prepared_bytes, void* out, int64_t M, int64_t N, int64_t K, int32_t bits,
                       int64_t words_per_row, int32_t group_size, const int32_t* chunk_offsets,
                       const uint16_t* chunk_cols, const uint8_t* chunk_vals, int64_t nnz, const float* lora_H,
                       const void* lora_B, const void* dora_gamma, const void* lora_A, float lora_scale, int32_t r,
                       void* workspace, size_t workspace_bytes, hipStream_t stream, const char* fn, bool strict) {
  wlq::Layer L{};
  int st = make_layer(q_packed, lut_c, N, K, bits, words_per_row, group_size, chunk_offsets, chunk_cols, chunk_vals,
                      fn, &L);
  if (st != WLQ_OK) return st;
  const wlq::Dora D = make_dora(lora_B, lora_H, dora_gamma, lora_A, lora_scale, r);
  const bool wide = M > kWideMinM && M <= wlq::wide_max_m();
  const bool prefill = M >= wlq::prefill_min_m();
  if (prepared != nullptr && M >= 1 && (M <= wlq::stream_max_m() || wide || prefill) && L.N > 0 && X != nullptr &&
      out != nullptr && wlq::prepared_supported(L.N, L.K, L.bits, L.group_size) && nnz >= 0 &&
      (L.offsets != nullptr || nnz == 0)) {
    const wlq::PreparedLayout lay = wlq::prepared_layout(L.N, L.K, L.group_size, nnz);
    const size_t need = lay.bytes;
    if (prepared_bytes < need) {
      wlq::set_error("%s: the prepared buffer holds %zu bytes, the layer needs %zu (nnz=%lld)", fn, prepared_bytes,
                     need, (long long)nnz);
      return WLQ_ERR_CAPACITY;
    }
    const bool fused_h = D.r > 0 && D.H == nullptr;
    const char* pbase = reinterpret_cast<const char*>(prepared);
    const wlq::PatchLists lists{reinterpret_cast<const uint32_t*>(pbase + lay.codes_off),
                                reinterpret_cast<const uint32_t*>(pbase + lay.planes_off),
                                reinterpret_cast<const uint32_t*>(pbase + lay.wpidx_off),
                                reinterpret_cast<const uint32_t*>(pbase + lay.wpatch_off), nnz, lay.T, lay.S, lay.ng};
    // the kernel stages B rows with 16-byte loads (r % 8 == 0) and x / lora_A rows likewise
    const bool dora_ok = D.r == 0 || (D.r % 8 == 0 && D.r <= wlq::stream_max_rank() &&
                                      (reinterpret_cast<uintptr_t>(D.B) & 15u) == 0);
    const bool aligned = (reinterpret_cast<uintptr_t>(X) & 15u) == 0 && (reinterpret_cast<uintptr_t>(prepared) & 255u) == 0 &&
                         (!fused_h || (reinterpret_cast<uintptr_t>(D.A) & 15u) == 0) && dora_ok;
    const size_t ws = workspace != nullptr ? workspace_bytes : 0;
    if (prefill) {
      const wlq::PrefillPlan p = wlq::plan_prefill(L.N, L.K, (int)M, L.group_size, current_cu_count(), D.r,
                                                   fused_h ? D.r : 0, L.chunk);
      const bool need_sync = p.splits > 1 || fused_h;
      const bool ws_ok = !need_sync || ws >= wlq::kSyncBytes + p.workspace_bytes;
      const bool runs = p.ok && aligned && (p.preferred || wlq::force_prefill());
      if (runs && !ws_ok && strict) {
        wlq::set_error("%s: M=%lld N=%lld K=%lld needs %zu bytes of scratch, more than the %zu bytes it holds", fn,
                       (long long)M, (long long)N, (long long)K, wlq::kSyncBytes + p.workspace_bytes, ws);
        return WLQ_ERR_CAPACITY;
      }
      if (runs && ws_ok) {
        char* wbase = reinterpret_cast<char*>(workspace);
        uint32_t* sync = need_sync ? reinterpret_cast<uint32_t*>(wbase) : nullptr;
        float* w = need_sync ? reinterpret_cast<float*>(wbase + wlq::kSyncBytes) : nullptr;
        return hip_status(wlq::launch_prefill(L, prepared, nnz, D, reinterpret_cast<const uint16_t*>(X),
                                              reinterpret_cast<uint16_t*>(out), (int)M, p, w, sync, stream),
                          fn);
      }
      return run_product(L, D, X, out, M, workspace, workspace_bytes, stream, fn, &lists);
    }
    if (wide) {
      const bool csr = L.offsets != nullptr && nnz > 0;
      const wlq::WidePlan p =
          wlq::plan_wide(L.N, L.K, (int)M, current_cu_count(), D.r, fused_h ? D.r : 0, L.chunk, csr);
      const bool need_sync = p.splits > 1 || fused_h;
      const bool ws_ok = !need_sync || ws >= wlq::kSyncBytes + p.workspace_bytes;
      const bool runs = p.ok && aligned;
      if (runs && !ws_ok && strict) {
        wlq::set_error("%s: M=%lld N=%lld K=%lld needs %zu bytes of scratch, more than the %zu bytes it holds", fn,
                       (long long)M, (long long)N, (long long)K, wlq::kSyncBytes + p.workspace_bytes, ws);
        return WLQ_ERR_CAPACITY;
      }
      if (runs && ws_ok) {
        char* wbase = reinterpret_cast<char*>(workspace);
        uint32_t* sync = need_sync ? reinterpret_cast<uint32_t*>(wbase) : nullptr;
        float* w = need_sync ? reinterpret_cast<float*>(wbase + wlq::kSyncBytes) : nullptr;
        return hip_status(wlq::launch_wide(L, prepared, nnz, D, reinterpret_cast<const uint16_t*>(X),
                                           reinterpret_cast<uint16_t*>(out), (int)M, p, w, sync, stream),
                          fn);
      }
      return run_product(L, D, X, out, M, workspace, workspace_bytes, stream, fn, &lists);
    }
    const wlq::StreamPlan p =
        wlq::plan_stream(L.N, L.K, (int)M, current_cu_count(), fused_h ? D.r : 0, L.chunk);
    const bool need_sync = p.splits > 1 || fused_h;
    const bool ws_ok = !need_sync || ws >= wlq::kSyncBytes + p.workspace_bytes;
    const bool runs = p.ok && aligned && (!fused_h || D.r <= wlq::stream_max_rank());
    if (runs && !ws_ok && strict) {
      wlq::set_error("%s: M=%lld N=%lld K=%lld needs %zu bytes of scratch, more than the %zu bytes it holds", fn,
                     (long long)M, (long long)N, (long long)K, wlq::kSyncBytes + p.workspace_bytes, ws);
      return WLQ_ERR_CAPACITY;
    }
    if (runs && ws_ok) {
      char* wbase = reinterpret_cast<char*>(workspace);
      uint32_t* sync = need_sync ? reinterpret_cast<uint32_t*>(wbase) : nullptr;
      float* w = need_sync ? reinterpret_cast<float*>(wbase + wlq::kSyncBytes) : nullptr;
      return hip_status(wlq::launch_stream(L, prepared, nnz, D, reinterpret_cast<const uint16_t*>(X),
                                           reinterpret_cast<uint16_t*>(out), (int)M, p, w, sync, stream),
                        fn);
    }
  }
  return run_product(L, D, X, out, M, workspace, workspace_bytes, stream, fn);
}

// ------------------------------------------------------------ no-allocation scratch
// Device memory of wlq_gemm_prepared_noalloc: one array per GPU (each device that loads
// the library holds its own copy until the process ends), in the same layout as a
// caller's workspace: the 16 KiB counter area, then split partials and DoRA H sums.
// On the host, `scratch` only names the symbol; its device address comes from
// hipGetSymbolAddress, once per device with that device current, and only that address
// is passed to kernels and fills.
constexpr size_t kScratchBytes = (size_t)16 << 20;  // 16 MiB
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The current device's scratch address; the first call on a device looks it up and
// clears the counter area on `stream` (the array is zero at load; the clear also holds
// when the library is loaded into a process that ran other code on the device).  Under
// graph capture the clear is recorded instead, and no clear is needed: the array is
// still as the loader left it, zero.
int scratch_for_current_device(hipStream_t stream, void** out_ptr) {
  int dev = 0;
  int st = hip_status(hipGetDevice(&dev), "wlq_gemm_prepared_noalloc");
  if (st != WLQ_OK) return st;
  if (dev < 0 || dev >= kMaxDevices) {
    wlq::set_error("wlq_gemm_prepared_noalloc: device %d is beyond the %d the library serves", dev, kMaxDevices);
    return WLQ_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    st = hip_status(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "wlq_gemm_prepared_noalloc: hipGetSymbolAddress");
    if (st != WLQ_OK) return st;
    if (ptr == nullptr) {
      wlq::set_error("wlq_gemm_prepared_noalloc: hipGetSymbolAddress returned a null scratch address");
      return WLQ_ERR_HIP;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
      (void)hipGetLastError();
      cs = hipStreamCaptureStatusNone;
    }
    if (cs == hipStreamCaptureStatusNone) {
      hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)(wlq::kSyncWords + 255) / 256), dim3(256), 0, stream,
                         reinterpret_cast<uint32_t*>(ptr), wlq::kSyncWords);
      st = hip_status(hipGetLastError(), "wlq_gemm_prepared_noalloc: clearing the scratch counters");
      if (st != WLQ_OK) return st;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out_ptr = g_scratch_ptr[dev];
  return WLQ_OK;
}

}  // namespace

extern "C" {

size_t wlq_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t bits, int32_t r, int32_t device) {
  if (bits < 1 || bits > 4 || M <= 0 || N <= 0 || K < 0) return 0;
  wlq::Layer L{};
  L.N = (int)N;
  L.K = (int)K;
  L.bits = bits;
  L.wpr = (int)wlq_words_per_row(K, bits);
  L.chunk = wlq_chunk_width(bits);
  L.nch = (int)((K + L.chunk - 1) / L.chunk);
  // sized as if outliers are present (the GEMM's prepared outlier entries); never dereferenced
  L.offsets = reinterpret_cast<const int32_t*>(&L);
  const int cus = device >= 0 ? cu_count_for(device) : current_cu_count();
  const size_t unlimited = ~(size_t)0;
  const bool skinny = M <= wlq::skinny_max_m();
  const bool fused = skinny && r > 0 && r <= wlq::skinny_max_fused_rank();
  const size_t hb = (r > 0 && !fused) ? round_up((size_t)M * r * sizeof(float)) : 0;
  const wlq::SplitPlan p = skinny ? wlq::plan_skinny(L, (int)M, cus, unlimited, fused ? r : 0)
                                  : wlq::plan_gemm(L, (int)M, cus, unlimited);
  const size_t hparts = hb > 0 ? wlq::lora_h_part_bytes((int)M, (int)K, r, cus) : 0;
  size_t need = hb + std::max(p.workspace_bytes, hparts);
  if (M <= wlq::stream_max_m() && (bits == 4 || bits == 3)) {  // the prepared-layout kernel may serve the call
    const wlq::StreamPlan sp = wlq::plan_stream((int)N, (int)K, (int)M, cus,
                                                r > 0 && r <= wlq::stream_max_rank() ? r : 0, L.chunk);
    need = std::max(need, sp.workspace_bytes + 256);
  }
  if (M > kWideMinM && M <= wlq::wide_max_m() && (bits == 4 || bits == 3)) {  // or the wide kernel
    const int rr = r > 0 && r <= wlq::stream_max_rank() ? r : 0;
    const wlq::WidePlan wp = wlq::plan_wide((int)N, (int)K, (int)M, cus, rr, rr, L.chunk, true);
    need = std::max(need, wp.workspace_bytes + 256);
  }
  if (M >= wlq::prefill_min_m() && (bits == 4 || bits == 3)) {  // or the prefill kernel
    const int rr = r > 0 && r <= wlq::stream_max_rank() ? r : 0;
    const wlq::PrefillPlan pp = wlq::plan_prefill((int)N, (int)K, (int)M, 0, cus, rr, rr, L.chunk);
    if (pp.ok) need = std::max(need, pp.workspace_bytes + 256);
  }
  return need > 0 ? wlq::kSyncBytes + need : 0;
}

size_t wlq_prepared_bytes(int64_t N, int64_t K, int32_t bits, int32_t group_size, int64_t nnz) {
  if (N <= 0 || K <= 0 || N > 0x3fffffff || K > 0x3fffffff || nnz < 0 || group_size < 0) return 0;
  const int gs = (group_size > 0 && group_size >= K) ? 0 : group_size;
  if (!wlq::prepared_supported((int)N, (int)K, bits, gs)) return 0;
  return wlq::prepared_layout((int)N, (int)K, gs, nnz).bytes;
}

int wlq_prepare(const int32_t* q_packed, const void* lut_c, int64_t N, int64_t K, int32_t bits, int32_t group_size,
                const int32_t* chunk_offsets, const uint16_t* chunk_cols, const uint8_t* chunk_vals, int64_t nnz,
                void* prepared, size_t prepared_bytes, hipStream_t stream) {
  wlq::Layer L{};
  int st = make_layer(q_packed, lut_c, N, K, bits, -1, group_size, chunk_offsets, chunk_cols, chunk_vals,
                      "wlq_prepare", &L);
  if (st != WLQ_OK) return st;
  if (nnz < 0 || (L.offsets == nullptr && nnz != 0)) {
    wlq::set_error("wlq_prepare: nnz=%lld does not match the outlier arrays", (long long)nnz);
    return WLQ_ERR_BAD_SHAPE;
  }
  if (!wlq::prepared_supported(L.N, L.K, L.bits, L.group_size)) {
    wlq::set_error("wlq_prepare: no prepared layout for bits=%d, group_size=%d, K=%lld (needs 4- or 3-bit, a per-row LUT "
                   "or a group size multiple of 32, K %% 8 == 0, K < 65536)",
                   (int)bits, (int)group_size, (long long)K);
    return WLQ_ERR_UNSUPPORTED;
  }
  const size_t need = wlq::prepared_layout(L.N, L.K, L.group_size, nnz).bytes;
  if (prepared == nullptr || prepared_bytes < need) {
    wlq::set_error("wlq_prepare: the prepared buffer needs %zu bytes (got %zu)", need, prepared_bytes);
    return prepared == nullptr ? WLQ_ERR_NULL_POINTER : WLQ_ERR_CAPACITY;
  }
  if ((reinterpret_cast<uintptr_t>(prepared) & 255u) != 0) {
    wlq::set_error("wlq_prepare: the prepared buffer must be 256-byte aligned");
    return WLQ_ERR_BAD_SHAPE;
  }
  return hip_status(wlq::launch_prepare(L, nnz, prepared, stream), "wlq_prepare");
}

int wlq_gemv(const int32_t* q_packed, const void* lut_c, const void* x, void* out, const int32_t* chunk_offsets,
             const uint16_t* chunk_cols, const uint8_t* chunk_vals, const void* lora_B, const float* lora_h,
             const void* dora_gamma, const void* lora_A, float lora_scale, int32_t r, int64_t N, int64_t K,
             int32_t bits, int32_t group_size, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  wlq::Layer L{};
  int st = make_layer(q_packed, lut_c, N, K, bits, -1, group_size, chunk_offsets, chunk_cols, chunk_vals,
                      "wlq_gemv", &L);
  if (st != WLQ_OK) return st;
  const wlq::Dora D = make_dora(lora_B, lora_h, dora_gamma, lora_A, lora_scale, r);
  return run_product(L, D, x, out, 1, workspace, workspace_bytes, stream, "wlq_gemv");
}

int wlq_gemm(const void* X, const int32_t* q_packed, const void* lut_c, void* out, int64_t M, int64_t N, int64_t K,
             int32_t bits, int64_t words_per_row, int32_t group_size, const int32_t* chunk_offsets,
             const uint16_t* chunk_cols, const uint8_t* chunk_vals, const float* lora_H, const void* lora_B,
             const void* dora_gamma, const void* lora_A, float lora_scale, int32_t r, void* workspace,
             size_t workspace_bytes, hipStream_t stream) {
  wlq::Layer L{};
  int st = make_layer(q_packed, lut_c, N, K, bits, words_per_row, group_size, chunk_offsets, chunk_cols, chunk_vals,
                      "wlq_gemm", &L);
  if (st != WLQ_OK) return st;
  const wlq::Dora D = make_dora(lora_B, lora_H, dora_gamma, lora_A, lora_scale, r);
  return run_product(L, D, X, out, M, workspace, workspace_bytes, stream, "wlq_gemm");
}

int wlq_gemm_prepared(const void* X, const int32_t* q_packed, const void* lut_c, const void* prepared,
                      size_t prepared_bytes, void* out, int64_t M, int64_t N, int64_t K, int32_t bits,
                      int64_t words_per_row, int32_t group_size, const int32_t* chunk_offsets,
                      const uint16_t* chunk_cols, const uint8_t* chunk_vals, int64_t nnz, const float* lora_H,
                      const void* lora_B, const void* dora_gamma, const void* lora_A, float lora_scale, int32_t r,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return gemm_prepared_impl(X, q_packed, lut_c, prepared, prepared_bytes, out, M, N, K, bits, words_per_row,
                            group_size, chunk_offsets, chunk_cols, chunk_vals, nnz, lora_H, lora_B, dora_gamma, lora_A,
                            lora_scale, r, workspace, workspace_bytes, stream, "wlq_gemm_prepared", false);
}

int wlq_gemm_prepared_noalloc(const void* X, const int32_t* q_packed, const void* lut_c, const void* prepared,
                              size_t prepared_bytes, void* out, int64_t M, int64_t N, int64_t K, int32_t bits,
                              int64_t words_per_row, int32_t group_size, const int32_t* chunk_offsets,
                              const uint16_t* chunk_cols, const uint8_t* chunk_vals, int64_t nnz,
                              const float* lora_H, const void* lora_B, const void* dora_gamma, const void* lora_A,
                              float lora_scale, int32_t r, hipStream_t stream) {
  void* ws = nullptr;
  const int st = scratch_for_current_device(stream, &ws);
  if (st != WLQ_OK) return st;
  return gemm_prepared_impl(X, q_packed, lut_c, prepared, prepared_bytes, out, M, N, K, bits, words_per_row,
                            group_size, chunk_offsets, chunk_cols, chunk_vals, nnz, lora_H, lora_B, dora_gamma, lora_A,
                            lora_scale, r, ws, kScratchBytes, stream, "wlq_gemm_prepared_noalloc", true);
}

int wlq_workspace_status(const void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (workspace == nullptr || workspace_bytes < wlq::kSyncBytes) return WLQ_OK;
  int st = hip_status(hipStreamSynchronize(stream), "wlq_workspace_status");
  if (st != WLQ_OK) return st;
  uint32_t err = 0;
  st = hip_status(hipMemcpy(&err, reinterpret_cast<const uint32_t*>(workspace) + wlq::kSyncErrorWord, sizeof(err),
                            hipMemcpyDeviceToHost),
                  "wlq_workspace_status");
  if (st != WLQ_OK) return st;
  if (err == 0) return WLQ_OK;
  wlq::set_error("wlq_workspace_status: hand-off failures on this workspace (error word 0x%x:%s%s); the rows concerned "
                 "and every later call's rows were written as NaN; clear it with wlq_workspace_reset",
                 err, (err & wlq::kErrHTimeout) ? " a wait for the DoRA H ran out of polls;" : "",
                 (err & wlq::kErrArrivals) ? " a counter exceeded one call's arrivals (not zero at entry: unordered "
                                             "calls on one workspace, or never zero-filled);" : "");
  return WLQ_ERR_SYNC;
}

int wlq_workspace_reset(void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (workspace == nullptr) {
    wlq::set_error("wlq_workspace_reset: workspace must be non-null");
    return WLQ_ERR_NULL_POINTER;
  }
  if ((reinterpret_cast<uintptr_t>(workspace) & 3u) != 0) {
    wlq::set_error("wlq_workspace_reset: workspace must be 4-byte aligned");
    return WLQ_ERR_BAD_SHAPE;
  }
  const int words = (int)(std::min(workspace_bytes, wlq::kSyncBytes) / 4);
  if (words == 0) return WLQ_OK;
  hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, stream,
                     reinterpret_cast<uint32_t*>(workspace), words);
  return hip_status(hipGetLastError(), "wlq_workspace_reset");
}

int wlq_dequant(const int32_t* q_packed, const void* lut_c, void* W_out, int64_t N, int64_t K, int32_t bits,
                int64_t words_per_row, int32_t group_size, const int32_t* chunk_offsets, const uint16_t* chunk_cols,
                const uint8_t* chunk_vals, hipStream_t stream) {
  wlq::Layer L{};
  int st = make_layer(q_packed, lut_c, N, K, bits, words_per_row, group_size, chunk_offsets, chunk_cols, chunk_vals,
                      "wlq_dequant", &L);
  if (st != WLQ_OK) return st;
  if (N == 0 || K == 0) return WLQ_OK;
  if (W_out == nullptr) {
    wlq::set_error("wlq_dequant: W_out must be non-null");
    return WLQ_ERR_NULL_POINTER;
  }
  return hip_status(wlq::launch_dequant(L, reinterpret_cast<uint16_t*>(W_out), stream), "wlq_dequant");
}

int wlq_dora_epilogue(void* out, const float* lora_H, const void* lora_B, const void* dora_gamma, float lora_scale,
                      int32_t r, int64_t M, int64_t N, hipStream_t stream) {
  if (M < 0 || N < 0 || M > 0x7fffffff || N > 0x7fffffff) {
    wlq::set_error("wlq_dora_epilogue: bad shape M=%lld N=%lld", (long long)M, (long long)N);
    return WLQ_ERR_BAD_SHAPE;
  }
  const wlq::Dora D = make_dora(lora_B, lora_H, dora_gamma, nullptr, lora_scale, r);
  if (M == 0 || N == 0 || D.r == 0) return WLQ_OK;
  if (out == nullptr) {
    wlq::set_error("wlq_dora_epilogue: out must be non-null");
    return WLQ_ERR_NULL_POINTER;
  }
  return hip_status(wlq::launch_dora_epilogue(reinterpret_cast<uint16_t*>(out), (int)M, (int)N, D, stream),
                    "wlq_dora_epilogue");
}

}  // extern "C"
