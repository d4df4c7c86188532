// PyTorch-ROCm extension `_C` of the vllm_wlq plugin.
//
// Same Python-visible functions, argument names and defaults as the reference
// binding (csrc/vllm_binding.cpp:455-532): gemv_forward, gemm_forward,
// dequant_w0, init_workspaces, decode_ef_to_chunk_csr,
// repack_q_indices_row_aligned.  Extensions are trailing defaulted arguments
// only: group_size (LUT per group of columns), lora_A (compute the DoRA H
// inside the product instead of taking lora_h / lora_H) and prepared (the
// layer's prepared layout from prepare_layer, an extra function).  Every
// device call goes through the C ABI of libwlq_hip.so (include/wlq_abi.h) on
// torch's current HIP stream.
//
// Differences from the reference, all stricter: dtypes, devices, contiguity and
// sizes are checked before launch, unsupported bit widths raise instead of
// silently doing nothing, and the split-K workspace is kept per (device, stream).
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "wlq_abi.h"

namespace {

void check_status(int st) {
  TORCH_CHECK(st == WLQ_OK, "wlq: ", wlq_status_string(st), ": ", wlq_last_error());
}

// Optional tensor -> pointer: absent, undefined or empty means nullptr
// (csrc/vllm_binding.cpp:272-285).
template <typename T>
const T* opt_ptr(const c10::optional<torch::Tensor>& t, c10::ScalarType want, const char* name,
                 const torch::Device& dev) {
  if (!t.has_value() || !t->defined() || t->numel() == 0) return nullptr;
  TORCH_CHECK(t->device() == dev, name, " must be on ", dev, ", got ", t->device());
  TORCH_CHECK(t->scalar_type() == want, name, " must be ", c10::toString(want), ", got ", t->scalar_type());
  TORCH_CHECK(t->is_contiguous(), name, " must be contiguous");
  return reinterpret_cast<const T*>(t->data_ptr());
}

// chunk_cols is uint16 in the checkpoint format; an int16 view of the same bytes is accepted too.
const uint16_t* cols_ptr(const c10::optional<torch::Tensor>& t, const torch::Device& dev) {
  if (!t.has_value() || !t->defined() || t->numel() == 0) return nullptr;
  const auto st = t->scalar_type();
  return opt_ptr<uint16_t>(t, st == torch::kInt16 ? torch::kInt16 : torch::kUInt16, "chunk_cols", dev);
}

void check_dev(const torch::Tensor& t, const char* name, const torch::Device& dev, c10::ScalarType want) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.device() == dev, name, " must be on ", dev, ", got ", t.device());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.scalar_type() == want, name, " must be ", c10::toString(want), ", got ", t.scalar_type());
}

int64_t lut_entries(int64_t bits) { return int64_t(1) << bits; }

void check_lut(const torch::Tensor& lut, int64_t N, int64_t K, int64_t bits, int64_t group_size) {
  int64_t ng = 1;
  if (group_size > 0 && group_size < K) ng = (K + group_size - 1) / group_size;
  TORCH_CHECK(lut.numel() == N * ng * lut_entries(bits), "lut_c has ", lut.numel(), " entries, expected N*",
              ng, "*", lut_entries(bits), " = ", N * ng * lut_entries(bits));
}

void check_csr(const c10::optional<torch::Tensor>& offs, const c10::optional<torch::Tensor>& cols,
               const c10::optional<torch::Tensor>& vals, int64_t N, int64_t K, int64_t bits) {
  if (!offs.has_value() || !offs->defined() || offs->numel() == 0) return;
  const int64_t nch = (K + wlq_chunk_width((int32_t)bits) - 1) / wlq_chunk_width((int32_t)bits);
  TORCH_CHECK(offs->numel() == N * (nch + 1), "chunk_offsets has ", offs->numel(), " entries, expected N*(nch+1) = ",
              N * (nch + 1));
  if (cols.has_value() && cols->defined() && vals.has_value() && vals->defined())
    TORCH_CHECK(cols->numel() == vals->numel(), "chunk_cols and chunk_vals differ in length");
}

// Workspaces (counter area + split-K / DoRA partial sums), one per (device, stream):
// the decode kernels hand partial results between blocks through the workspace, so
// two calls on one workspace must be ordered, and only calls on the same stream are
// (csrc/vllm_binding.cpp:238-251 keeps one per process, shared by every stream).
// init_workspaces sets a per-device size floor.  A stream's workspace is created (or
// replaced by a larger one) on demand; its 16 KiB counter area is zeroed by a fill
// kernel on that stream.  Replaced workspaces are never freed, since captured graphs
// may still use them.  Created while the stream is being captured, the fill kernel
// is only recorded (every replay of the graph runs it first), so the workspace is
// zeroed again before its next eager call.
constexpr size_t kCounterBytes = 16384;

struct Workspace {
  torch::Tensor buf;
  bool zero_before_eager = false;
  bool captured = false;  // handed to a call under graph capture: never freed
};

std::mutex g_ws_mu;
std::map<std::pair<int, uintptr_t>, Workspace> g_ws;
std::map<int, size_t> g_ws_floor;
std::vector<torch::Tensor> g_ws_retired;

bool stream_capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return st != hipStreamCaptureStatusNone;
}

// `stream` is torch's current stream on `dev` (the allocation and the fill run on it).
torch::Tensor workspace_for(const torch::Device& dev, size_t bytes, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  bytes = std::max({bytes, g_ws_floor[dev.index()], kCounterBytes});
  Workspace& w = g_ws[{dev.index(), reinterpret_cast<uintptr_t>(stream)}];
  const bool capturing = stream_capturing(stream);
  if (!w.buf.defined() || (size_t)w.buf.numel() < bytes) {
    // a buffer only eager calls used is released to torch's allocator (stream-ordered on `stream`)
    if (w.buf.defined() && w.captured) g_ws_retired.push_back(w.buf);
    w.buf = torch::empty({(int64_t)bytes}, torch::TensorOptions().dtype(torch::kUInt8).device(dev));
    w.buf.narrow(0, 0, (int64_t)kCounterBytes).zero_();  // a fill kernel (valid inside graph capture)
    w.zero_before_eager = capturing;
    w.captured = false;
  } else if (w.zero_before_eager && !capturing) {
    w.buf.narrow(0, 0, (int64_t)kCounterBytes).zero_();
    w.zero_before_eager = false;
  }
  w.captured = w.captured || capturing;
  return w.buf;
}

hipStream_t current_stream(const torch::Device& dev) { return c10::hip::getCurrentHIPStream(dev.index()).stream(); }

// The prepared layout is a uint8 buffer built by prepare_layer (empty or absent: not used).
const void* prepared_ptr(const c10::optional<torch::Tensor>& t, const torch::Device& dev) {
  if (!t.has_value() || !t->defined() || t->numel() == 0) return nullptr;
  check_dev(*t, "prepared", dev, torch::kUInt8);
  return t->data_ptr();
}

int64_t nnz_of(const c10::optional<torch::Tensor>& cols, const int32_t* offs) {
  if (offs == nullptr || !cols.has_value() || !cols->defined()) return 0;
  return cols->numel();
}

}  // namespace

void init_workspaces(int64_t max_N, int64_t max_K, torch::Device device) {
  TORCH_CHECK(device.is_cuda(), "init_workspaces: device must be a GPU");
  size_t need = 0;
  for (int bits = 1; bits <= 4; ++bits) {
    for (int32_t r : {0, 64}) {
      for (int64_t M = 1; M <= 32; ++M)
        need = std::max(need, wlq_gemm_workspace_bytes(M, max_N, max_K, bits, r, device.index()));
    }
    for (int64_t M = 64; M <= 16384; M *= 2)
      need = std::max(need, wlq_gemm_workspace_bytes(M, max_N, max_K, bits, 0, device.index()));
  }
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    size_t& f = g_ws_floor[device.index()];
    f = std::max(f, need);
  }
  workspace_for(device, need, current_stream(device));
}

// Raises when a cross-block hand-off failed on any workspace of `device` (the rows
// concerned were written as NaN); waits for the streams of those workspaces.
void check_workspaces(torch::Device device) {
  std::vector<std::pair<uintptr_t, torch::Tensor>> ws;
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    for (auto& kv : g_ws)
      if (kv.first.first == device.index()) ws.emplace_back(kv.first.second, kv.second.buf);
  }
  for (auto& w : ws)
    check_status(wlq_workspace_status(w.second.data_ptr(), (size_t)w.second.numel(),
                                      reinterpret_cast<hipStream_t>(w.first)));
}

// Clears the counter area of every workspace of `device` on its own stream (after a
// reported failure, once the calls that used them are done).
void reset_workspaces(torch::Device device) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  for (auto& kv : g_ws)
    if (kv.first.first == device.index())
      check_status(wlq_workspace_reset(kv.second.buf.data_ptr(), (size_t)kv.second.buf.numel(),
                                       reinterpret_cast<hipStream_t>(kv.first.second)));
}

void gemv_forward(torch::Tensor q_packed, torch::Tensor lut_c, torch::Tensor x, torch::Tensor out, int64_t N,
                  int64_t K, int64_t bits, c10::optional<torch::Tensor> chunk_offsets,
                  c10::optional<torch::Tensor> chunk_cols, c10::optional<torch::Tensor> chunk_vals,
                  c10::optional<torch::Tensor> lora_B, c10::optional<torch::Tensor> lora_h,
                  c10::optional<torch::Tensor> dora_gamma, double lora_scale, int64_t group_size,
                  c10::optional<torch::Tensor> lora_A, c10::optional<torch::Tensor> prepared) {
  const torch::Device dev = x.device();
  check_dev(q_packed, "q_packed", dev, torch::kInt32);
  check_dev(lut_c, "lut_c", dev, torch::kFloat16);
  check_dev(x, "x", dev, torch::kFloat16);
  check_dev(out, "out", dev, torch::kFloat16);
  TORCH_CHECK(bits >= 1 && bits <= 4, "gemv_forward: unsupported bits=", bits);
  TORCH_CHECK(x.numel() == K, "gemv_forward: x has ", x.numel(), " elements, expected K=", K);
  TORCH_CHECK(out.numel() == N, "gemv_forward: out has ", out.numel(), " elements, expected N=", N);
  TORCH_CHECK(q_packed.numel() >= N * wlq_words_per_row(K, (int32_t)bits), "q_packed is too small");
  check_lut(lut_c, N, K, bits, group_size);
  check_csr(chunk_offsets, chunk_cols, chunk_vals, N, K, bits);
  const int32_t* offs = opt_ptr<int32_t>(chunk_offsets, torch::kInt32, "chunk_offsets", dev);
  const uint16_t* cols = cols_ptr(chunk_cols, dev);
  const uint8_t* vals = opt_ptr<uint8_t>(chunk_vals, torch::kUInt8, "chunk_vals", dev);
  const void* B = opt_ptr<void>(lora_B, torch::kFloat16, "lora_B", dev);
  const float* h = opt_ptr<float>(lora_h, torch::kFloat32, "lora_h", dev);
  const void* g = opt_ptr<void>(dora_gamma, torch::kFloat16, "dora_gamma", dev);
  const void* A = opt_ptr<void>(lora_A, torch::kFloat16, "lora_A", dev);
  const int32_t r = (lora_B.has_value() && lora_B->defined() && lora_B->dim() > 1) ? (int32_t)lora_B->size(1) : 0;
  if (B && g && r > 0 && (h || A)) {
    TORCH_CHECK(lora_B->numel() == N * r, "lora_B must be [N, r]");
    if (h) TORCH_CHECK(lora_h->numel() == r, "lora_h must have r=", r, " elements");
    if (!h) TORCH_CHECK(lora_A->numel() == r * K, "lora_A must be [r, K]");
    TORCH_CHECK(dora_gamma->numel() == N, "dora_gamma must have N elements");
  }
  const size_t need = wlq_gemm_workspace_bytes(1, N, K, (int32_t)bits, (h || !A) ? 0 : r, dev.index());
  torch::Tensor ws = workspace_for(dev, need, current_stream(dev));
  const void* prep = prepared_ptr(prepared, dev);
  if (prep != nullptr) {
    check_status(wlq_gemm_prepared(x.data_ptr(), q_packed.data_ptr<int32_t>(), lut_c.data_ptr(), prep,
                                   (size_t)prepared->numel(), out.data_ptr(), 1, N, K, (int32_t)bits,
                                   wlq_words_per_row(K, (int32_t)bits), (int32_t)group_size, offs, cols, vals,
                                   nnz_of(chunk_cols, offs), h, B, g, A, (float)lora_scale, r, ws.data_ptr(),
                                   (size_t)ws.numel(), current_stream(dev)));
    return;
  }
  check_status(wlq_gemv(q_packed.data_ptr<int32_t>(), lut_c.data_ptr(), x.data_ptr(), out.data_ptr(), offs, cols,
                        vals, B, h, g, A, (float)lora_scale, r, N, K, (int32_t)bits, (int32_t)group_size,
                        ws.data_ptr(), (size_t)ws.numel(), current_stream(dev)));
}

void gemm_forward(torch::Tensor X, torch::Tensor q_packed, torch::Tensor lut_c, torch::Tensor out, int64_t N,
                  int64_t K, int64_t bits, int64_t words_per_row, c10::optional<torch::Tensor> chunk_offsets,
                  c10::optional<torch::Tensor> chunk_cols, c10::optional<torch::Tensor> chunk_vals,
                  c10::optional<torch::Tensor> lora_H, c10::optional<torch::Tensor> lora_B,
                  c10::optional<torch::Tensor> dora_gamma, double lora_scale, int64_t group_size,
                  c10::optional<torch::Tensor> lora_A, c10::optional<torch::Tensor> prepared) {
  const torch::Device dev = X.device();
  check_dev(X, "X", dev, torch::kFloat16);
  check_dev(q_packed, "q_packed", dev, torch::kInt32);
  check_dev(lut_c, "lut_c", dev, torch::kFloat16);
  check_dev(out, "out", dev, torch::kFloat16);
  TORCH_CHECK(bits >= 1 && bits <= 4, "gemm_forward: unsupported bits=", bits);
  TORCH_CHECK(X.dim() == 2 && X.size(1) == K, "gemm_forward: X must be [M, K=", K, "]");
  const int64_t M = X.size(0);
  TORCH_CHECK(out.numel() == M * N, "gemm_forward: out must hold M*N elements");
  TORCH_CHECK(q_packed.numel() >= N * words_per_row, "q_packed is too small");
  check_lut(lut_c, N, K, bits, group_size);
  check_csr(chunk_offsets, chunk_cols, chunk_vals, N, K, bits);
  const int32_t* offs = opt_ptr<int32_t>(chunk_offsets, torch::kInt32, "chunk_offsets", dev);
  const uint16_t* cols = cols_ptr(chunk_cols, dev);
  const uint8_t* vals = opt_ptr<uint8_t>(chunk_vals, torch::kUInt8, "chunk_vals", dev);
  const float* H = opt_ptr<float>(lora_H, torch::kFloat32, "lora_H", dev);
  const void* B = opt_ptr<void>(lora_B, torch::kFloat16, "lora_B", dev);
  const void* g = opt_ptr<void>(dora_gamma, torch::kFloat16, "dora_gamma", dev);
  const void* A = opt_ptr<void>(lora_A, torch::kFloat16, "lora_A", dev);
  const int32_t r = (lora_B.has_value() && lora_B->defined() && lora_B->dim() > 1) ? (int32_t)lora_B->size(1) : 0;
  if (B && g && r > 0 && (H || A)) {
    TORCH_CHECK(lora_B->numel() == N * r, "lora_B must be [N, r]");
    if (H) TORCH_CHECK(lora_H->numel() == M * r, "lora_H must be [M, r]");
    if (!H) TORCH_CHECK(lora_A->numel() == r * K, "lora_A must be [r, K]");
    TORCH_CHECK(dora_gamma->numel() == N, "dora_gamma must have N elements");
  }
  const size_t need = wlq_gemm_workspace_bytes(M, N, K, (int32_t)bits, (H || !A) ? 0 : r, dev.index());
  torch::Tensor ws = workspace_for(dev, need, current_stream(dev));
  const void* prep = prepared_ptr(prepared, dev);
  if (prep != nullptr) {
    check_status(wlq_gemm_prepared(X.data_ptr(), q_packed.data_ptr<int32_t>(), lut_c.data_ptr(), prep,
                                   (size_t)prepared->numel(), out.data_ptr(), M, N, K, (int32_t)bits, words_per_row,
                                   (int32_t)group_size, offs, cols, vals, nnz_of(chunk_cols, offs), H, B, g, A,
                                   (float)lora_scale, r, ws.data_ptr(), (size_t)ws.numel(), current_stream(dev)));
    return;
  }
  check_status(wlq_gemm(X.data_ptr(), q_packed.data_ptr<int32_t>(), lut_c.data_ptr(), out.data_ptr(), M, N, K,
                        (int32_t)bits, words_per_row, (int32_t)group_size, offs, cols, vals, H, B, g, A,
                        (float)lora_scale, r, ws.data_ptr(), (size_t)ws.numel(), current_stream(dev)));
}

void dequant_w0(torch::Tensor q_packed, torch::Tensor lut_c, torch::Tensor W_out, int64_t N, int64_t K, int64_t bits,
                int64_t words_per_row, torch::Tensor chunk_offsets, torch::Tensor chunk_cols,
                torch::Tensor chunk_vals, int64_t group_size) {
  const torch::Device dev = W_out.device();
  check_dev(q_packed, "q_packed", dev, torch::kInt32);
  check_dev(lut_c, "lut_c", dev, torch::kFloat16);
  check_dev(W_out, "W_out", dev, torch::kFloat16);
  TORCH_CHECK(W_out.numel() == N * K, "dequant_w0: W_out must hold N*K elements");
  check_lut(lut_c, N, K, bits, group_size);
  const bool csr = chunk_offsets.numel() > 0 && chunk_cols.numel() > 0 && chunk_vals.numel() > 0;
  if (csr) {
    check_dev(chunk_offsets, "chunk_offsets", dev, torch::kInt32);
    TORCH_CHECK(chunk_cols.device() == dev && chunk_vals.device() == dev, "outlier tensors must be on ", dev);
    check_csr(chunk_offsets, chunk_cols, chunk_vals, N, K, bits);
  }
  check_status(wlq_dequant(q_packed.data_ptr<int32_t>(), lut_c.data_ptr(), W_out.data_ptr(), N, K, (int32_t)bits,
                           words_per_row, (int32_t)group_size, csr ? chunk_offsets.data_ptr<int32_t>() : nullptr,
                           csr ? reinterpret_cast<const uint16_t*>(chunk_cols.data_ptr()) : nullptr,
                           csr ? reinterpret_cast<const uint8_t*>(chunk_vals.data_ptr()) : nullptr,
                           current_stream(dev)));
}

// Prepared (tile-contiguous) layout for the decode kernel, built on the device; an
// empty tensor when the layer has none (wlq_prepared_bytes == 0).
torch::Tensor prepare_layer(torch::Tensor q_packed, torch::Tensor lut_c, int64_t N, int64_t K, int64_t bits,
                            int64_t group_size, c10::optional<torch::Tensor> chunk_offsets,
                            c10::optional<torch::Tensor> chunk_cols, c10::optional<torch::Tensor> chunk_vals) {
  const torch::Device dev = q_packed.device();
  check_dev(q_packed, "q_packed", dev, torch::kInt32);
  check_dev(lut_c, "lut_c", dev, torch::kFloat16);
  TORCH_CHECK(bits >= 1 && bits <= 4, "prepare_layer: unsupported bits=", bits);
  TORCH_CHECK(q_packed.numel() >= N * wlq_words_per_row(K, (int32_t)bits), "q_packed is too small");
  check_lut(lut_c, N, K, bits, group_size);
  check_csr(chunk_offsets, chunk_cols, chunk_vals, N, K, bits);
  const int32_t* offs = opt_ptr<int32_t>(chunk_offsets, torch::kInt32, "chunk_offsets", dev);
  const uint16_t* cols = cols_ptr(chunk_cols, dev);
  const uint8_t* vals = opt_ptr<uint8_t>(chunk_vals, torch::kUInt8, "chunk_vals", dev);
  const bool csr = offs && cols && vals;
  const int64_t nnz = csr ? chunk_cols->numel() : 0;
  const size_t bytes = wlq_prepared_bytes(N, K, (int32_t)bits, (int32_t)group_size, nnz);
  auto opts = torch::TensorOptions().dtype(torch::kUInt8).device(dev);
  if (bytes == 0) return torch::empty({0}, opts);
  torch::Tensor buf = torch::empty({(int64_t)bytes}, opts);  // the caching allocator returns 512-byte aligned blocks
  check_status(wlq_prepare(q_packed.data_ptr<int32_t>(), lut_c.data_ptr(), N, K, (int32_t)bits, (int32_t)group_size,
                           csr ? offs : nullptr, csr ? cols : nullptr, csr ? vals : nullptr, nnz, buf.data_ptr(),
                           bytes, current_stream(dev)));
  return buf;
}

std::tuple<torch::Tensor, torch::Tensor> decode_ef_to_chunk_csr(torch::Tensor ef_tile_meta, torch::Tensor ef_bitstream,
                                                                int64_t N, int64_t K, int64_t tile_size,
                                                                int64_t chunk_m) {
  auto meta = ef_tile_meta.to(torch::kCPU, torch::kInt64).contiguous();
  auto bs = ef_bitstream.to(torch::kCPU).contiguous();
  TORCH_CHECK(bs.element_size() == 4 || bs.numel() == 0, "ef_bitstream must hold 32-bit words");
  TORCH_CHECK(chunk_m > 0, "chunk_m must be positive");
  const int64_t tiles = meta.numel() / 2;
  const int64_t nch = (K + chunk_m - 1) / chunk_m;
  auto offsets = torch::zeros({N, nch + 1}, torch::TensorOptions().dtype(torch::kInt32));
  const int64_t cap = wlq_ef_total(meta.data_ptr<int64_t>(), tiles);
  auto cols = torch::empty({cap}, torch::TensorOptions().dtype(torch::kUInt16));
  int64_t nnz = 0;
  check_status(wlq_ef_decode_chunk_csr(meta.data_ptr<int64_t>(), tiles,
                                       reinterpret_cast<const uint32_t*>(bs.numel() ? bs.data_ptr() : nullptr),
                                       bs.numel(), N, K, tile_size, chunk_m, offsets.data_ptr<int32_t>(),
                                       reinterpret_cast<uint16_t*>(cap ? cols.data_ptr() : nullptr), cap, &nnz));
  return std::make_tuple(offsets, cols.narrow(0, 0, nnz).clone());
}

std::tuple<torch::Tensor, int64_t> repack_q_indices_row_aligned(torch::Tensor q_packed_raw, int64_t N, int64_t K,
                                                                int64_t bits) {
  TORCH_CHECK(bits >= 1 && bits <= 4, "repack_q_indices_row_aligned: unsupported bits=", bits);
  auto src = q_packed_raw.to(torch::kCPU).contiguous();
  TORCH_CHECK(src.element_size() == 4 || src.numel() == 0, "q_packed_raw must hold 32-bit words");
  const int64_t wpr = wlq_words_per_row(K, (int32_t)bits);
  auto out = torch::zeros({N * wpr}, torch::TensorOptions().dtype(torch::kInt32));
  check_status(wlq_repack_row_aligned(reinterpret_cast<const uint32_t*>(src.numel() ? src.data_ptr() : nullptr),
                                      src.numel(), N, K, (int32_t)bits,
                                      reinterpret_cast<uint32_t*>(out.numel() ? out.data_ptr() : nullptr), N * wpr));
  return std::make_tuple(out, wpr);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("dequant_w0", &dequant_w0, "Bit-exact W0 reconstruction (LUT dequant + outlier overwrite)",
        py::arg("q_packed"), py::arg("lut_c"), py::arg("W_out"), py::arg("N"), py::arg("K"), py::arg("bits"),
        py::arg("words_per_row"), py::arg("chunk_offsets"), py::arg("chunk_cols"), py::arg("chunk_vals"),
        py::arg("group_size") = 0);
  m.def("decode_ef_to_chunk_csr", &decode_ef_to_chunk_csr, "Elias-Fano tiles -> chunk CSR (host)",
        py::arg("ef_tile_meta"), py::arg("ef_bitstream"), py::arg("N"), py::arg("K"), py::arg("tile_size"),
        py::arg("chunk_m"));
  m.def("repack_q_indices_row_aligned", &repack_q_indices_row_aligned,
        "Continuous -> row-aligned code packing (host)", py::arg("q_packed_raw"), py::arg("N"), py::arg("K"),
        py::arg("bits"));
  m.def("init_workspaces", &init_workspaces, "Pre-size the split-K workspace for graph capture", py::arg("max_N"),
        py::arg("max_K"), py::arg("device"));
  m.def("check_workspaces", &check_workspaces,
        "Raise if a cross-block hand-off failed on a workspace of the device (waits for its streams)",
        py::arg("device"));
  m.def("reset_workspaces", &reset_workspaces, "Clear the counter area of every workspace of the device",
        py::arg("device"));
  m.def("gemv_forward", &gemv_forward, "WLQ decode product (one activation row)", py::arg("q_packed"),
        py::arg("lut_c"), py::arg("x"), py::arg("out"), py::arg("N"), py::arg("K"), py::arg("bits"),
        py::arg("chunk_offsets") = py::none(), py::arg("chunk_cols") = py::none(), py::arg("chunk_vals") = py::none(),
        py::arg("lora_B") = py::none(), py::arg("lora_h") = py::none(), py::arg("dora_gamma") = py::none(),
        py::arg("lora_scale") = 1.0, py::arg("group_size") = 0, py::arg("lora_A") = py::none(),
        py::arg("prepared") = py::none());
  m.def("gemm_forward", &gemm_forward, "WLQ product for M activation rows", py::arg("X"), py::arg("q_packed"),
        py::arg("lut_c"), py::arg("out"), py::arg("N"), py::arg("K"), py::arg("bits"), py::arg("words_per_row"),
        py::arg("chunk_offsets") = py::none(), py::arg("chunk_cols") = py::none(), py::arg("chunk_vals") = py::none(),
        py::arg("lora_H") = py::none(), py::arg("lora_B") = py::none(), py::arg("dora_gamma") = py::none(),
        py::arg("lora_scale") = 1.0, py::arg("group_size") = 0, py::arg("lora_A") = py::none(),
        py::arg("prepared") = py::none());
  m.def("prepare_layer", &prepare_layer, "Prepared (tile-contiguous) layout of a layer for the decode kernel",
        py::arg("q_packed"), py::arg("lut_c"), py::arg("N"), py::arg("K"), py::arg("bits"), py::arg("group_size") = 0,
        py::arg("chunk_offsets") = py::none(), py::arg("chunk_cols") = py::none(), py::arg("chunk_vals") = py::none());
}
