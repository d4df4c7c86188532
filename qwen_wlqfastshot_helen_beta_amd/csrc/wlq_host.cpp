// Host-side (CPU) part of libwlq_hip.so: status strings, per-thread error
// messages, layout arithmetic, the continuous -> row-aligned repacker and the
// Elias-Fano -> chunk-CSR decoder (load-time formats).
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "wlq_abi.h"

namespace wlq {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int window_cols_for(int bits) { return bits == 4 ? 32 : bits == 3 ? 40 : bits == 2 ? 64 : 128; }

static int symbols_per_word(int bits) { return bits == 3 ? 10 : 32 / bits; }

}  // namespace wlq

extern "C" {

int wlq_abi_version(void) { return WLQ_ABI_VERSION; }

const char* wlq_status_string(int status) {
  switch (status) {
    case WLQ_OK: return "ok";
    case WLQ_ERR_NULL_POINTER: return "null pointer";
    case WLQ_ERR_BAD_SHAPE: return "bad shape";
    case WLQ_ERR_UNSUPPORTED: return "unsupported";
    case WLQ_ERR_CAPACITY: return "insufficient capacity";
    case WLQ_ERR_HIP: return "HIP error";
    case WLQ_ERR_FORMAT: return "malformed input";
    case WLQ_ERR_SYNC: return "cross-block hand-off failed (outputs written as NaN)";
    default: return "unknown status";
  }
}

const char* wlq_last_error(void) { return wlq::g_last_error.c_str(); }

int64_t wlq_words_per_row(int64_t K, int32_t bits) {
  if (bits < 1 || bits > 4 || K < 0) return -1;
  const int64_t spw = wlq::symbols_per_word(bits);
  const int64_t raw = (K + spw - 1) / spw;
  return (raw + 3) / 4 * 4;
}

int32_t wlq_chunk_width(int32_t bits) { return bits == 3 ? 640 : 512; }

// Reads symbol by symbol from the continuous stream (flat index n*K + k), as
// the reference repacker does (csrc/vllm_binding.cpp:216-233).
int wlq_repack_row_aligned(const uint32_t* src, int64_t src_words, int64_t N, int64_t K, int32_t bits,
                           uint32_t* dst, int64_t dst_words) {
  if (bits < 1 || bits > 4) {
    wlq::set_error("wlq_repack_row_aligned: unsupported bits=%d", (int)bits);
    return WLQ_ERR_UNSUPPORTED;
  }
  if (N < 0 || K < 0 || src_words < 0) {
    wlq::set_error("wlq_repack_row_aligned: bad shape");
    return WLQ_ERR_BAD_SHAPE;
  }
  const int64_t wpr = wlq_words_per_row(K, bits);
  if (dst_words < N * wpr) {
    wlq::set_error("wlq_repack_row_aligned: dst holds %lld words, need %lld", (long long)dst_words,
                   (long long)(N * wpr));
    return WLQ_ERR_CAPACITY;
  }
  if ((N * wpr > 0 && dst == nullptr) || (src_words > 0 && src == nullptr)) {
    wlq::set_error("wlq_repack_row_aligned: null buffer");
    return WLQ_ERR_NULL_POINTER;
  }
  const int64_t spw = wlq::symbols_per_word(bits);
  const uint32_t mask = (1u << bits) - 1u;
  if (K % spw == 0 && K / spw == wpr) {
    // every row is whole source words with no padding (Qwen2.5's K at 4 bits): the layouts
    // coincide word for word (3-bit: the two unused top bits cleared as the repack leaves them)
    const int64_t need = N * wpr;
    const int64_t have = std::min(need, src_words);
    if (bits == 3) {
      for (int64_t w = 0; w < have; ++w) dst[w] = src[w] & 0x3FFFFFFFu;
    } else if (have > 0) {
      std::memcpy(dst, src, sizeof(uint32_t) * (size_t)have);
    }
    if (need > have) std::memset(dst + have, 0, sizeof(uint32_t) * (size_t)(need - have));
    return WLQ_OK;
  }
  std::memset(dst, 0, sizeof(uint32_t) * (size_t)(N * wpr));
  int64_t f = 0;  // flat symbol index in the source stream
  for (int64_t n = 0; n < N; ++n) {
    uint32_t* row = dst + n * wpr;
    for (int64_t k = 0; k < K; ++k, ++f) {
      const int64_t sw = f / spw;
      const uint32_t sym = sw < src_words ? (src[sw] >> ((f - sw * spw) * bits)) & mask : 0u;
      row[k / spw] |= sym << ((k % spw) * bits);
    }
  }
  return WLQ_OK;
}

int64_t wlq_ef_total(const int64_t* tile_meta, int64_t num_tiles) {
  if (tile_meta == nullptr || num_tiles <= 0) return 0;
  int64_t t = 0;
  for (int64_t i = 0; i < num_tiles; ++i) t += std::max<int64_t>(0, tile_meta[2 * i + 1]);
  return t;
}

int wlq_ef_decode_chunk_csr(const int64_t* tile_meta, int64_t num_tiles, const uint32_t* bitstream,
                            int64_t stream_words, int64_t N, int64_t K, int64_t tile_size, int64_t chunk_m,
                            int32_t* offsets, uint16_t* cols, int64_t cols_capacity, int64_t* nnz_out) {
  if (N < 0 || K < 0 || tile_size <= 0 || chunk_m <= 0 || chunk_m > 65536 || num_tiles < 0 || stream_words < 0) {
    wlq::set_error("wlq_ef_decode_chunk_csr: bad shape");
    return WLQ_ERR_BAD_SHAPE;
  }
  if (offsets == nullptr && N > 0) {
    wlq::set_error("wlq_ef_decode_chunk_csr: offsets must be non-null");
    return WLQ_ERR_NULL_POINTER;
  }
  const int64_t nch = (K + chunk_m - 1) / chunk_m;
  std::memset(offsets, 0, sizeof(int32_t) * (size_t)(N * (nch + 1)));
  if (nnz_out) *nnz_out = 0;
  const int64_t total = wlq_ef_total(tile_meta, num_tiles);
  if (total == 0) return WLQ_OK;
  if (tile_meta == nullptr || (stream_words > 0 && bitstream == nullptr)) {
    wlq::set_error("wlq_ef_decode_chunk_csr: null input");
    return WLQ_ERR_NULL_POINTER;
  }
  const int64_t tiles_x = (K + tile_size - 1) / tile_size;
  const int64_t U = tile_size * tile_size;
  const int64_t total_bits = stream_words * 32;
  auto bit_at = [&](int64_t b) -> uint32_t { return (bitstream[b >> 5] >> (b & 31)) & 1u; };

  std::vector<uint64_t> coords;
  coords.reserve((size_t)total);
  for (int64_t t = 0; t < num_tiles; ++t) {
    const int64_t start = tile_meta[2 * t];
    const int64_t m = tile_meta[2 * t + 1];
    if (m <= 0) continue;
    if (start < 0) {
      wlq::set_error("wlq_ef_decode_chunk_csr: negative start bit in tile %lld", (long long)t);
      return WLQ_ERR_FORMAT;
    }
    int L = 0;  // low-bit width floor(log2(U / m)), 0 when m >= U
    if (U > m) L = std::max(0, (int)std::floor(std::log2((double)U / (double)m)));
    if (start + m * L > total_bits) {
      wlq::set_error("wlq_ef_decode_chunk_csr: tile %lld low bits past the stream end", (long long)t);
      return WLQ_ERR_FORMAT;
    }
    const int64_t base_r = (t / tiles_x) * tile_size;
    const int64_t base_c = (t % tiles_x) * tile_size;
    int64_t pos = start + m * L;  // unary high parts follow the low bits
    int64_t high = 0;
    for (int64_t i = 0; i < m; ++i) {
      uint64_t low = 0;
      for (int j = 0; j < L; ++j) low |= (uint64_t)bit_at(start + i * L + j) << j;
      while (pos < total_bits) {
        const uint32_t b = bit_at(pos++);
        if (b) break;
        ++high;
      }
      const int64_t local = (high << L) | (int64_t)low;
      const int64_t r = base_r + local / tile_size;
      const int64_t c = base_c + local % tile_size;
      if (r < N && c < K) coords.push_back(((uint64_t)r << 32) | (uint64_t)c);
    }
  }
  std::sort(coords.begin(), coords.end());
  const int64_t nnz = (int64_t)coords.size();
  if (nnz > cols_capacity || (nnz > 0 && cols == nullptr)) {
    wlq::set_error("wlq_ef_decode_chunk_csr: cols capacity %lld < %lld outliers", (long long)cols_capacity,
                   (long long)nnz);
    return WLQ_ERR_CAPACITY;
  }
  if (nnz > 0x7fffffff) {
    wlq::set_error("wlq_ef_decode_chunk_csr: too many outliers for int32 offsets");
    return WLQ_ERR_CAPACITY;
  }
  for (int64_t i = 0; i < nnz; ++i) {
    const int64_t r = (int64_t)(coords[i] >> 32);
    const int64_t c = (int64_t)(coords[i] & 0xffffffffu);
    cols[i] = (uint16_t)(c % chunk_m);
    offsets[r * (nch + 1) + c / chunk_m + 1] += 1;
  }
  int32_t running = 0;
  for (int64_t r = 0; r < N; ++r) {
    int32_t* row = offsets + r * (nch + 1);
    row[0] = running;
    for (int64_t c = 0; c < nch; ++c) {
      running += row[c + 1];
      row[c + 1] = running;
    }
  }
  if (nnz_out) *nnz_out = nnz;
  return WLQ_OK;
}

}  // extern "C"
