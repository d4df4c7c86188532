// Device-side building blocks shared by the WLQ kernels (gfx950 / CDNA4).
//
// LUT dequantization.  A code selects an fp16 entry of a 2^bits-entry LUT.  On
// CDNA there is no per-lane indexed register read, so each lane keeps its LUT as
// two byte planes (the low and the high byte of every entry) and looks codes up
// with V_PERM_B32, which picks four bytes out of an 8-byte register pair under a
// 4-byte selector.  Selector values 0..7 pick a byte; values >= 13 produce 0xFF.
//
//  * 2^bits <= 8: one perm per plane looks up four codes.
//  * 16 entries: entries 0-7 and 8-15 live in two register pairs.  A selector
//    byte for code c is c (c < 8) or 0x80|c (c >= 8, i.e. >= 13 -> 0xFF); xor
//    0x88 gives the selector for the upper pair (0xFF for c < 8, c-8 else).  The
//    two lookups are combined with AND, so one 4-code lookup per plane costs two
//    perms and one AND.
//
// Eight codes at columns 0..7 of an 8-column block come out as four fp16 pairs
// in the column order P = [0,2,4,6,1,3,5,7]; activations are staged in the same
// order so both MFMA operands agree on the k index.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wlq {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  // byte i of the result = byte sel.byte[i] of the 64-bit value {hi:lo}
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Geometry of the packed code layout per bit width.  A "window" is what one
// lane reads with one 16-byte load: 4 words.
template <int BITS> struct CodeGeom;
template <> struct CodeGeom<4> { static constexpr int kSpw = 8;  static constexpr int kWin = 32;  };
template <> struct CodeGeom<3> { static constexpr int kSpw = 10; static constexpr int kWin = 40;  };
template <> struct CodeGeom<2> { static constexpr int kSpw = 16; static constexpr int kWin = 64;  };
template <> struct CodeGeom<1> { static constexpr int kSpw = 32; static constexpr int kWin = 128; };

// Byte planes of one LUT: lo[p]/hi[p] hold the low/high bytes of entries 4p..4p+3.
template <int BITS> struct LutPlanes {
  static constexpr int kRegs = (BITS == 4) ? 4 : 2;
  uint32_t lo[kRegs];
  uint32_t hi[kRegs];
};

// Raw LUT entries as fp16 pairs (entry 2j in the low half of raw[j]).
template <int BITS> struct LutRaw {
  static constexpr int kRegs = (BITS == 4) ? 8 : (BITS == 3) ? 4 : (BITS == 2) ? 2 : 1;
  uint32_t r[kRegs];
};

template <int BITS>
__device__ __forceinline__ void lut_load(LutRaw<BITS>& raw, const uint16_t* __restrict__ p) {
  if constexpr (BITS == 4) {
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(p);
    const u32x4_t b = *reinterpret_cast<const u32x4_t*>(p + 8);
    raw.r[0] = a.x; raw.r[1] = a.y; raw.r[2] = a.z; raw.r[3] = a.w;
    raw.r[4] = b.x; raw.r[5] = b.y; raw.r[6] = b.z; raw.r[7] = b.w;
  } else if constexpr (BITS == 3) {
    const u32x4_t a = *reinterpret_cast<const u32x4_t*>(p);
    raw.r[0] = a.x; raw.r[1] = a.y; raw.r[2] = a.z; raw.r[3] = a.w;
  } else if constexpr (BITS == 2) {
    const u32x2_t a = *reinterpret_cast<const u32x2_t*>(p);
    raw.r[0] = a.x; raw.r[1] = a.y;
  } else {
    raw.r[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

template <int BITS>
__device__ __forceinline__ void lut_zero(LutRaw<BITS>& raw) {
#pragma unroll
  for (int j = 0; j < LutRaw<BITS>::kRegs; ++j) raw.r[j] = 0u;
}

template <int BITS>
__device__ __forceinline__ LutPlanes<BITS> lut_planes(const LutRaw<BITS>& raw) {
  LutPlanes<BITS> t;
  if constexpr (BITS == 4) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      t.lo[p] = perm_b32(raw.r[2 * p + 1], raw.r[2 * p], 0x06040200u);
      t.hi[p] = perm_b32(raw.r[2 * p + 1], raw.r[2 * p], 0x07050301u);
    }
  } else if constexpr (BITS == 3) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      t.lo[p] = perm_b32(raw.r[2 * p + 1], raw.r[2 * p], 0x06040200u);
      t.hi[p] = perm_b32(raw.r[2 * p + 1], raw.r[2 * p], 0x07050301u);
    }
  } else if constexpr (BITS == 2) {
    t.lo[0] = perm_b32(raw.r[1], raw.r[0], 0x06040200u);
    t.hi[0] = perm_b32(raw.r[1], raw.r[0], 0x07050301u);
    t.lo[1] = 0u; t.hi[1] = 0u;
  } else {
    t.lo[0] = perm_b32(0u, raw.r[0], 0x06040200u);
    t.hi[0] = perm_b32(0u, raw.r[0], 0x07050301u);
    t.lo[1] = 0u; t.hi[1] = 0u;
  }
  return t;
}

// Interleave four low bytes and four high bytes into two fp16 pairs:
// (byte0, byte1) and (byte2, byte3) of the planes.
__device__ __forceinline__ void interleave(uint32_t lo, uint32_t hi, uint32_t& p01, uint32_t& p23) {
  p01 = perm_b32(hi, lo, 0x05010400u);
  p23 = perm_b32(hi, lo, 0x07030602u);
}

// 16-entry lookup of four codes whose selector bytes are already prepared
// (sel_a for entries 0-7 with 0x8X for the upper half, sel_b = sel_a ^ 0x88).
__device__ __forceinline__ void lookup16(const LutPlanes<4>& t, uint32_t sel_a, uint32_t sel_b,
                                         uint32_t& lo, uint32_t& hi) {
  lo = perm_b32(t.lo[1], t.lo[0], sel_a) & perm_b32(t.lo[3], t.lo[2], sel_b);
  hi = perm_b32(t.hi[1], t.hi[0], sel_a) & perm_b32(t.hi[3], t.hi[2], sel_b);
}

// 4-bit: one packed word (8 codes, code j at bits 4j) -> 4 fp16 pairs in order P.
__device__ __forceinline__ void dequant_word4(uint32_t w, const LutPlanes<4>& t, uint32_t out[4]) {
  const uint32_t ce = w & 0x0F0F0F0Fu;                               // codes 0,2,4,6
  const uint32_t se = ce | ((w << 4) & 0x80808080u);                 // bit7 <- bit3
  const uint32_t co = (w >> 4) & 0x0F0F0F0Fu;                        // codes 1,3,5,7
  const uint32_t so = co | (w & 0x80808080u);
  uint32_t le, he, lo, ho;
  lookup16(t, se, se ^ 0x88888888u, le, he);
  lookup16(t, so, so ^ 0x88888888u, lo, ho);
  interleave(le, he, out[0], out[1]);
  interleave(lo, ho, out[2], out[3]);
}

// Prepared ("selector-ready") 4-bit encoding of 8 codes c0..c7 (columns 0..7) in one word,
// used by the prepared layout of the decode kernel.  Byte j (j = 0..3) holds
//   bits 0-2: c_j & 7        bit 7: c_j >> 3                    (the "A" codes, columns 0-3)
//   bits 4-6: c_{4+j} & 7    bit 3: c_{4+((j+3)&3)} >> 3        (the "B" codes, columns 4-7)
// so  w & 0x87878787  is the lower-table selector of the A codes (c or 0x80|c, >= 13 -> 0xFF)
// and, after a 4-bit rotate right (each byte's high nibble moves down and the next byte's
// low nibble moves up, bringing the B code's top bit to bit 7), the same mask gives the B
// selectors.  XOR 0x80 turns a lower-table selector into the upper-table one.  Per 8
// codes: 5 selector ops, 8 perms + 4 ANDs for the two planes, 4 perms to interleave.
__host__ __device__ constexpr uint32_t sel_encode_byte(const uint32_t c[8], int j) {
  return (c[j] & 7u) | ((c[j] >> 3) << 7) | ((c[4 + j] & 7u) << 4) | ((c[4 + ((j + 3) & 3)] >> 3) << 3);
}

// One selector-encoded word -> 4 fp16 pairs in natural column order (0,1), (2,3), (4,5), (6,7).
__device__ __forceinline__ void dequant_word4s(uint32_t w, const LutPlanes<4>& t, uint32_t out[4]) {
  const uint32_t sa = w & 0x87878787u;
  const uint32_t rb = __builtin_amdgcn_alignbit(w, w, 4);  // rotate right by 4
  const uint32_t sb = rb & 0x87878787u;
  uint32_t la, ha, lb, hb;
  lookup16(t, sa, sa ^ 0x80808080u, la, ha);
  lookup16(t, sb, sb ^ 0x80808080u, lb, hb);
  interleave(la, ha, out[0], out[1]);
  interleave(lb, hb, out[2], out[3]);
}

// <= 8 entries: selector bytes are the codes themselves.
template <int BITS>
__device__ __forceinline__ void dequant_sel8(uint32_t se, uint32_t so, const LutPlanes<BITS>& t, uint32_t out[4]) {
  const uint32_t le = perm_b32(t.lo[1], t.lo[0], se);
  const uint32_t he = perm_b32(t.hi[1], t.hi[0], se);
  const uint32_t lo = perm_b32(t.lo[1], t.lo[0], so);
  const uint32_t ho = perm_b32(t.hi[1], t.hi[0], so);
  interleave(le, he, out[0], out[1]);
  interleave(lo, ho, out[2], out[3]);
}

// Selector bytes for the 8 codes of block s (codes 8s..8s+7 of a lane window).
// Window = 4 packed words w[0..3]; every shift below is a compile-time constant.
template <int BITS, int S>
__device__ __forceinline__ void block_selectors(const uint32_t w[4], uint32_t& se, uint32_t& so) {
  constexpr int spw = CodeGeom<BITS>::kSpw;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  uint32_t c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int idx = 8 * S + j;
    c[j] = (w[idx / spw] >> ((idx % spw) * BITS)) & mask;
  }
  se = c[0] | (c[2] << 8) | (c[4] << 16) | (c[6] << 24);
  so = c[1] | (c[3] << 8) | (c[5] << 16) | (c[7] << 24);
}

// Block s of a lane window -> 4 fp16 pairs (8 weights) in column order P.
template <int BITS, int S>
__device__ __forceinline__ void dequant_block(const uint32_t w[4], const LutPlanes<BITS>& t, uint32_t out[4]) {
  if constexpr (BITS == 4) {
    dequant_word4(w[S], t, out);
  } else {
    uint32_t se, so;
    block_selectors<BITS, S>(w, se, so);
    dequant_sel8<BITS>(se, so, t, out);
  }
}

// Permute 8 consecutive fp16 (natural order, as 4 pairs) into order P.
__device__ __forceinline__ u32x4_t permute_p(u32x4_t v) {
  u32x4_t r;
  r.x = perm_b32(v.y, v.x, 0x05040100u);  // (x0, x2)
  r.y = perm_b32(v.w, v.z, 0x05040100u);  // (x4, x6)
  r.z = perm_b32(v.y, v.x, 0x07060302u);  // (x1, x3)
  r.w = perm_b32(v.w, v.z, 0x07060302u);  // (x5, x7)
  return r;
}

// Position inside an 8-column block where column j is stored in order P.
__device__ __forceinline__ int p_slot(int j) { return (j & 1) ? (4 + (j >> 1)) : (j >> 1); }

__device__ __forceinline__ float h2f(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}

__device__ __forceinline__ uint16_t f2h_rn(float f) {
  const _Float16 h = static_cast<_Float16>(f);  // round to nearest even
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Code of column `col` in a packed row (runtime column).
template <int BITS>
__device__ __forceinline__ uint32_t code_at(const uint32_t* __restrict__ row, int col) {
  constexpr int spw = CodeGeom<BITS>::kSpw;
  const int wi = col / spw;
  const int sh = (col - wi * spw) * BITS;
  return (row[wi] >> sh) & ((1u << BITS) - 1u);
}

__device__ __forceinline__ float4_t mfma16x16x32(u32x4_t a, u32x4_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                0, 0, 0);
}

}  // namespace wlq
