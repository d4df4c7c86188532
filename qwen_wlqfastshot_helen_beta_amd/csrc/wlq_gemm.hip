// Prefill-shaped WLQ product (M > 32): dequantization into LDS feeding MFMA.
//
// Reference behaviour replaced: the M >= 16 path of gemm_forward
// (csrc/vllm_binding.cpp:355-393: full-matrix dequant into a workspace, cuBLAS
// HGEMM, separate DoRA pass) and gemm_metalog_dora_kernel's overwrite semantics
// (csrc/gemm_kernel.cu:204-228).  W is never materialized in HBM.
//
// Block tile 256 (M) x 128 (N), K step 64, 512 threads in two roles:
//
// * 4 consumer waves (one per SIMD), each a 128x64 sub-tile of
//   V_MFMA_F32_16X16X32_F16 (accumulators in AGPRs): per K step they read the
//   step's fragments from LDS and issue 64 MFMAs each, nothing else.
// * 4 producer waves (one per SIMD) fill the other LDS buffer with the next
//   step meanwhile: activations as they are, codes expanded through their LUT
//   byte planes into natural column order (two threads per W row, 32 columns each),
//   outliers overwritten (the reference's W0 = e5m2 << 8 at outlier positions).
//   Their global loads run four steps ahead in registers (two for 3-bit).
//
// So each SIMD runs one MFMA wave and one VALU wave side by side; one barrier
// per step hands the buffers over.  The roles run separate loops (the same
// number of barriers), so neither carries the other's registers.
//
// LDS tiles are unpadded 128-byte rows whose 16-byte units are XOR-swizzled by
// row: unit u of row r sits at u ^ swz(r), swz(r) = ((r >> 1) & 7) ^ ((r >> 3) & 1).
// The 16 rows of an MFMA fragment read land on distinct bank groups, and so do the
// producers' stores, whose activation loads stay 128-byte coalesced rows.  The
// consumers issue all fragment reads of a step before its MFMAs need them.
//
// The producer loop runs one 512-column outlier chunk (640 for 3-bit) per trip
// with its steps unrolled, so everything tied to chunk boundaries is fixed at
// compile time.  Outliers come from one of:
// * the layer's prepared patch lists (a layer with a prepared buffer): per 16-row tile and
//   128-column slab, the list of (row, column, e5m2) patches with duplicates resolved.  The
//   32 threads of list l (the rows producer wave l / 2 dequantizes, so its LDS writes stay in
//   program order behind that wave's tile stores) each take one entry per slab, loaded with
//   the step's prefetch; the list starts of the block's K range sit in LDS.  A wave whose
//   lists hold more than 32 entries in some slab walks its rows' CSR entries instead;
// * records prepared per (N tile, chunk) and producer thread by tile_entries_kernel: a
//   column mask per step and the values in column order, which a W thread writes over its
//   dequantized columns;
// * the row's CSR entries, walked directly (no workspace room for the records).
//
// DoRA: the low-rank term s * H . B^T is added in the epilogue of split 0 with
// V_MFMA_F32_16X16X4_F32 (fp32 operands, exact products) and every split scales
// by gamma; one split writes fp16((acc + s H B^T) * gamma), several write fp32
// partials that splitk_sum_kernel adds and rounds.  The producers stage the tile's H
// rows, B rows and gamma in LDS (the K loop is over, every buffer is free; for r <= 16
// the operands are loaded during the last K step), so the epilogue reads no global memory.
//
// Blocks are mapped so that each XCD works through a contiguous range of
// tiles, N-tile major: consecutive blocks of one XCD share W tiles in its L2.
#include <algorithm>
#include <utility>

#include "wlq_device.h"
#include "wlq_internal.h"

namespace wlq {
namespace {

constexpr int BM = 256;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int NT = 512;
constexpr int NP = 256;          // producer threads (waves 4..7)
// Outlier records, one slot of ol_slot_words(spc) words per (N tile, chunk), spc = K steps per
// chunk; producer thread t handles row t / 2 of the tile, columns 32 (t % 2) + [0, 32) of each
// 64-column K step:
//   [spc][NP]    masks: bit c of mask[s][t] = an outlier at that column of step s
//   [spc][NP][2] the first kOlVals e5m2 values of (s, t) in column order
constexpr int kOlSteps = 10;     // K steps per outlier chunk: 640 / 64 (3-bit), 512 / 64 otherwise
constexpr int kOlVals = 8;
constexpr int ol_slot_words(int spc) { return 3 * spc * NP; }
constexpr int kMaxSplits = 32;
constexpr int kXcds = 8;
// DoRA operands staged in LDS for the epilogue of split 0, kDr ranks per round (padded strides
// against bank conflicts): fp32 H rows [BM][kDhStride], fp16 B rows [BN][kDbStride], gamma [BN].
constexpr int kDr = 64;
constexpr int kDrPre = 16;                    // ranks loaded during the last K step
constexpr int kDhStride = kDr + 1;
constexpr int kDbStride = kDr + 2;
constexpr int kDbOff = BM * kDhStride * 4;    // bytes
constexpr int kDgOff = kDbOff + BN * kDbStride * 2;
// Patch-list starts of a block's K range in LDS: 8 lists x (slabs + 1) words.  Prepared layers
// have K <= 65535 (512 slabs; whole 640-column chunks reach 515).
constexpr int kTabSlabs = 520;
constexpr int kTabBytes = 8 * kTabSlabs * 4;
enum OlMode : int { kOlDirect = 0, kOlRecords = 1, kOlLists = 2 };

struct GemmArgs {
  const uint32_t* q;
  const uint16_t* lut;
  const uint16_t* X;
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
  uint32_t g_magic;
  int ksteps_per_split, splits;
  int tiles_m, tiles_n, tiles;
  int has_csr;
  const uint32_t* tent;  // outlier records [tiles_n * nch][ol_slot_words], or nullptr (direct CSR reads)
  const uint32_t* wpidx;   // prepared patch lists (nullptr: records or CSR walk)
  const uint32_t* wpatch;
  uint32_t patch_bytes;
  int T, S;                // prepared 16-row tiles and 128-column slabs
  const uint32_t* pcodes;  // prepared codes and LUT planes (PREP kernels)
  const uint32_t* pplanes;
  int png;                 // LUT groups per row of the prepared planes
};

struct GemmSmem {
  uint16_t a[2][BM * BK];
  uint16_t b[2][BN * BK];
};
static_assert(kDgOff + BN * 2 <= (int)sizeof(GemmSmem), "staged DoRA operands fit the tile buffers");

__device__ __forceinline__ int group_of(int col, uint32_t magic) { return (int)__umulhi((uint32_t)col, magic); }

// Swizzle of a tile row (depends on row % 16 only).
__device__ __forceinline__ int swz(int row) { return ((row >> 1) & 7) ^ ((row >> 3) & 1); }

// Buffer resources (raw, stride 0): a load whose offset is at or past the
// resource's size returns zeros, which is how activation columns past K and
// code words past the last row read as harmless values without per-lane checks.
constexpr int kRsrcWord3 = 0x00020000;         // raw buffer, 32-bit data format (gfx9)
constexpr uint32_t kOutOfRange = 0x80000000u;  // past every resource (sizes are < 2^31 bytes)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}

// LUT modes: one LUT per row (loaded once); groups of G % 128 == 0 columns (a group
// spans two K steps: planes built on even steps); G % 64 == 0 (one group per step);
// G % 32 == 0 (one group per thread's 32 columns of a step).
enum LutMode : int { kLutRow = 0, kLutPair = 1, kLutStep = 2, kLutHalf = 3 };

// Code words of one thread's 32 columns of a step.
template <int BITS> struct StepCodes { static constexpr int kWords = BITS == 4 ? 4 : BITS == 3 ? 6 : BITS == 2 ? 2 : 1; };

// Columns c0 .. c0 + 31 (c0 % 32 == 0) of the row at byte offset qbase.
template <int BITS>
__device__ __forceinline__ void load_codes(__amdgpu_buffer_rsrc_t rq, uint32_t qbase, int c0,
                                           uint32_t w[StepCodes<BITS>::kWords]) {
  if constexpr (BITS == 4) {  // words c0/8 .. + 3
    const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)(qbase + (uint32_t)(c0 >> 1)), 0, 0);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else if constexpr (BITS == 2) {  // words c0/16, + 1
    const u32x2_t a = __builtin_amdgcn_raw_buffer_load_b64(rq, (int)(qbase + (uint32_t)(c0 >> 2)), 0, 0);
    w[0] = a.x; w[1] = a.y;
  } else if constexpr (BITS == 1) {  // word c0/32
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(rq, (int)(qbase + (uint32_t)(c0 >> 3)), 0, 0);
  } else {  // 3-bit: per 16-column piece p the three words from (c0 + 16 p) / 10
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const uint32_t off = qbase + 4u * (uint32_t)((c0 + 16 * p) / 10);
#pragma unroll
      for (int j = 0; j < 3; ++j) w[3 * p + j] = __builtin_amdgcn_raw_buffer_load_b32(rq, (int)(off + 4u * j), 0, 0);
    }
  }
}

template <int BITS>
__device__ __forceinline__ void lut_load_buf(LutRaw<BITS>& raw, __amdgpu_buffer_rsrc_t rl, uint32_t voff,
                                             uint32_t soff) {
  if constexpr (BITS == 4) {
    const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(rl, (int)voff, (int)soff, 0);
    const u32x4_t b = __builtin_amdgcn_raw_buffer_load_b128(rl, (int)(voff + 16u), (int)soff, 0);
    raw.r[0] = a.x; raw.r[1] = a.y; raw.r[2] = a.z; raw.r[3] = a.w;
    raw.r[4] = b.x; raw.r[5] = b.y; raw.r[6] = b.z; raw.r[7] = b.w;
  } else if constexpr (BITS == 3) {
    const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(rl, (int)voff, (int)soff, 0);
    raw.r[0] = a.x; raw.r[1] = a.y; raw.r[2] = a.z; raw.r[3] = a.w;
  } else if constexpr (BITS == 2) {
    const u32x2_t a = __builtin_amdgcn_raw_buffer_load_b64(rl, (int)voff, (int)soff, 0);
    raw.r[0] = a.x; raw.r[1] = a.y;
  } else {
    raw.r[0] = __builtin_amdgcn_raw_buffer_load_b32(rl, (int)voff, (int)soff, 0);
  }
}

// 8 columns (unit U of the thread's 32, columns c0 + 8U ..) expanded to fp16 pairs in
// natural column order (the activations are then staged as they are in memory).
template <int BITS, int U>
__device__ __forceinline__ void dequant_unit(const uint32_t* w, int c0, const LutPlanes<BITS>& t, uint32_t out[4]) {
  if constexpr (BITS == 4) {
    uint32_t p[4];  // order P: (c0,c2) (c4,c6) (c1,c3) (c5,c7)
    dequant_word4(w[U], t, p);
    out[0] = perm_b32(p[2], p[0], 0x05040100u);  // (c0, c1)
    out[1] = perm_b32(p[2], p[0], 0x07060302u);  // (c2, c3)
    out[2] = perm_b32(p[3], p[1], 0x05040100u);  // (c4, c5)
    out[3] = perm_b32(p[3], p[1], 0x07060302u);  // (c6, c7)
  } else {
    constexpr int P = U >> 1;    // 16-column piece
    constexpr int BLK = U & 1;   // 8-column block inside the piece
    uint32_t code[8];
    if constexpr (BITS == 2) {
#pragma unroll
      for (int j = 0; j < 8; ++j) code[j] = (w[P] >> (2 * (8 * BLK + j))) & 3u;
    } else if constexpr (BITS == 1) {
      const uint32_t v = w[0] >> (16 * P + 8 * BLK);
#pragma unroll
      for (int j = 0; j < 8; ++j) code[j] = (v >> j) & 1u;
    } else {  // 3-bit: slot s0 = c16 % 10 of word c16 / 10; codes up to slot s0 + 15 < 25
      const int c16 = c0 + 16 * P;
      const int s0 = c16 - (c16 / 10) * 10;
      const uint32_t* pw = w + 3 * P;
      // the 25 slots of three words as two 64-bit windows (values only: no indexed access)
      const uint64_t lo = (uint64_t)pw[0] | ((uint64_t)pw[1] << 30);   // slots 0..19 at 3 bits each
      const uint64_t hi = (uint64_t)pw[1] | ((uint64_t)pw[2] << 30);   // slots 10..29
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int idx = s0 + 8 * BLK + j;
        const uint64_t src = idx < 20 ? lo : hi;
        const int sh = 3 * (idx < 20 ? idx : idx - 10);
        code[j] = (uint32_t)(src >> sh) & 7u;
      }
    }
    // selectors of columns 0-3 and 4-7: the lookups then come out in natural order
    const uint32_t s0 = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
    const uint32_t s1 = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
    dequant_sel8<BITS>(s0, s1, t, out);
  }
}

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// ------------------------------------------------------------------ kernel

// Producer registers carrying one K step from global memory to LDS.
template <int BITS>
struct StepRegs {
  u32x4_t x[8];                             // activation units u = ptid + NP * j
  uint32_t cw[StepCodes<BITS>::kWords];     // code words of the thread's 32 columns
  LutRaw<BITS> lr;                          // group LUT of the step
  uint32_t pe, pok;                         // patch-list entry of the step's slab, whether it is one
  u32x4_t plo, phi;                         // prepared LUT planes of the step's group (PREP)
};

// PREP: codes and LUT planes from the layer's prepared buffer (4-bit selector-ready nibbles; 3-bit
// layers are stored there as nibbles with 16-entry planes), outliers from its patch lists; BITS then
// only sets the outlier chunk (640 columns for 3-bit).  Otherwise the row-layout tensors, with
// outlier records (a.tent) or the CSR walk.
template <int BITS, int LUTM, bool HAS_CSR, bool X_VEC, bool LISTS>
__global__ __launch_bounds__(NT, 2) void gemm_kernel(const GemmArgs a) {
  constexpr int NCB = 1 << BITS;
  constexpr int SPC = (BITS == 3 ? 640 : 512) / BK;  // K steps per outlier chunk (even)
  static_assert(SPC % 2 == 0, "register sets keep their step parity");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  GemmSmem& sm = *reinterpret_cast<GemmSmem*>(smem_raw);

  const int tid = threadIdx.x;
  const int wave = tid >> 6;

  // tile of this block: XCD-contiguous ranges, N-tile major
  const int split = blockIdx.x / a.tiles;
  int t = blockIdx.x - split * a.tiles;
  if (a.tiles % kXcds == 0) {
    const int per = a.tiles / kXcds;
    t = (t % kXcds) * per + t / kXcds;
  }
  const int tn = t / a.tiles_m;
  const int m0 = (t - tn * a.tiles_m) * BM;
  const int n0 = tn * BN;

  // K range: whole outlier chunks; steps past K (the last chunk's tail) read zero
  // activations and add nothing
  const int ksteps_total = (a.K + BK - 1) / BK;
  const int kt_begin = split * a.ksteps_per_split;
  const int kt_end = min(ksteps_total, kt_begin + a.ksteps_per_split);
  const int ck_begin = kt_begin / SPC;
  const int ck_end = (kt_end + SPC - 1) / SPC;
  const bool has_work = kt_begin < kt_end;

  // Outliers: prepared patch lists, records (when the workspace holds them) or direct reads of
  // the CSR arrays.
  const int ol_mode = !HAS_CSR ? kOlDirect : LISTS ? kOlLists : a.tent != nullptr ? kOlRecords : kOlDirect;
  const int prologue_barriers = 1;

  if (wave < 4) {
    // ------------------------------------------------------------ consumer waves
    const int lane = tid & 63;
    const int wm = wave >> 1;  // 0..1: 128-row slice of the M tile
    const int wn = wave & 1;   // 0..1: 64-column slice of the N tile
    const int r = lane & 15;
    const int kq = lane >> 4;

    float4_t acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    if (has_work) {
      // fragment rows 16 i + r of the wave's slices; k unit 4 ks + kq, swizzled by row
      const int a_frag = (128 * wm + r) * BK;
      const int b_frag = (64 * wn + r) * BK;
      const int f_unit0 = 8 * ((0 + kq) ^ swz(r));
      const int f_unit1 = 8 * ((4 + kq) ^ swz(r));
      for (int i = 0; i < prologue_barriers; ++i) __syncthreads();
      const int steps = (ck_end - ck_begin) * SPC;
      for (int st = 0; st < steps; ++st) {
        const int buf = st & 1;
        // all fragments of the step in flight early: ks = 0 first, ks = 1 spread over
        // the ks = 0 MFMAs, so no MFMA waits for an LDS round trip of its own
        u32x4_t af[2][8], bf[2][4];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int fu = ks ? f_unit1 : f_unit0;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            bf[ks][j] = *reinterpret_cast<const u32x4_t*>(&sm.b[buf][b_frag + 16 * j * BK + fu]);
#pragma unroll
          for (int i = 0; i < 8; ++i)
            af[ks][i] = *reinterpret_cast<const u32x4_t*>(&sm.a[buf][a_frag + 16 * i * BK + fu]);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma16x16x32(af[ks][i], bf[ks][j], acc[i][j]);
        __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // DS read: ks = 0 fragments
#pragma unroll
        for (int q = 0; q < 12; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read: a ks = 1 fragment
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 40, 0);
        __syncthreads();
      }
    }

    // Epilogue.  Lane holds D[4*kq + e][r] of every 16x16 tile (i, j).  Split 0 adds the
    // DoRA term and every split scales by gamma (the split-K sum of gamma-scaled partials
    // is gamma times the sum), so the split-K reduce is a plain sum.
    const bool dora = a.r > 0 && split == 0;
    if (dora) {
      // acc += s * H . B^T on the matrix core in fp32 (V_MFMA_F32_16X16X4_F32: A = s*H,
      // lane l holds row l%16, k = l/16; B = B^T, lane l holds k = l/16, column l%16), the
      // operands read from the producers' staging (rows past M / N and ranks past r as zero).
      const float* hb = reinterpret_cast<const float*>(smem_raw) + (128 * wm + r) * kDhStride + kq;
      const uint16_t* bb = reinterpret_cast<const uint16_t*>(smem_raw + kDbOff) + (64 * wn + r) * kDbStride + kq;
      for (int c0 = 0; c0 < a.r; c0 += kDr) {
        __syncthreads();  // ranks c0 .. c0 + kDr - 1 staged
        const int nr = min(kDr, a.r - c0);
        for (int kb = 0; kb < nr; kb += 16) {
          float hv[4][8], bv[4][4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
#pragma unroll
            for (int i = 0; i < 8; ++i) hv[u][i] = a.scale * hb[16 * i * kDhStride + kb + 4 * u];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[u][j] = h2f(bb[16 * j * kDbStride + kb + 4 * u]);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
              for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(hv[u][i], bv[u][j], acc[i][j], 0, 0, 0);
        }
        if (c0 + kDr < a.r) __syncthreads();  // round read
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + 64 * wn + 16 * j + r;
      if (n >= a.N) continue;
      const float g = dora ? h2f(reinterpret_cast<const uint16_t*>(smem_raw + kDgOff)[64 * wn + 16 * j + r])
                           : a.r > 0 ? h2f(a.gamma[n]) : 1.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m0 + 128 * wm + 16 * i + 4 * kq + e;
          if (m >= a.M) continue;
          const float v = a.r > 0 ? acc[i][j][e] * g : acc[i][j][e];
          if (a.splits == 1)
            a.out[(size_t)m * a.N + n] = f2h_rn(v);
          else
            a.partial[((size_t)split * a.M + m) * a.N + n] = v;
        }
      }
    }
    return;
  }

  // -------------------------------------------------------------- producer waves
  const int ptid = tid - 4 * 64;

  // DoRA operands of split 0: thread ptid stages H row m0 + ptid, half of B row n0 + ptid / 2
  // and gamma of row n0 + ptid.  With r <= kDrPre they are loaded during the last K step.
  const bool dora = a.r > 0 && split == 0;
  const bool pre = dora && a.r <= kDrPre && has_work;
  float dh[kDrPre];
  uint16_t db[kDrPre / 2];
  auto dora_pre = [&]() __attribute__((always_inline)) {
    const int m = m0 + ptid;
    const float* hrow = a.H + (size_t)min(m, a.M - 1) * a.r;
#pragma unroll
    for (int k = 0; k < kDrPre; ++k) {
      const float v = hrow[min(k, a.r - 1)];
      dh[k] = (m < a.M && k < a.r) ? v : 0.f;
    }
    const int nbr = n0 + (ptid >> 1);
    const uint16_t* brow = a.B + (size_t)min(nbr, a.N - 1) * a.r;
#pragma unroll
    for (int k = 0; k < kDrPre / 2; ++k) {
      const int rk = (kDrPre / 2) * (ptid & 1) + k;
      const uint16_t v = brow[min(rk, a.r - 1)];
      db[k] = (nbr < a.N && rk < a.r) ? v : (uint16_t)0;
    }
  };

  // A producer: units u = ptid + NP * j, row u / 8 = ptid / 8 + 32 j, columns 8 (ptid % 8) + [0, 8)
  // (eight lanes read one 128-byte row)
  const int xc8 = ptid & 7;
  const int xrow0 = ptid >> 3;
  const int xoff = xrow0 * BK + 8 * (xc8 ^ swz(xrow0));  // rows + 32 j share the swizzle
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.X, (uint32_t)((size_t)a.M * a.K * 2));
  uint32_t xbase[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    xbase[j] = (uint32_t)(((size_t)min(m0 + xrow0 + 32 * j, a.M - 1) * a.K + 8 * xc8) * 2);
  const int xlim = a.K - 8 * xc8;  // the unit holds activations while k0 < xlim

  // W producer: row nl of the tile, columns [32 h, 32 h + 32) of each step
  const int nl = ptid >> 1;
  const int hh = ptid & 1;
  const int nb = n0 + nl;
  const bool brow_ok = nb < a.N;
  const int nbc = brow_ok ? nb : (a.N - 1);
  const int wsw = swz(nl);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q, (uint32_t)((size_t)a.N * a.wpr * 4));
  const __amdgpu_buffer_rsrc_t rl = make_rsrc(a.lut, (uint32_t)((size_t)a.N * a.ng * NCB * 2));
  const uint32_t qbase = (uint32_t)nbc * (uint32_t)a.wpr * 4u;
  const uint32_t lbase = (uint32_t)nbc * (uint32_t)(a.ng * NCB * 2);

  // Prepared layout: this thread's 32 columns of step kt are the 16 bytes of lane
  // (row % 16) + 16 (2 (kt % 2) + hh) of tile (n0 + nl) / 16, slab kt / 2; its row's LUT planes
  // of group g are the 16-byte rows (row % 16) of planes [tile][g][0 / 1].
  const int ptl = (n0 + nl) >> 4;
  const __amdgpu_buffer_rsrc_t rpq = make_rsrc(a.pcodes, LISTS ? (uint32_t)((size_t)a.T * a.S * 1024) : 0u);
  const __amdgpu_buffer_rsrc_t rpl = make_rsrc(a.pplanes, LISTS ? (uint32_t)((size_t)a.T * a.png * 512) : 0u);
  const uint32_t pqbase = (uint32_t)((size_t)ptl * a.S * 1024 + (size_t)((nl & 15) + 16 * hh) * 16);
  const uint32_t plbase = (uint32_t)((size_t)ptl * a.png * 512 + (size_t)(nl & 15) * 16);
  LutPlanes<4> pp_row;
  if constexpr (LISTS && LUTM == kLutRow) {
    const u32x4_t lo = __builtin_amdgcn_raw_buffer_load_b128(rpl, (int)plbase, 0, 0);
    const u32x4_t hi = __builtin_amdgcn_raw_buffer_load_b128(rpl, (int)(plbase + 256u), 0, 0);
    pp_row.lo[0] = lo.x; pp_row.lo[1] = lo.y; pp_row.lo[2] = lo.z; pp_row.lo[3] = lo.w;
    pp_row.hi[0] = hi.x; pp_row.hi[1] = hi.y; pp_row.hi[2] = hi.z; pp_row.hi[3] = hi.w;
  }
  LutPlanes<BITS> pl_row;
  if constexpr (!LISTS && LUTM == kLutRow) {
    LutRaw<BITS> raw;
    lut_load_buf<BITS>(raw, rl, lbase, 0u);
    pl_row = lut_planes<BITS>(raw);
  }
  LutPlanes<BITS> pl_pair;  // kLutPair: planes of the current two-step group

  // Outliers.  Prepared: at the start of the step that stages step st of chunk ck (before that
  // step's prefetch loads, so waiting for them leaves the prefetch in flight) the thread loads
  // its column mask of that step and the step's first kOlVals values.  A step costs one test when
  // its mask is empty; each set bit writes the next value.  A step with more than kOlVals
  // outliers in the thread's 32 columns, or no records at all, reads the row's CSR entries of the
  // chunk directly for that step.
  uint32_t om = 0u, ov0 = 0u, ov1 = 0u;
  auto ol_issue = [&](int ck, auto st_c) __attribute__((always_inline)) {
    constexpr int ST = decltype(st_c)::value;
    const uint32_t* slot = a.tent + ((size_t)tn * a.nch + ck) * ol_slot_words(SPC);
    om = slot[ST * NP + ptid];
    const uint32_t* vw = slot + SPC * NP + 2 * (ST * NP + ptid);
    ov0 = vw[0];
    ov1 = vw[1];
  };

  // Patch lists: thread ptid takes entry ptid % 32 of list li = ptid / 32 of each slab, the list
  // of prepared tile 8 tn + li (rows 16 li .. 16 li + 15 of the N tile, which producer wave li / 2
  // dequantizes).  ltab[li][i]: start of the list of slab s_first + i; slabs past K hold empty
  // lists.
  const int li = ptid >> 5;
  const int es = ptid & 31;
  const int s_first = kt_begin >> 1;  // the range starts at a whole chunk (an even step)
  const int ntab = (ck_end - ck_begin) * (SPC / 2) + 1;
  uint32_t* ltab = reinterpret_cast<uint32_t*>(smem_raw + sizeof(GemmSmem));
  const __amdgpu_buffer_rsrc_t rpatch = make_rsrc(a.wpatch, a.patch_bytes);

  // Start and length of the list of step kt's slab (read a step before the loads that use them:
  // right after a barrier the LDS queue holds the consumers' fragment reads).
  auto list_of = [&](int kt, uint32_t& st, uint32_t& cnt) __attribute__((always_inline)) {
    const int si = min((kt >> 1) - s_first, ntab - 2);
    st = ltab[li * ntab + si];
    cnt = ltab[li * ntab + si + 1] - st;
  };
  // Loads of step kt into S.  EVEN: the step's index from the range start is even.  LISTS: the
  // thread's entry of list (st, cnt), the one of the step's slab.
  auto load_step = [&](StepRegs<BITS>& S, int kt, auto even_c, auto lists_c, uint32_t st, uint32_t cnt)
                       __attribute__((always_inline)) {
    constexpr bool kEven = decltype(even_c)::value;
    if constexpr (decltype(lists_c)::value) {
      const bool ok = (uint32_t)es < cnt;
      S.pok = ok ? 1u : 0u;
      S.pe = __builtin_amdgcn_raw_buffer_load_b32(rpatch, (int)(ok ? (st + (uint32_t)es) * 4u : kOutOfRange), 0, 0);
    }
    const int k0 = kt * BK;
    if constexpr (X_VEC) {
      const bool in = k0 < xlim;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        S.x[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(in ? xbase[j] + 2u * (uint32_t)k0 : kOutOfRange),
                                                       0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int m = m0 + xrow0 + 32 * j;
        const int col = k0 + 8 * xc8;
        u32x4_t v = {0u, 0u, 0u, 0u};
        if (m < a.M) {
          const uint16_t* src = a.X + (size_t)m * a.K + col;
          uint32_t e[8];
#pragma unroll
          for (int q2 = 0; q2 < 8; ++q2) e[q2] = (col + q2 < a.K) ? (uint32_t)src[q2] : 0u;
          v.x = e[0] | (e[1] << 16);
          v.y = e[2] | (e[3] << 16);
          v.z = e[4] | (e[5] << 16);
          v.w = e[6] | (e[7] << 16);
        }
        S.x[j] = v;
      }
    }
    const int c0 = k0 + 32 * hh;
    if constexpr (LISTS) {
      const u32x4_t cv = __builtin_amdgcn_raw_buffer_load_b128(rpq, (int)(pqbase + (uint32_t)(kt >> 1) * 1024u +
                                                                          (uint32_t)(kt & 1) * 512u), 0, 0);
      S.cw[0] = cv.x; S.cw[1] = cv.y; S.cw[2] = cv.z; S.cw[3] = cv.w;
      if constexpr (LUTM != kLutRow) {
        const int g = min(group_of(c0, a.g_magic), a.png - 1);
        S.plo = __builtin_amdgcn_raw_buffer_load_b128(rpl, (int)(plbase + (uint32_t)g * 512u), 0, 0);
        S.phi = __builtin_amdgcn_raw_buffer_load_b128(rpl, (int)(plbase + (uint32_t)g * 512u + 256u), 0, 0);
      }
      return;
    }
    load_codes<BITS>(rq, qbase, c0, S.cw);
    if constexpr (LUTM == kLutStep || (LUTM == kLutPair && kEven)) {
      const int g = min(group_of(k0, a.g_magic), a.ng - 1);  // uniform
      lut_load_buf<BITS>(S.lr, rl, lbase, (uint32_t)(g * NCB * 2));
    } else if constexpr (LUTM == kLutHalf) {
      const int g = min(group_of(c0, a.g_magic), a.ng - 1);
      lut_load_buf<BITS>(S.lr, rl, lbase + (uint32_t)(g * NCB * 2), 0u);
    }
  };

  // A and W tiles of step kt into LDS buffer buf (outliers separately).
  auto store_main = [&](const StepRegs<BITS>& S, int kt, int buf, auto even_c) __attribute__((always_inline)) {
    constexpr bool kEven = decltype(even_c)::value;
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<u32x4_t*>(&sm.a[buf][xoff + 32 * j * BK]) = S.x[j];
    if constexpr (LISTS) {
      LutPlanes<4> pp;
      if constexpr (LUTM == kLutRow) {
        pp = pp_row;
      } else {
        pp.lo[0] = S.plo.x; pp.lo[1] = S.plo.y; pp.lo[2] = S.plo.z; pp.lo[3] = S.plo.w;
        pp.hi[0] = S.phi.x; pp.hi[1] = S.phi.y; pp.hi[2] = S.phi.z; pp.hi[3] = S.phi.w;
      }
      uint16_t* brow = &sm.b[buf][nl * BK];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        uint32_t o[4];
        dequant_word4s(S.cw[u], pp, o);
        *reinterpret_cast<u32x4_t*>(brow + 8 * ((4 * hh + u) ^ wsw)) = u32x4_t{o[0], o[1], o[2], o[3]};
      }
      return;
    }
    LutPlanes<BITS> pl;
    if constexpr (LUTM == kLutRow) {
      pl = pl_row;
    } else if constexpr (LUTM == kLutPair) {
      if constexpr (kEven) pl_pair = lut_planes<BITS>(S.lr);
      pl = pl_pair;
    } else {
      pl = lut_planes<BITS>(S.lr);
    }
    const int c0 = kt * BK + 32 * hh;
    uint16_t* brow = &sm.b[buf][nl * BK];
    static_for<0, 4>([&](auto u_c) __attribute__((always_inline)) {
      constexpr int U = decltype(u_c)::value;
      uint32_t o[4];
      dequant_unit<BITS, U>(S.cw, c0, pl, o);
      *reinterpret_cast<u32x4_t*>(brow + 8 * ((4 * hh + U) ^ wsw)) = u32x4_t{o[0], o[1], o[2], o[3]};
    });
  };

  auto direct_walk = [&](int ck, int lo, uint16_t* brow) __attribute__((always_inline)) {
    const int32_t* offr = a.offsets + (size_t)nb * (a.nch + 1);
    const int s1 = offr[ck + 1];
    for (int e = offr[ck]; e < s1; ++e) {
      const int col = (int)a.cols[e];
      if (col >= lo && col < lo + 32 && ck * a.chunk + col < a.K) {
        const int cs = col - lo;
        brow[8 * ((4 * hh + (cs >> 3)) ^ wsw) + (cs & 7)] = (uint16_t)((uint32_t)a.vals[e] << 8);
      }
    }
  };

  // Outliers of step (chunk ck, KIN columns into it, mask om) overwritten into the W tile in buf.
  auto store_outliers = [&](int ck, int buf, auto kin_c, auto prep) __attribute__((always_inline)) {
    constexpr int KIN = decltype(kin_c)::value;
    constexpr bool kPrep = decltype(prep)::value;
    const int lo = KIN + 32 * hh;  // my 32 columns inside the chunk
    uint16_t* brow = &sm.b[buf][nl * BK];
    if constexpr (kPrep) {
      if (__popc(om) <= kOlVals) {
        uint32_t m = om;
        int rank = 0;
        while (m != 0u) {
          const int cs = __builtin_ctz(m);  // column inside my 32
          m &= m - 1u;
          const uint32_t v = ((rank < 4 ? ov0 : ov1) >> (8 * (rank & 3))) & 0xFFu;
          ++rank;
          brow[8 * ((4 * hh + (cs >> 3)) ^ wsw) + (cs & 7)] = (uint16_t)(v << 8);
        }
      } else if (brow_ok) {
        direct_walk(ck, lo, brow);
      }
    } else if (brow_ok) {
      direct_walk(ck, lo, brow);
    }
  };

  // Patch of list entry pv over the W tile of step kt in buf (when it lies in the step's half of
  // its slab): lane = row % 16 + 16 (column / 32) of the slab, bits 6..10 the column % 32.
  auto apply_patch = [&](uint32_t pv, int kt, int buf) __attribute__((always_inline)) {
    const uint32_t l6 = pv & 63u;
    const uint32_t kq = l6 >> 4;
    if ((int)(kq >> 1) == (kt & 1)) {
      const uint32_t c32 = (pv >> 6) & 31u;
      const int nlr = 16 * li + (int)(l6 & 15u);
      sm.b[buf][nlr * BK + 8 * ((int)(4u * (kq & 1u) + (c32 >> 3)) ^ swz(nlr)) + (int)(c32 & 7u)] =
          (uint16_t)((pv >> 24) << 8);
    }
  };
  auto store_lists = [&](const StepRegs<BITS>& S, int kt, int buf) __attribute__((always_inline)) {
    if (S.pok != 0u) apply_patch(S.pe, kt, buf);
  };
  // Wave w writes the list starts of lists 2w, 2w + 1 (the lists its threads read; LDS keeps a
  // wave's accesses in order, so no barrier) and returns whether any of them is longer than 32
  // entries in some slab of the range.
  auto fill_lists = [&]() __attribute__((always_inline)) {
    const int wv = ptid >> 6;
    const int ln = ptid & 63;
    for (int i0 = 0; i0 < 2 * ntab; i0 += 512) {
      uint32_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = i0 + ln + 64 * j;
        const int l = 2 * wv + (i >= ntab ? 1 : 0);
        const int si = i >= ntab ? i - ntab : i;
        const int ptl = 8 * tn + l;
        v[j] = (i < 2 * ntab && ptl < a.T) ? a.wpidx[(size_t)ptl * a.S + min(s_first + si, a.S)] : 0u;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = i0 + ln + 64 * j;
        if (i < 2 * ntab) ltab[(2 * wv + (i >= ntab ? 1 : 0)) * ntab + (i >= ntab ? i - ntab : i)] = v[j];
      }
    }
    bool lng = false;
    for (int i = ln; i < 2 * ntab; i += 64) {
      const int l = 2 * wv + (i >= ntab ? 1 : 0);
      const int si = i >= ntab ? i - ntab : i;
      if (si + 1 < ntab && ltab[l * ntab + si + 1] - ltab[l * ntab + si] > 32u) lng = true;
    }
    return __builtin_amdgcn_ballot_w64(lng) != 0;
  };

  // Register sets: DIST steps of loads in flight (the sets rotate by step index; even
  // DIST keeps a set's step parity fixed, which the two-step group LUTs rely on).
  constexpr int DIST = (SPC % 4 == 0) ? 4 : 2;
  auto run = [&](auto mode_c) __attribute__((always_inline)) {
    constexpr int kMode = decltype(mode_c)::value;
    constexpr bool kPrep = HAS_CSR && kMode == kOlRecords;
    constexpr bool kLists = HAS_CSR && kMode == kOlLists;
    const std::integral_constant<bool, kPrep> prep{};
    const std::integral_constant<bool, kLists> lists{};
    StepRegs<BITS> rs[DIST];  // set d holds steps of index d (mod DIST) from the range start
    uint32_t pst = 0u, pcnt = 0u;  // list of the next step to load
    if constexpr (kPrep) ol_issue(ck_begin, std::integral_constant<int, 0>{});
    static_for<0, DIST>([&](auto d_c) __attribute__((always_inline)) {
      constexpr int d = decltype(d_c)::value;
      if constexpr (kLists) list_of(kt_begin + d, pst, pcnt);
      load_step(rs[d], kt_begin + d, std::integral_constant<bool, d % 2 == 0>{}, lists, pst, pcnt);
    });
    if constexpr (kLists) list_of(kt_begin + DIST, pst, pcnt);
    store_main(rs[0], kt_begin, 0, std::integral_constant<bool, true>{});
    if constexpr (kLists)
      store_lists(rs[0], kt_begin, 0);
    else if constexpr (HAS_CSR)
      store_outliers(ck_begin, 0, std::integral_constant<int, 0>{}, prep);
    // drain the prologue's loads once: the loop then starts from the same wait state as
    // its back edge, and the compiler does not add first-iteration waits to every trip
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt unconstrained (gfx9 encoding)
    __syncthreads();

    // One chunk per trip, its SPC steps unrolled.  Step s (the consumers run the MFMAs
    // of step kt meanwhile): loads of step kt+DIST, LDS stores of step kt+1 into the
    // other buffer, barrier.  The range's last step has no next step to stage; it loads the
    // DoRA operands instead (r <= kDrPre).
    auto chunk = [&](int c, auto nsteps_c) __attribute__((always_inline)) {
      const int kb = c * SPC;
      static_for<0, decltype(nsteps_c)::value>([&](auto s_c) __attribute__((always_inline)) {
        constexpr int s = decltype(s_c)::value;
        constexpr int buf = s & 1;
        const int kt = kb + s;
        if constexpr (kPrep)  // outlier record of the step staged below
          if (s + 1 < SPC || c + 1 < ck_end)
            ol_issue(s + 1 < SPC ? c : c + 1, std::integral_constant<int, (s + 1) % SPC>{});
        load_step(rs[s % DIST], kt + DIST, std::integral_constant<bool, s % 2 == 0>{}, lists, pst, pcnt);
        // keep the loads ahead of the stores of the other sets
        __builtin_amdgcn_sched_barrier(0);
        store_main(rs[(s + 1) % DIST], kt + 1, buf ^ 1, std::integral_constant<bool, (s + 1) % 2 == 0>{});
        if constexpr (kLists) {
          if (s + 1 < SPC || c + 1 < ck_end) store_lists(rs[(s + 1) % DIST], kt + 1, buf ^ 1);
          list_of(kt + DIST + 1, pst, pcnt);  // done by the barrier's wait
        } else if constexpr (HAS_CSR) {
          constexpr int KIN = ((s + 1) % SPC) * BK;
          if (s + 1 < SPC || c + 1 < ck_end)
            store_outliers(s + 1 < SPC ? c : c + 1, buf ^ 1, std::integral_constant<int, KIN>{}, prep);
        }
        __syncthreads();
      });
    };
    for (int c = ck_begin; c + 1 < ck_end; ++c) chunk(c, std::integral_constant<int, SPC>{});
    chunk(ck_end - 1, std::integral_constant<int, SPC - 1>{});
    if (pre) dora_pre();
    __syncthreads();
  };
  if (!has_work) {
    if (!dora) return;
  } else if constexpr (HAS_CSR && LISTS) {
    // a wave with a list longer than its 32 threads in some slab walks its rows' CSR entries
    if (fill_lists())
      run(std::integral_constant<int, kOlDirect>{});
    else
      run(std::integral_constant<int, kOlLists>{});
  } else if constexpr (HAS_CSR) {
    if (ol_mode == kOlRecords)
      run(std::integral_constant<int, kOlRecords>{});
    else
      run(std::integral_constant<int, kOlDirect>{});
  } else {
    run(std::integral_constant<int, kOlDirect>{});
  }
  if (!dora) return;
  // Staging, kDr ranks per round (the consumers read a round between two barriers).
  float* hs = reinterpret_cast<float*>(smem_raw) + ptid * kDhStride;
  uint16_t* bsr = reinterpret_cast<uint16_t*>(smem_raw + kDbOff) + (ptid >> 1) * kDbStride;
  const int m = m0 + ptid;
  const int nbr = n0 + (ptid >> 1);
  for (int c0 = 0; c0 < a.r; c0 += kDr) {
    if (c0 > 0) __syncthreads();  // the consumers read the previous round
    const int nr = (min(kDr, a.r - c0) + 15) & ~15;  // ranks staged this round (zeros past r)
    if (pre) {
#pragma unroll
      for (int k = 0; k < kDrPre; ++k) hs[k] = dh[k];
#pragma unroll
      for (int k = 0; k < kDrPre / 2; ++k) bsr[(kDrPre / 2) * (ptid & 1) + k] = db[k];
    } else {
      for (int k0 = 0; k0 < nr; k0 += 16) {
        float hv[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const int rk = c0 + k0 + k;
          const float v = a.H[(size_t)min(m, a.M - 1) * a.r + min(rk, a.r - 1)];
          hv[k] = (m < a.M && rk < a.r) ? v : 0.f;
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) hs[k0 + k] = hv[k];
      }
      const int half = nr / 2;
      for (int k0 = 0; k0 < half; k0 += 8) {
        uint16_t bv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const int rk = c0 + half * (ptid & 1) + k0 + k;
          const uint16_t v = a.B[(size_t)min(nbr, a.N - 1) * a.r + min(rk, a.r - 1)];
          bv[k] = (nbr < a.N && rk < a.r) ? v : (uint16_t)0;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) bsr[half * (ptid & 1) + k0 + k] = bv[k];
      }
    }
    if (c0 == 0 && ptid < BN)
      reinterpret_cast<uint16_t*>(smem_raw + kDgOff)[ptid] = n0 + ptid < a.N ? a.gamma[n0 + ptid] : (uint16_t)0;
    __syncthreads();  // round staged
  }
}

// Outlier records: one block per (N tile, chunk), one thread per GEMM producer thread (row
// ptid / 2 of the tile, columns 32 (ptid % 2) + [0, 32) of each 64-column step).  The thread walks
// its row's entries of the chunk, sets the mask bit of each one in its half (dropping chunk
// columns past the chunk and global columns past K, as the reference's dequant does) and stores
// its value at its rank among the set bits, so the values come out in (step, column) order
// whatever the entry order; a later duplicate of a column overwrites the earlier one.
__global__ __launch_bounds__(NP) void tile_entries_kernel(const int32_t* __restrict__ offsets,
                                                          const uint16_t* __restrict__ cols,
                                                          const uint8_t* __restrict__ vals, int N, int K, int nch,
                                                          int chunk, uint32_t* __restrict__ tent) {
  const int tn = blockIdx.x / nch;
  const int ck = blockIdx.x - tn * nch;
  const int t = threadIdx.x;
  const int n = tn * BN + (t >> 1);
  const int hh = t & 1;
  uint32_t mask[kOlSteps];
#pragma unroll
  for (int s = 0; s < kOlSteps; ++s) mask[s] = 0u;
  int o1 = 0, o2 = 0;
  if (n < N) {
    o1 = offsets[(size_t)n * (nch + 1) + ck];
    o2 = offsets[(size_t)n * (nch + 1) + ck + 1];
  }
  auto in_half = [&](int c) { return c < chunk && ck * chunk + c < K && ((c >> 5) & 1) == hh; };
  for (int e = o1; e < o2; ++e) {
    const int c = (int)cols[e];
    if (in_half(c)) {
      const uint32_t bit = 1u << (c & 31);
#pragma unroll
      for (int s = 0; s < kOlSteps; ++s)
        if ((c >> 6) == s) mask[s] |= bit;
    }
  }
  const int spc = chunk / BK;
  uint32_t* slot = tent + (size_t)blockIdx.x * ol_slot_words(spc);
  uint8_t* rv = reinterpret_cast<uint8_t*>(slot + spc * NP);  // [spc][NP][8] bytes
  for (int e = o1; e < o2; ++e) {
    const int c = (int)cols[e];
    if (in_half(c)) {
      const int s = c >> 6;
      const int b = c & 31;
      uint32_t ms = 0u;
#pragma unroll
      for (int q = 0; q < kOlSteps; ++q)
        if (q == s) ms = mask[q];
      const int rank = __popc(ms & ((1u << b) - 1u));  // set bits of the step below b
      if (rank < kOlVals) rv[((size_t)s * NP + t) * 8 + rank] = vals[e];
    }
  }
#pragma unroll
  for (int s = 0; s < kOlSteps; ++s)
    if (s < spc) slot[s * NP + t] = mask[s];
}

template <int BITS, int LUTM, bool HAS_CSR, bool X_VEC, bool LISTS = false>
hipError_t launch_variant(const GemmArgs& a, dim3 grid, hipStream_t stream) {
  auto* fn = gemm_kernel<BITS, LUTM, HAS_CSR, X_VEC, LISTS>;
  // > 64 KiB of LDS is requested once per kernel and device
  static uint64_t attr_set = 0;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  if (!(__atomic_load_n(&attr_set, __ATOMIC_ACQUIRE) & bit)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)(sizeof(GemmSmem) + kTabBytes));
    if (e != hipSuccess) return e;
    __atomic_fetch_or(&attr_set, bit, __ATOMIC_ACQ_REL);
  }
  const size_t lds = sizeof(GemmSmem) + (a.wpidx != nullptr ? kTabBytes : 0);
  hipLaunchKernelGGL(fn, grid, dim3(NT), lds, stream, a);
  return hipGetLastError();
}

template <int BITS, int LUTM, bool X_VEC>
hipError_t launch_csr(const GemmArgs& a, dim3 grid, hipStream_t stream) {
  if constexpr (X_VEC && (BITS == 4 || BITS == 3)) {  // prepared layers (3/4-bit): codes, planes, patch lists
    if (a.pcodes != nullptr) {
      if (a.has_csr && a.wpidx != nullptr) return launch_variant<BITS, LUTM, true, true, true>(a, grid, stream);
      if (!a.has_csr) return launch_variant<BITS, LUTM, false, true, true>(a, grid, stream);
    }
  }
  return a.has_csr ? launch_variant<BITS, LUTM, true, X_VEC>(a, grid, stream)
                   : launch_variant<BITS, LUTM, false, X_VEC>(a, grid, stream);
}

template <int BITS>
hipError_t launch_bits(const GemmArgs& a, int lutm, bool x_vec, dim3 grid, hipStream_t stream) {
  if (!x_vec)  // unaligned or ragged activations: generic loads, row or per-32-column group LUTs
    return lutm == kLutRow ? launch_csr<BITS, kLutRow, false>(a, grid, stream)
                           : launch_csr<BITS, kLutHalf, false>(a, grid, stream);
  switch (lutm) {
    case kLutRow: return launch_csr<BITS, kLutRow, true>(a, grid, stream);
    case kLutPair: return launch_csr<BITS, kLutPair, true>(a, grid, stream);
    case kLutStep: return launch_csr<BITS, kLutStep, true>(a, grid, stream);
    default: return launch_csr<BITS, kLutHalf, true>(a, grid, stream);
  }
}

hipError_t launch_any(const GemmArgs& a, int bits, int lutm, bool x_vec, dim3 grid, hipStream_t stream) {
  switch (bits) {
    case 1: return launch_bits<1>(a, lutm, x_vec, grid, stream);
    case 2: return launch_bits<2>(a, lutm, x_vec, grid, stream);
    case 3: return launch_bits<3>(a, lutm, x_vec, grid, stream);
    default: return launch_bits<4>(a, lutm, x_vec, grid, stream);
  }
}

}  // namespace

SplitPlan plan_gemm(const Layer& L, int M, int cu_count, size_t workspace_bytes, bool lists) {
  SplitPlan p{};
  const int ksteps = std::max(1, (L.K + BK - 1) / BK);
  const int spc = std::max(1, L.chunk / BK);
  const int nchunks = (ksteps + spc - 1) / spc;
  const long tiles = (long)((L.N + BN - 1) / BN) * (long)((M + BM - 1) / BM);
  const int target = std::max(1, cu_count);  // one 512-thread block per CU (LDS-bound)
  // per-call outlier records, when the workspace holds them (not with prepared patch lists)
  const size_t ent_bytes = (L.offsets != nullptr && !lists)
                               ? (size_t)((L.N + BN - 1) / BN) * (size_t)L.nch * ol_slot_words(spc) * sizeof(uint32_t)
                               : 0;
  const size_t ent_room = workspace_bytes >= ent_bytes ? ent_bytes : 0;
  int splits = 1;
  // Split K only while a whole extra round of tiles fits on the CUs: with one block per CU,
  // tiles >= CUs/2 gain nothing from splitting (the rounds stay the same) and pay the reduce.
  if (2 * tiles <= target) splits = (int)std::min<long>(target / tiles, kMaxSplits);
  splits = std::min(splits, nchunks);  // splits hold whole outlier chunks
  const size_t per_split = (size_t)M * (size_t)L.N * sizeof(float);
  while (splits > 1 && (size_t)splits * per_split + ent_room > workspace_bytes) --splits;
  const int cps = (nchunks + splits - 1) / splits;  // chunks per split
  const int kps = cps * spc;
  p.splits = (ksteps + kps - 1) / kps;
  p.slabs_per_split = kps;
  p.seg_slabs = 0;
  const size_t part_bytes = p.splits > 1 ? (size_t)p.splits * per_split : 0;
  p.aux_bytes = (part_bytes + ent_bytes <= workspace_bytes) ? ent_bytes : 0;
  p.workspace_bytes = part_bytes + p.aux_bytes;
  return p;
}

hipError_t launch_gemm(const Layer& L, const Dora& D, const uint16_t* X, uint16_t* out, int M,
                       const SplitPlan& plan, float* workspace, hipStream_t stream, const PatchLists* lists) {
  GemmArgs a{};
  a.q = L.q;
  a.lut = L.lut;
  a.X = X;
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
  a.ksteps_per_split = plan.slabs_per_split;
  a.splits = plan.splits;
  a.tiles_m = (M + BM - 1) / BM;
  a.tiles_n = (L.N + BN - 1) / BN;
  a.tiles = a.tiles_m * a.tiles_n;
  // buffer offsets are 32-bit: activations, codes and LUTs stay below 2^31 bytes
  const bool x_vec = (reinterpret_cast<uintptr_t>(X) & 15u) == 0 && (L.K % 8) == 0 && L.K >= 8 &&
                     ((size_t)M + BM) * (size_t)L.K * 2 < kOutOfRange;
  if ((size_t)L.N * L.wpr * 4 >= kOutOfRange || (size_t)L.N * L.ng * ((size_t)2 << L.bits) >= kOutOfRange)
    return hipErrorInvalidValue;
  if (L.chunk != (L.bits == 3 ? 640 : 512)) return hipErrorInvalidValue;
  if (L.group_size > 0 && L.ng > 1 && L.group_size % 32 != 0) return hipErrorInvalidValue;
  const size_t part_bytes = plan.splits > 1 ? (size_t)plan.splits * M * L.N * sizeof(float) : 0;
  a.tent = nullptr;
  a.wpidx = nullptr;
  a.wpatch = nullptr;
  a.pcodes = nullptr;
  a.pplanes = nullptr;
  if (lists != nullptr && (L.bits == 4 || L.bits == 3) && x_vec) {
    if (lists->T != (L.N + 15) / 16 || lists->S != (L.K + 127) / 128 ||
        (size_t)lists->T * lists->S * 1024 >= kOutOfRange || (size_t)lists->T * lists->ng * 512 >= kOutOfRange)
      return hipErrorInvalidValue;
    a.pcodes = lists->codes;
    a.pplanes = lists->planes;
    a.png = lists->ng;
    a.T = lists->T;
    a.S = lists->S;
  }
  if (a.has_csr && lists != nullptr && lists->nnz > 0) {
    // the list starts of a block's K range must fit the LDS table
    const int spc = L.chunk / BK;
    const int ksteps = (L.K + BK - 1) / BK;
    const int nchunks = (ksteps + spc - 1) / spc;
    const int cps = (plan.slabs_per_split + spc - 1) / spc;
    if (lists->T != (L.N + 15) / 16 || lists->S != (L.K + 127) / 128 || (size_t)lists->nnz * 4 >= kOutOfRange ||
        std::min(cps, nchunks) * (spc / 2) + 1 > kTabSlabs)
      return hipErrorInvalidValue;
    a.wpidx = lists->wpidx;
    a.wpatch = lists->wpatch;
    a.patch_bytes = (uint32_t)(lists->nnz * 4);
    a.T = lists->T;
    a.S = lists->S;
  } else if (a.has_csr && plan.aux_bytes > 0) {
    a.tent = reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(workspace) + part_bytes);
    hipLaunchKernelGGL(tile_entries_kernel, dim3(a.tiles_n * L.nch), dim3(NP), 0, stream, L.offsets, L.cols,
                       L.vals, L.N, L.K, L.nch, L.chunk, const_cast<uint32_t*>(a.tent));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const dim3 grid(a.tiles * plan.splits);
  const int G = L.group_size;
  const int lutm = (G <= 0 || L.ng == 1) ? kLutRow : (G % 128 == 0) ? kLutPair : (G % 64 == 0) ? kLutStep : kLutHalf;
  const hipError_t err = launch_any(a, L.bits, lutm, x_vec, grid, stream);
  if (err != hipSuccess) return err;
  if (plan.splits > 1) return launch_splitk_sum(workspace, plan.splits, M, L.N, out, stream);
  return hipSuccess;
}

}  // namespace wlq
