// Device code of the quantised matrix kernels: tiled-layout repack, exact
// dequantisation and the MFMA dequant-matvec with its fused prologues and
// epilogues.  Included by one translation unit per weight type.
//
// Arithmetic of the matvec.  cpu.go:164-215 computes, per row and per block of
// 32, s = sum_j (q_j - 8) x_j in f32 and then sum += d * s.  Here the block
// product runs on the matrix cores: the weights (q - 8, or q, or int8) are
// exact in f16; each activation is scaled by a power of two per token (so its
// largest magnitude sits in [2^14, 2^15)) and split exactly into
// hi = f16(x) and lo = f16(x - hi), two MFMA rows, 22 significant bits in
// all.  v_mfma_f32_16x16x32_f16 sums the 32 products of a block in f32 for 16
// rows at once; the block scale d is applied in f32 afterwards, as in the CPU
// path.  The result differs from the CPU path only by f32 rounding order
// (about 1e-7 relative), within the 1e-5 tolerance of the kernel sweep.
#pragma once

#include "gemv.h"
#include "wave.h"

namespace llmhip {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// F16ToF32 of f16.go:6-28 in integer operations: exact for every pattern,
// NaN payloads included.
__device__ __forceinline__ float f16_exact(uint32_t h) {
  uint32_t sign = (h >> 15) << 31, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
  if (exp == 0) {
    if (man == 0) return __uint_as_float(sign);
    uint32_t sh = __clz(man) - 21;  // shifts until bit 10 is set
    return __uint_as_float(sign | (113u - sh) << 23 | ((man << sh) & 0x3ff) << 13);
  }
  if (exp == 31) return __uint_as_float(sign | 0xffu << 23 | man << 13);
  return __uint_as_float(sign | (exp + 112u) << 23 | man << 13);
}

// The f16 bits of a scale as f32 through the hardware conversion (exact for
// every finite value, subnormals included).
__device__ __forceinline__ float f16_hw(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16 bytes of streamed weights: a non-temporal load (read once per pass).
__device__ __forceinline__ uint4 ld_stream16(const uint8_t* p) {
  u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return uint4{v[0], v[1], v[2], v[3]};
}


// f32(1 / sqrt(x)) of a double x (cpu.go:92-95: float32(1/math.Sqrt(...)))
// without the f64 divide and square-root sequences on the decode kernels'
// critical path: v_rsq_f64's estimate refined by two Newton steps in f64
// (each at least doubles its correct bits), then rounded to f32.  x > 0 and
// finite (the sum of squares plus eps); anything else takes the exact form.
__device__ __forceinline__ float rms_scale(double x) {
  if (!(x > 0.0 && x <= 1.7976931348623157e308)) return (float)(1.0 / sqrt(x));
  double y = __builtin_amdgcn_rsq(x);
  const double h = 0.5 * x;
  y = y * (1.5 - h * y * y);
  y = y * (1.5 - h * y * y);
  return (float)y;
}

// ------------------------------------------------------------ row maps

// (hd, the head size of a NEOX map, is a power of two: the model admits 64
// and 128; shifts instead of divisions)
__host__ __device__ inline uint32_t pos_of_row(uint32_t lr, uint32_t map, uint32_t hd, uint32_t seg0, uint32_t seg1,
                                               uint32_t ff) {
  if (map == MAP_NEOX && lr >= seg0 && lr < seg1) {
    uint32_t local = lr - seg0, h = local >> __builtin_ctz(hd), k = local & (hd - 1), hp = hd / 2;
    uint32_t side = k >= hp, i = side ? k - hp : k;
    return seg0 + h * hd + 16 * (i / 8) + (i % 8) + 8 * side;
  }
  if (map == MAP_GATEUP) {
    uint32_t side = lr >= ff, i = side ? lr - ff : lr;
    return 16 * (i / 8) + 8 * side + (i % 8);
  }
  return lr;
}

__host__ __device__ inline uint32_t row_of_pos(uint32_t p, uint32_t map, uint32_t hd, uint32_t seg0, uint32_t seg1,
                                               uint32_t ff) {
  if (map == MAP_NEOX && p >= seg0 && p < seg1) {
    uint32_t local = p - seg0, h = local >> __builtin_ctz(hd), w = local & (hd - 1), c = w % 16;
    return seg0 + h * hd + (c / 8) * (hd / 2) + 8 * (w / 16) + (c % 8);
  }
  if (map == MAP_GATEUP) {
    uint32_t c = p % 16;
    return (c / 8) * ff + 8 * (p / 16) + (c % 8);
  }
  return p;
}

// ------------------------------------------------------------- layout

template <uint32_t QT>
struct QT_ {
  static constexpr uint32_t BB = QT == LLMHIP_Q4_0 ? 18 : QT == LLMHIP_Q4_1 ? 20 : 34;  // GGUF bytes/block
  static constexpr uint32_t QB = QT == LLMHIP_Q8_0 ? 32 : 16;                          // quant bytes/block
  static constexpr uint32_t SB = QT == LLMHIP_Q4_1 ? 4 : 2;                            // scale bytes/block
  static constexpr uint32_t QO = QT == LLMHIP_Q4_1 ? 4 : 2;                            // quants offset in GGUF block
};

// Device layout of a quantised matrix, one buffer: tile t (16 rows of nb
// blocks, ng groups of 4 and a tail of nb % 4) at t * 16 * nb * (QB + SB),
// its quants then its scales.  Quants: group g is one QG-byte chunk in MFMA
// lane order (lane l = 16*w + r finds word w of each block of row r at 16*l;
// Q8: two 1 KiB halves, blocks 0-1 and 2-3, 8 bytes per block), the tail
// after the groups with `tail` words (Q8 pairs) per lane.  Scales:
// [group][row][block] f16 (Q4_1: d, m pairs), the tail's [row][block] last.
// A tile's bytes are contiguous, and so are its scales.  Device bytes equal
// GGUF bytes for rows % 16 == 0.
template <uint32_t QT>
struct Lay {
  static constexpr uint32_t QW = QT == LLMHIP_Q8_0 ? 2 : 1;  // quant words per block and lane
  static constexpr uint32_t QB = QT_<QT>::QB, SB = QT_<QT>::SB;
  static constexpr uint32_t QG = 1024 * QW;  // quant bytes of a group
  __host__ __device__ static uint64_t tile(uint64_t t, uint32_t nb) { return t * 16 * nb * (QB + SB); }
  // the 4 bytes (Q8: 8) lane word lw holds of block b, from the tile's start
  __host__ __device__ static uint32_t qoff(uint32_t b, uint32_t lw, uint32_t ng, uint32_t tail) {
    const uint32_t g = b / 4, j = b % 4;
    if (g < ng) return g * QG + (QT == LLMHIP_Q8_0 ? (j / 2) * 1024 + lw * 16 + (j % 2) * 8 : lw * 16 + j * 4);
    return ng * QG + (lw * tail + j) * 4 * QW;
  }
  // the scale of row r, block b, from the tile's start
  __host__ __device__ static uint32_t soff(uint32_t b, uint32_t r, uint32_t nb, uint32_t ng, uint32_t tail) {
    const uint32_t g = b / 4, j = b % 4;
    return 16 * nb * QB + (g < ng ? g * 64 * SB + (r * 4 + j) * SB : ng * 64 * SB + (r * tail + j) * SB);
  }
};

// One thread per GGUF block: scales verbatim, quants into MFMA lane order.
// Q8_0 bytes of k-group w are reordered to the element order the
// dequantiser produces (see dq8): word0 = e(4w), e(16+4w), e(4w+2),
// e(16+4w+2); word1 = e(4w+1), e(16+4w+1), e(4w+3), e(16+4w+3).
template <uint32_t QT>
__global__ void repack_kernel(const uint8_t* __restrict__ raw, uint64_t n, uint64_t blk0, uint64_t row_off,
                              uint8_t* __restrict__ wq, uint64_t tiles, uint32_t nb, uint32_t ng, uint32_t tail,
                              uint32_t map, uint32_t hd, uint32_t seg0, uint32_t seg1, uint32_t ff) {
  typedef QT_<QT> T;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint64_t gb = blk0 + i;
  uint32_t lr = (uint32_t)(row_off + gb / nb), b = (uint32_t)(gb % nb);
  uint32_t p = pos_of_row(lr, map, hd, seg0, seg1, ff), t = p / 16, r = p % 16;
  const uint8_t* blk = raw + i * T::BB;
  (void)tiles;
  uint8_t* tb = wq + Lay<QT>::tile(t, nb);
  uint8_t* sct = tb + Lay<QT>::soff(b, r, nb, ng, tail);
  for (uint32_t k = 0; k < T::SB; k++) sct[k] = blk[k];
  const uint8_t* q = blk + T::QO;
  if (QT == LLMHIP_Q8_0) {
    for (uint32_t w = 0; w < 4; w++) {
      uint32_t w0 = q[4 * w] | q[16 + 4 * w] << 8 | q[4 * w + 2] << 16 | (uint32_t)q[16 + 4 * w + 2] << 24;
      uint32_t w1 = q[4 * w + 1] | q[16 + 4 * w + 1] << 8 | q[4 * w + 3] << 16 | (uint32_t)q[16 + 4 * w + 3] << 24;
      uint8_t* o = tb + Lay<QT>::qoff(b, 16 * w + r, ng, tail);
      *(uint32_t*)o = w0;
      *(uint32_t*)(o + 4) = w1;
    }
  } else {
    for (uint32_t w = 0; w < 4; w++) {
      uint32_t word = q[4 * w] | q[4 * w + 1] << 8 | q[4 * w + 2] << 16 | (uint32_t)q[4 * w + 3] << 24;
      *(uint32_t*)(tb + Lay<QT>::qoff(b, 16 * w + r, ng, tail)) = word;
    }
  }
}

// The 32 f32 weights of block b of the row at tile position p, exactly as
// cpu.go forms them: d*f32(q-8) (Q4_0), d*f32(q)+m (Q4_1), d*f32(i8) (Q8_0).
template <uint32_t QT>
__device__ inline void dequant_block(const uint8_t* wq, uint64_t tiles, uint32_t nb, uint32_t ng, uint32_t tail,
                                     uint32_t p, uint32_t b, float* out) {
  (void)tiles;
  const uint32_t t = p / 16, r = p % 16;
  const uint8_t* tb = wq + Lay<QT>::tile(t, nb);
  const uint8_t* sct = tb + Lay<QT>::soff(b, r, nb, ng, tail);
  float d = f16_exact(sct[0] | sct[1] << 8);
  float m = 0;
  if (QT == LLMHIP_Q4_1) m = f16_exact(sct[2] | sct[3] << 8);
  for (uint32_t w = 0; w < 4; w++) {
    const uint8_t* o = tb + Lay<QT>::qoff(b, 16 * w + r, ng, tail);
    if (QT == LLMHIP_Q8_0) {
      uint32_t w0 = *(const uint32_t*)o, w1 = *(const uint32_t*)(o + 4);
      const uint32_t e0[4] = {4 * w, 16 + 4 * w, 4 * w + 2, 16 + 4 * w + 2};
      const uint32_t e1[4] = {4 * w + 1, 16 + 4 * w + 1, 4 * w + 3, 16 + 4 * w + 3};
      for (int i = 0; i < 4; i++) {
        out[e0[i]] = __fmul_rn(d, (float)(int8_t)(w0 >> (8 * i)));
        out[e1[i]] = __fmul_rn(d, (float)(int8_t)(w1 >> (8 * i)));
      }
    } else {
      uint32_t word = *(const uint32_t*)o;
      for (int i = 0; i < 4; i++) {
        uint32_t byte = (word >> (8 * i)) & 255u;
        int lo = byte & 15, hi = byte >> 4;
        if (QT == LLMHIP_Q4_0) {
          out[4 * w + i] = __fmul_rn(d, (float)(lo - 8));
          out[16 + 4 * w + i] = __fmul_rn(d, (float)(hi - 8));
        } else {
          out[4 * w + i] = __fadd_rn(__fmul_rn(d, (float)lo), m);
          out[16 + 4 * w + i] = __fadd_rn(__fmul_rn(d, (float)hi), m);
        }
      }
    }
  }
}

// out[lr][k] for every logical row; one thread per (row, block).
template <uint32_t QT>
__global__ void dequant_kernel(const uint8_t* __restrict__ wq, uint64_t tiles, uint32_t rows, uint32_t nb,
                               uint32_t ng, uint32_t tail, uint32_t map, uint32_t hd, uint32_t seg0, uint32_t seg1,
                               uint32_t ff, float* __restrict__ out) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (uint64_t)rows * nb) return;
  uint32_t lr = (uint32_t)(i / nb), b = (uint32_t)(i % nb);
  float v[32];
  dequant_block<QT>(wq, tiles, nb, ng, tail, pos_of_row(lr, map, hd, seg0, seg1, ff), b, v);
  float* o = out + (uint64_t)lr * nb * 32 + b * 32;
  for (int j = 0; j < 32; j++) o[j] = v[j];
}

// Embedding gather (kernels.go:19-73): x[t][:] = row tokens[state[1]+t].
template <uint32_t QT>
__global__ void embed_kernel(const uint8_t* __restrict__ wq, uint64_t tiles, uint32_t nb, uint32_t ng, uint32_t tail,
                             const int32_t* __restrict__ tokens, const uint32_t* __restrict__ state,
                             float* __restrict__ x) {
  uint32_t t = blockIdx.y;
  uint32_t row = (uint32_t)tokens[state[1] + t];
  for (uint32_t b = threadIdx.x; b < nb; b += blockDim.x) {
    float v[32];
    dequant_block<QT>(wq, tiles, nb, ng, tail, row, b, v);
    float* o = x + (uint64_t)t * nb * 32 + b * 32;
    for (int j = 0; j < 32; j++) o[j] = v[j];
  }
}

// ------------------------------------------------------------ dequantisers

// Word w of a Q4 block (byte i: element 4w+i low nibble, 16+4w+i high) as
// eight f16 weights in the order 4w, 4w+2, 16+4w, 16+4w+2, 4w+1, 4w+3,
// 16+4w+1, 16+4w+3.  0x6400|n is the f16 1024+n; a nibble in bits 4-7 gives
// 1024+16n, scaled back by 1/16.  Every step is exact.  The masks and the
// 0x6400 exponent are held in registers: gfx9's three-operand encoding takes
// no literal, so with literal constants each (w & mask) | 0x6400.. would be
// two instructions; from registers it is one v_and_or_b32 (the exponent bits
// and the masks do not overlap).
struct Dq4K {
  uint32_t m0, m1, magic;
};
__device__ __forceinline__ Dq4K dq4_consts() {
  Dq4K k{0x000F000Fu, 0x00F000F0u, 0x64006400u};
  // not volatile: identical copies merge and leave loops
  asm("" : "+s"(k.m0), "+s"(k.m1), "+v"(k.magic));
  return k;
}
template <bool Q41>
__device__ __forceinline__ h8 dq4k(uint32_t w, const Dq4K& k) {
  const h2 lo_off = Q41 ? h2{(_Float16)-1024, (_Float16)-1024} : h2{(_Float16)-1032, (_Float16)-1032};
  const h2 hi_off = Q41 ? h2{(_Float16)-64, (_Float16)-64} : h2{(_Float16)-72, (_Float16)-72};
  const h2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const uint32_t w8 = w >> 8;
  h2 a = as_h2((w & k.m0) | k.magic) + lo_off;
  h2 b = as_h2((w & k.m1) | k.magic) * s16 + hi_off;
  h2 c = as_h2((w8 & k.m0) | k.magic) + lo_off;
  h2 d = as_h2((w8 & k.m1) | k.magic) * s16 + hi_off;
  return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// The same with literal constants (measured faster in the decode tile kernel,
// whose per-unit code the register form reschedules for the worse).
template <bool Q41>
__device__ __forceinline__ h8 dq4(uint32_t w) {
  const h2 lo_off = Q41 ? h2{(_Float16)-1024, (_Float16)-1024} : h2{(_Float16)-1032, (_Float16)-1032};
  const h2 hi_off = Q41 ? h2{(_Float16)-64, (_Float16)-64} : h2{(_Float16)-72, (_Float16)-72};
  const h2 s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const uint32_t w8 = w >> 8;
  h2 a = as_h2((w & 0x000F000Fu) | 0x64006400u) + lo_off;
  h2 b = as_h2((w & 0x00F000F0u) | 0x64006400u) * s16 + hi_off;
  h2 c = as_h2((w8 & 0x000F000Fu) | 0x64006400u) + lo_off;
  h2 d = as_h2((w8 & 0x00F000F0u) | 0x64006400u) * s16 + hi_off;
  return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Two repacked Q8_0 words as eight f16 weights in the same element order:
// bytes 0 and 2 of a word form one pair, bytes 1 and 3 the other.  With
// the sign bit flipped a byte is i8+128; 0x64 above it gives 1024+i8+128.
__device__ __forceinline__ h8 dq8(uint32_t w0, uint32_t w1) {
  const h2 off = {(_Float16)-1152, (_Float16)-1152};
  uint32_t a = w0 ^ 0x80808080u, b = w1 ^ 0x80808080u;
  h2 p = as_h2(__builtin_amdgcn_perm(0x64646464u, a, 0x04020400u)) + off;
  h2 q = as_h2(__builtin_amdgcn_perm(0x64646464u, a, 0x04030401u)) + off;
  h2 r = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04020400u)) + off;
  h2 s = as_h2(__builtin_amdgcn_perm(0x64646464u, b, 0x04030401u)) + off;
  return h8{p[0], p[1], q[0], q[1], r[0], r[1], s[0], s[1]};
}

// ------------------------------------------------------------ reductions

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
// wave-uniform sum / max through DPP (whole wave active)
__device__ __forceinline__ float wave_sum_dpp(float v) { return rows_sum4(row_sum16(v)); }
__device__ __forceinline__ float wave_max_dpp(float v) { return rows_max4(row_max16(v)); }

// -------------------------------------------------------------- the kernel

constexpr int MAXI = 2;  // 8-element activation items staged per thread and token

// LDS layout of one launch (bytes).
struct Lds {
  uint32_t xs, misc, bsum, dx, part, total;
};

// q8: room for the activation block scales of PRO_Q8.
__host__ __device__ inline Lds lds_layout(int NT, uint32_t qtype, uint32_t nb, uint32_t waves, bool q8 = false) {
  Lds L;
  uint32_t o = 0;
  L.xs = o;
  o += nb * 4 * 2 * NT * 16;
  L.misc = o;
  o += 128 * 4;
  L.bsum = o;
  if (qtype == LLMHIP_Q4_1) o += nb * NT * 4;
  L.dx = o;
  if (q8) o += nb * NT * 4;
  L.part = o;
  o += waves * 64 * 2 * 4;
  L.total = o;
  return L;
}

// (value, index) order of greedy sampling: larger value, then lower index;
// an empty slot (index ~0u) always loses.
__device__ __forceinline__ bool amax_better(float v, uint32_t i, float bv, uint32_t bi) {
  return i != 0xffffffffu && (bi == 0xffffffffu || v > bv || (v == bv && i < bi));
}

// RoundF16 (f16.go): the binary16 nearest the f32 value v, ties to even,
// subnormals kept (v_cvt_f16_f32).  The empty asm makes v opaque, so the
// multiply or add that produced it cannot be fused with the conversion into
// one mixed-precision instruction (v_fma_mix*_f16), which would round the
// exact result to binary16 once instead of rounding the f32 value -- a
// different binary16 wherever the f32 value is a tie.
__device__ __forceinline__ _Float16 to_f16(float v) {
  asm volatile("" : "+v"(v));
  return (_Float16)v;
}

// One element into the KV cache: f32, or rounded to binary16 (RoundF16 of
// the F16KV mode, cpu.go:298-299).
__device__ __forceinline__ void kv_store(const GemvArgs& a, uint64_t i, float v) {
  if (a.kv16) ((_Float16*)a.kv)[i] = to_f16(v);
  else a.kv[i] = v;
}

// The inputs of a row's epilogue that do not depend on the product: the
// residual rows (EPI_ACC), the bias and the RoPE table entries (EPI_QKV).
// The decode kernel loads them before its prologue, so that their round trips
// (state, then the table) overlap the activation staging instead of following
// the product.
struct EpiIn {
  float yA = 0, yB = 0, bias = 0, cA = 0, sA = 0, cB = 0, sB = 0;
};

template <int EPI>
__device__ __forceinline__ EpiIn epi_load(const GemvArgs& a, uint32_t tile, int r, bool active, uint32_t tokA,
                                          bool okA, uint32_t tokB, bool okB) {
  EpiIn e;
  const uint32_t lr = row_of_pos(tile * 16 + r, a.map, a.map_hd, a.map_seg0, a.map_seg1, a.ff);
  if (!active || lr >= a.rows) return e;
  if (EPI == EPI_ACC) {
    const float* yr = a.yin ? a.yin : a.y;
    if (okA) e.yA = yr[(uint64_t)tokA * a.ldy + lr];
    if (okB) e.yB = yr[(uint64_t)tokB * a.ldy + lr];
  }
  if (EPI == EPI_QKV) {
    const uint32_t lf = a.row_base + lr;
    if (a.bias) e.bias = a.bias[lf];
    if (lf < a.nq + a.nk) {
      const uint32_t hd = a.hd, hp = hd / 2;
      const uint32_t j = lf < a.nq ? lf : lf - a.nq, w = j & (hd - 1);  // hd: 64 or 128
      const uint32_t i = a.neox ? w & (hp - 1) : w / 2;
      const uint32_t p0 = state_pos(a.state);
      if (okA) {
        const uint64_t o = ((uint64_t)(p0 + tokA) * hp + i) * 2;
        e.cA = a.cs[o];
        e.sA = a.cs[o + 1];
      }
      if (okB) {
        const uint64_t o = ((uint64_t)(p0 + tokB) * hp + i) * 2;
        e.cB = a.cs[o];
        e.sB = a.cs[o + 1];
      }
    }
  }
  return e;
}

// The per-row epilogue of both matrix kernels.  The lane holds row r of tile
// `tile` for two tokens of the launch (tokA, tokB; okA/okB say whether they
// exist), already unscaled; `pre` holds its epi_load inputs, or is null and
// they are loaded here.  Every lane of the wave must call it: the RoPE and
// SwiGLU epilogues exchange values between lanes.
template <int EPI>
__device__ __forceinline__ void row_epilogue(const GemvArgs& a, uint32_t tile, int r, bool active, uint32_t tokA,
                                             bool okA, float vA, uint32_t tokB, bool okB, float vB,
                                             const EpiIn* pre = nullptr, float* yo = nullptr) {
  const uint32_t lr = row_of_pos(tile * 16 + r, a.map, a.map_hd, a.map_seg0, a.map_seg1, a.ff);
  const bool rvalid = active && lr < a.rows;
  const EpiIn e = pre ? *pre : epi_load<EPI>(a, tile, r, active, tokA, okA, tokB, okB);
  if (EPI == EPI_SWIGLU) {
    // act = g / (1 + exp(-g)) * u (cpu.go:345) with g from the gate's own launch
    if (rvalid) {
      if (okA) {
        uint64_t o = (uint64_t)tokA * a.ldy + lr;
        float gg = a.aux[o];
        a.y[o] = gg / (1.f + __expf(-gg)) * vA;
        if (a.up) a.up[o] = vA;  // after the gate was read: up may alias aux
      }
      if (okB) {
        uint64_t o = (uint64_t)tokB * a.ldy + lr;
        float gg = a.aux[o];
        a.y[o] = gg / (1.f + __expf(-gg)) * vB;
        if (a.up) a.up[o] = vB;
      }
    }
  }
  if (EPI == EPI_STORE || EPI == EPI_ACC || EPI == EPI_ARGMAX) {
    float* Y = yo ? yo : a.y;  // yo: a k-part's own output row
    if (rvalid) {
      if (okA) Y[(uint64_t)tokA * a.ldy + lr] = EPI == EPI_ACC ? e.yA + vA : vA;
      if (okB) Y[(uint64_t)tokB * a.ldy + lr] = EPI == EPI_ACC ? e.yB + vB : vB;
    }
  }
  if (EPI == EPI_QKV) {
    // bias (qwen2), then RoPE of (q, k) pairs with the host table, then
    // K and V into the cache at pos (kernels_fused.go:47-73; cpu.go:284-303).
    // lf is the row in [q; k; v]; a launch may cover one of the three.
    const uint32_t lf = a.row_base + lr;
    if (a.bias && rvalid) {
      vA += e.bias;
      vB += e.bias;
    }
    const int pm = a.neox ? 8 : 1;
    float oA = __shfl_xor(vA, pm), oB = __shfl_xor(vB, pm);
    if (rvalid) {
      const uint32_t hd = a.hd, hp = hd / 2;
      const uint32_t p0 = state_pos(a.state);
      for (int u = 0; u < 2; u++) {
        if (!(u ? okB : okA)) continue;
        uint32_t tok = u ? tokB : tokA;
        float v = u ? vB : vA, o = u ? oB : oA;
        uint32_t pos = p0 + tok;
        if (lf < a.nq + a.nk) {
          uint32_t j = lf < a.nq ? lf : lf - a.nq, w = j & (hd - 1);  // hd: 64 or 128
          bool first = a.neox ? w < hp : (w % 2) == 0;
          const float c = u ? e.cB : e.cA, sn = u ? e.sB : e.sA;
          float x = first ? v : o, z = first ? o : v;
          float res = first ? __fsub_rn(__fmul_rn(x, c), __fmul_rn(z, sn))    // cpu.go:381
                            : __fadd_rn(__fmul_rn(x, sn), __fmul_rn(z, c));  // cpu.go:382
          if (lf < a.nq) a.y[(uint64_t)tok * a.nq + lf] = res;
          else kv_store(a, (uint64_t)pos * a.kvd + j, res);
        } else {
          kv_store(a, (uint64_t)a.ctx * a.kvd + (uint64_t)pos * a.kvd + (lf - a.nq - a.nk), v);
        }
      }
    }
  }
  if (EPI == EPI_GATEUP) {
    // act = g / (1 + exp(-g)) * u (cpu.go:345); gate row i at lane r, up row i at r+8
    // (lanes r >= 8 hold the up rows: with a.up they store them there, in the
    // same store instruction as the activations)
    float uA = __shfl_xor(vA, 8), uB = __shfl_xor(vB, 8);
    const uint32_t i = 8 * tile + (r & 7);
    float* dst = r < 8 ? a.y : a.up;
    if (active && i < a.ff && dst) {
      if (okA) dst[(uint64_t)tokA * a.ff + i] = r < 8 ? vA / (1.f + __expf(-vA)) * uA : vA;
      if (okB) dst[(uint64_t)tokB * a.ff + i] = r < 8 ? vB / (1.f + __expf(-vB)) * uB : vB;
    }
  }
}

// Activations of nt tokens staged once per workgroup (the prologue of both
// matrix-vector kernels): one round of global loads of items (block b,
// k-group g) of 8 elements (4g..4g+3 and 16+4g..16+4g+3), RMSNorm for PRO_RMS
// (cpu.go:90-96), then per token a power-of-two scale 2^ex[t] (largest
// magnitude in [2^14, 2^15)) and the split into f16 hi + lo, stored in MFMA
// operand order.  Per-wave partials go through LDS; every thread then
// finishes each reduction itself (the same sums in the same order).  Ends
// with a barrier after which xs (and bsum, Q4_1) are complete.
//
// PRO_Q8 (ExactGGML): after the RMSNorm each block of 32 is quantised as
// quantizeQ8 does (cpu.go:117-140): d = amax / 127, q = round half away from
// zero of x * (1/d), in f32; hi = q (exact in f16), lo = 0, no scale (ex = 0);
// dxs[t][b] = RoundF16(d) and, for Q4_1, bsum[t][b] = RoundF16(d * sum q).
//
// stage_x in two steps: its loads (the activation items and, PRO_RMS, the
// norm weights), then the rest from the loaded values, so that a caller can
// issue other loads in between (vector loads return in issue order: loads
// issued before the activations would hold up the staging).
template <int NT>
struct XItems {
  f4 va[NT][MAXI], vc[NT][MAXI], wa[MAXI], wc[MAXI];
};

template <int NT, int PRO>
__device__ __forceinline__ void stage_x_load(const GemvArgs& a, uint32_t t0, int nt, XItems<NT>& xi) {
  const uint32_t bd = blockDim.x;
  const int tid = threadIdx.x;
  const uint32_t NI = a.nb * 4;
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int k = 0; k < MAXI; k++) {
      uint32_t it = tid + k * bd;
      f4 A = {0, 0, 0, 0}, C = {0, 0, 0, 0};
      if (t < nt && it < NI) {
        const float* xr = a.x + (uint64_t)(a.xrow0 + t0 + t) * a.ldx + (it / 4) * 32 + 4 * (it % 4);
        A = *(const f4*)xr;
        C = *(const f4*)(xr + 16);
      }
      xi.va[t][k] = A;
      xi.vc[t][k] = C;
    }
  if (PRO & PRO_RMS) {
#pragma unroll
    for (int k = 0; k < MAXI; k++) {
      uint32_t it = tid + k * bd;
      xi.wa[k] = xi.wc[k] = f4{0, 0, 0, 0};
      if (it < NI) {
        const float* wr = a.nw + (it / 4) * 32 + 4 * (it % 4);
        xi.wa[k] = *(const f4*)wr;
        xi.wc[k] = *(const f4*)(wr + 16);
      }
    }
  }
}

template <uint32_t QT, int NT, int PRO>
__device__ __forceinline__ void stage_x_from(const GemvArgs& a, int nt, XItems<NT>& xi, h8* xs, float* misc,
                                             float* bsum, float* dxs, int ex[NT]) {
  constexpr int S = 2 * NT;
  const uint32_t bd = blockDim.x, nwv = bd >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const uint32_t nb = a.nb, K = a.k, NI = nb * 4;
  f4(&va)[NT][MAXI] = xi.va;
  f4(&vc)[NT][MAXI] = xi.vc;
  if (PRO & PRO_RMS) {
    // ss = sum x^2 (f32); s = f32(1/sqrt(f64(ss/n + eps))); h = x*s*w
    const f4(&wa)[MAXI] = xi.wa;
    const f4(&wc)[MAXI] = xi.wc;
#pragma unroll
    for (int t = 0; t < NT; t++) {
      float ss = 0;
#pragma unroll
      for (int k = 0; k < MAXI; k++)
        for (int i = 0; i < 4; i++) ss += va[t][k][i] * va[t][k][i] + vc[t][k][i] * vc[t][k][i];
      ss = wave_sum_dpp(ss);
      if (lane == 0) misc[wave * NT + t] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; t++) {
      float ss = 0;
      for (uint32_t w = 0; w < nwv; w++) ss += misc[w * NT + t];
      const float s = t < nt ? (float)(1.0 / sqrt((double)(ss / (float)K + a.eps))) : 0.f;
#pragma unroll
      for (int k = 0; k < MAXI; k++)
        for (int i = 0; i < 4; i++) {
          va[t][k][i] = __fmul_rn(__fmul_rn(va[t][k][i], s), wa[k][i]);  // cpu.go:96
          vc[t][k][i] = __fmul_rn(__fmul_rn(vc[t][k][i], s), wc[k][i]);
        }
    }
  }
  if (PRO & PRO_Q8) {
    // a block's four items sit in four consecutive lanes: its max and its
    // sum of q are two xor-shuffles
#pragma unroll
    for (int t = 0; t < NT; t++) {
      ex[t] = 0;
#pragma unroll
      for (int k = 0; k < MAXI; k++) {
        const uint32_t it = tid + k * bd;
        const f4 A = va[t][k], C = vc[t][k];
        float am = 0;
        for (int i = 0; i < 4; i++) am = fmaxf(am, fmaxf(fabsf(A[i]), fabsf(C[i])));
        am = fmaxf(am, __shfl_xor(am, 1));
        am = fmaxf(am, __shfl_xor(am, 2));
        const float d = __fdiv_rn(am, 127.f);
        const float id = d != 0.f ? __fdiv_rn(1.f, d) : 0.f;
        const float v[8] = {A[0], A[2], C[0], C[2], A[1], A[3], C[1], C[3]};
        h8 hi;
        int qs = 0;
        for (int i = 0; i < 8; i++) {
          const float qv = roundf(__fmul_rn(v[i], id));
          hi[i] = (_Float16)qv;
          qs += (int)qv;
        }
        qs += __shfl_xor(qs, 1);
        qs += __shfl_xor(qs, 2);
        if (it < NI) {
          xs[it * S + 2 * t] = hi;
          xs[it * S + 2 * t + 1] = h8{};
          if ((it & 3) == 0) {
            dxs[t * nb + it / 4] = (float)to_f16(d);
            if (QT == LLMHIP_Q4_1) bsum[t * nb + it / 4] = (float)to_f16(__fmul_rn(d, (float)qs));
          }
        }
      }
    }
    __syncthreads();
    return;
  }
  float* mpart = misc + 64;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    float m = 0;
#pragma unroll
    for (int k = 0; k < MAXI; k++)
      for (int i = 0; i < 4; i++) m = fmaxf(m, fmaxf(fabsf(va[t][k][i]), fabsf(vc[t][k][i])));
    m = wave_max_dpp(m);
    if (lane == 0) mpart[wave * NT + t] = m;
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < NT; t++) {
    float m = 0;
    for (uint32_t w = 0; w < nwv; w++) m = fmaxf(m, mpart[w * NT + t]);
    int e = 0;
    if (t < nt && m > 0 && m <= 3.0e38f) {
      int E;
      frexpf(m, &E);
      e = 15 - E;
    }
    ex[t] = e;
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
#pragma unroll
    for (int k = 0; k < MAXI; k++) {
      uint32_t it = tid + k * bd;
      if (it >= NI) continue;
      const f4 A = va[t][k], C = vc[t][k];
      const float v[8] = {A[0], A[2], C[0], C[2], A[1], A[3], C[1], C[3]};
      h8 hi, lo;
      for (int i = 0; i < 8; i++) {
        float s = ldexpf(v[i], ex[t]);
        _Float16 h = (_Float16)s;
        hi[i] = h;
        lo[i] = (_Float16)(s - (float)h);
      }
      xs[it * S + 2 * t] = hi;
      xs[it * S + 2 * t + 1] = lo;
      if (QT == LLMHIP_Q4_1) {
        // block sums sum_j x_j (cpu.go:196-198), scaled like the operand
        float sx = (A[0] + A[1] + A[2] + A[3]) + (C[0] + C[1] + C[2] + C[3]);
        sx += __shfl_xor(sx, 1);
        sx += __shfl_xor(sx, 2);
        if ((it & 3) == 0) bsum[t * nb + it / 4] = ldexpf(sx, ex[t]);
      }
    }
  }
  __syncthreads();
}

template <uint32_t QT, int NT, int PRO>
__device__ __forceinline__ void stage_x(const GemvArgs& a, uint32_t t0, int nt, h8* xs, float* misc, float* bsum,
                                        float* dxs, int ex[NT]) {
  XItems<NT> xi;
  stage_x_load<NT, PRO>(a, t0, nt, xi);
  stage_x_from<QT, NT, PRO>(a, nt, xi, xs, misc, bsum, dxs, ex);
}

// One unit of a tile's weights in registers: a group of four blocks (Q4: w0
// holds the lane's word of each block; Q8: w0, w1 two words of blocks 0,1 and
// 2,3; sv the scales of row r) or the tail of nb % 4 blocks (component j of
// w0 / w1 / sv for tail block j).
struct WUnit {
  uint4 w0, w1, sv;
};

// Load group g (< ng) of tile t of the matrix at wq.  The layer matrices use
// ordinary (cacheable) loads; the streaming kernel's are non-temporal, so the
// one-pass read of the vocabulary head does not push the layers out of cache.
// With `real` false the unit is not needed: every lane reads the tile's first
// bytes (one cache line), so the load stays unconditional and costs nothing.
template <uint32_t QT, bool STREAM = false, bool SCALES = true>
__device__ __forceinline__ void load_group(WUnit& u, const uint8_t* wq, uint32_t nb, uint32_t t, uint32_t g,
                                           int lane, int r, bool real = true) {
  typedef Lay<QT> LY;
  const uint8_t* tb = wq + LY::tile(t, nb);
  const uint32_t ql = real ? g * LY::QG + lane * 16 : 0;
  if (STREAM) {
    u.w0 = ld_stream16(tb + ql);
    if (QT == LLMHIP_Q8_0) u.w1 = ld_stream16(tb + ql + (real ? 1024 : 0));
  } else {
    u.w0 = *(const uint4*)(tb + ql);
    if (QT == LLMHIP_Q8_0) u.w1 = *(const uint4*)(tb + ql + (real ? 1024 : 0));
  }
  if (!SCALES) return;
  const uint8_t* sp = tb + (real ? 16 * nb * LY::QB + g * 64 * LY::SB + r * 4 * LY::SB : 0);
  if (QT == LLMHIP_Q4_1) {
    u.sv = *(const uint4*)sp;
  } else {
    uint2 x2 = *(const uint2*)sp;
    u.sv = uint4{x2.x, x2.y, 0, 0};
  }
}

// The scales of groups 4h .. 4h+3 of tile t (no tail blocks), one load for
// four groups: lane L holds row L % 16 of group 4h + L / 16 (groups past
// NG - 1 read group NG - 1 again).  `real` false: one lane-invariant line.
template <uint32_t QT, int NG>
__device__ __forceinline__ uint4 load_scales4(const uint8_t* wq, uint32_t nb, uint32_t t, int h, int lane,
                                              bool real) {
  typedef Lay<QT> LY;
  constexpr uint32_t SR = 4 * LY::SB;  // one row's scale bytes in a group
  const uint32_t g = min(4 * h + (lane >> 4), NG - 1);
  const uint8_t* sp = wq + LY::tile(t, nb) + (real ? 16 * nb * LY::QB + g * 16 * SR + (lane & 15) * SR : 0);
  if (SR == 16) return *(const uint4*)sp;
  const uint2 x = *(const uint2*)sp;
  return uint4{x.x, x.y, 0, 0};
}

// Group g's scales of row r, as load_group leaves them in WUnit::sv, from
// the four-group load that holds them (lane 16 (g % 4) + r).
template <uint32_t QT>
__device__ __forceinline__ uint4 group_scales(const uint4& s4, int g, int r) {
  const int src = (16 * (g & 3) + r) * 4;
  uint4 v;
  v.x = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)s4.x);
  v.y = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)s4.y);
  v.z = QT == LLMHIP_Q4_1 ? (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)s4.z) : 0u;
  v.w = QT == LLMHIP_Q4_1 ? (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)s4.w) : 0u;
  return v;
}

// Load unit g (< ng: a group, == ng: the tail) of tile t of the matrix at wq.
template <uint32_t QT, bool STREAM = false>
__device__ __forceinline__ void load_unit(WUnit& u, const uint8_t* wq, uint32_t nb, uint32_t t, uint32_t g,
                                          uint32_t ng, uint32_t tail, int lane, int r) {
  typedef Lay<QT> LY;
  if (g < ng) {
    load_group<QT, STREAM>(u, wq, nb, t, g, lane, r);
    return;
  }
  const uint8_t* tb = wq + LY::tile(t, nb);
  uint32_t q0[3] = {0, 0, 0}, q1[3] = {0, 0, 0}, s[3] = {0, 0, 0};
#pragma unroll
  for (uint32_t j = 0; j < 3; j++) {
    if (j >= tail) continue;
    const uint32_t b = 4 * ng + j;
    const uint8_t* qq = tb + LY::qoff(b, lane, ng, tail);
    q0[j] = *(const uint32_t*)qq;
    if (QT == LLMHIP_Q8_0) q1[j] = *(const uint32_t*)(qq + 4);
    const uint8_t* sp = tb + LY::soff(b, r, nb, ng, tail);
    s[j] = QT == LLMHIP_Q4_1 ? *(const uint32_t*)sp : (uint32_t)*(const uint16_t*)sp;
  }
  u.w0 = uint4{q0[0], q0[1], q0[2], 0};
  u.w1 = uint4{q1[0], q1[1], q1[2], 0};
  u.sv = uint4{s[0], s[1], s[2], 0};
}

// One block through the MFMA: D[token slot][row] = x_slot . w_row over its 32
// elements, then acc += d * (hi + lo) (and m * sum x for Q4_1).  Q8: the
// activations are Q8 blocks (hi = q, lo = 0), D is ggml's integer block sum,
// exact in f32 (at most 32 * 128 * 127 in magnitude), and the block adds
// d_w * d_x * f32(sum) (+ m_w * s_x), rounded as cpu.go:174-210 rounds it.
template <uint32_t QT, int NT, bool Q8>
__device__ __forceinline__ void mfma_block(const h8* xs, const float* bsum, const float* dxs, uint32_t nb, int q,
                                           int slot, uint32_t b, h8 B, uint32_t dbits, uint32_t mbits, float& acc0,
                                           float& acc1) {
  // Branch-free (a clamped read, then a select) so that the blocks of a unit
  // form one basic block and their LDS reads and MFMAs overlap.
  constexpr int S = 2 * NT;
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  const u4v X = __builtin_bit_cast(u4v, xs[(b * 4 + q) * S + min(slot, S - 1)]);
  const h8 A = __builtin_bit_cast(h8, X & (slot < S ? ~0u : 0u));
  f4 D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, f4{0, 0, 0, 0}, 0, 0, 0);
  float d = f16_hw(dbits);
  if (Q8) {
    const int tA = min(2 * q, NT - 1), tB = min(2 * q + 1, NT - 1);
    float pA = __fmul_rn(__fmul_rn(d, dxs[tA * nb + b]), D[0] + D[1]);
    float pB = __fmul_rn(__fmul_rn(d, dxs[tB * nb + b]), D[2] + D[3]);
    if (QT == LLMHIP_Q4_1) {
      const float m = f16_hw(mbits);
      pA = __fadd_rn(pA, __fmul_rn(m, bsum[tA * nb + b]));
      pB = __fadd_rn(pB, __fmul_rn(m, bsum[tB * nb + b]));
    }
    acc0 += 2 * q < NT ? pA : 0.f;
    if (NT > 1) acc1 += 2 * q + 1 < NT ? pB : 0.f;
    return;
  }
  acc0 += d * (D[0] + D[1]);
  if (NT > 1) acc1 += d * (D[2] + D[3]);
  if (QT == LLMHIP_Q4_1) {
    const float m = f16_hw(mbits);
    const float s0 = bsum[min(2 * q, NT - 1) * nb + b], s1 = bsum[min(2 * q + 1, NT - 1) * nb + b];
    acc0 += 2 * q < NT ? m * s0 : 0.f;
    acc1 += 2 * q + 1 < NT ? m * s1 : 0.f;
  }
}

// The four blocks of group g of a tile (see WUnit).
template <uint32_t QT, int NT, bool Q8 = false>
__device__ __forceinline__ void group_mfma(const WUnit& u, uint32_t g, const h8* xs, const float* bsum,
                                           const float* dxs, uint32_t nb, int q, int slot, float& acc0, float& acc1) {
  {
    const uint32_t b0 = 4 * g;
    if (QT == LLMHIP_Q8_0) {
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 0, dq8(u.w0.x, u.w0.y), u.sv.x & 0xffff, 0, acc0, acc1);
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 1, dq8(u.w0.z, u.w0.w), u.sv.x >> 16, 0, acc0, acc1);
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 2, dq8(u.w1.x, u.w1.y), u.sv.y & 0xffff, 0, acc0, acc1);
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 3, dq8(u.w1.z, u.w1.w), u.sv.y >> 16, 0, acc0, acc1);
    } else if (QT == LLMHIP_Q4_1) {
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 0, dq4<true>(u.w0.x), u.sv.x & 0xffff, u.sv.x >> 16,
                             acc0, acc1);
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 1, dq4<true>(u.w0.y), u.sv.y & 0xffff, u.sv.y >> 16,
                             acc0, acc1);
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 2, dq4<true>(u.w0.z), u.sv.z & 0xffff, u.sv.z >> 16,
                             acc0, acc1);
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 3, dq4<true>(u.w0.w), u.sv.w & 0xffff, u.sv.w >> 16,
                             acc0, acc1);
    } else {
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 0, dq4<false>(u.w0.x), u.sv.x & 0xffff, 0, acc0, acc1);
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 1, dq4<false>(u.w0.y), u.sv.x >> 16, 0, acc0, acc1);
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 2, dq4<false>(u.w0.z), u.sv.y & 0xffff, 0, acc0, acc1);
      mfma_block<QT, NT, Q8>(xs, bsum, dxs, nb, q, slot, b0 + 3, dq4<false>(u.w0.w), u.sv.y >> 16, 0, acc0, acc1);
    }
  }
}

// group_mfma for one token with f32 activations whose MFMA operands are
// already in registers (xa: the group's four blocks, slots past hi/lo zero).
// Only lanes of q == 0 hold the token's sums; the others accumulate values
// the epilogue drops, so no per-lane selects.
template <uint32_t QT, int XS = 1>
__device__ __forceinline__ void group_pre(const WUnit& u, uint32_t g, const h8* xa, const float* bsum,
                                          const Dq4K& K, float& acc) {
  auto blk = [&](int j, h8 B, uint32_t dbits, uint32_t mbits) {
    const f4 D = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[j * XS], B, f4{0, 0, 0, 0}, 0, 0, 0);
    acc += f16_hw(dbits) * (D[0] + D[1]);
    if (QT == LLMHIP_Q4_1) acc += f16_hw(mbits) * bsum[4 * g + j];
  };
  if (QT == LLMHIP_Q8_0) {
    blk(0, dq8(u.w0.x, u.w0.y), u.sv.x & 0xffff, 0);
    blk(1, dq8(u.w0.z, u.w0.w), u.sv.x >> 16, 0);
    blk(2, dq8(u.w1.x, u.w1.y), u.sv.y & 0xffff, 0);
    blk(3, dq8(u.w1.z, u.w1.w), u.sv.y >> 16, 0);
  } else if (QT == LLMHIP_Q4_1) {
    blk(0, dq4k<true>(u.w0.x, K), u.sv.x & 0xffff, u.sv.x >> 16);
    blk(1, dq4k<true>(u.w0.y, K), u.sv.y & 0xffff, u.sv.y >> 16);
    blk(2, dq4k<true>(u.w0.z, K), u.sv.z & 0xffff, u.sv.z >> 16);
    blk(3, dq4k<true>(u.w0.w, K), u.sv.w & 0xffff, u.sv.w >> 16);
  } else {
    blk(0, dq4k<false>(u.w0.x, K), u.sv.x & 0xffff, 0);
    blk(1, dq4k<false>(u.w0.y, K), u.sv.x >> 16, 0);
    blk(2, dq4k<false>(u.w0.z, K), u.sv.y & 0xffff, 0);
    blk(3, dq4k<false>(u.w0.w, K), u.sv.y >> 16, 0);
  }
}

// ---- the streaming kernel's products on the integer matrix cores
// (v_mfma_i32_16x16x64_i8; f32 activations, k = 896: seven groups per tile).
// The staged activation x_s = hi + lo (stage_x_from: max |x_s| in
// [2^14, 2^15)) becomes the integer x_i = round(128 x_s) (|x_i| < 2^22) and
// three balanced int8 digits, x_i = a 2^16 + b 2^8 + c, b and c in
// [-128, 127], a in [-65, 65].  The weights enter as int8 (Q8_0 as stored;
// Q4_0 and Q4_1 nibbles masked out of the lane's words: element 4q + i of a
// block in the low nibble of byte i of word q, element 16 + 4q + i in its high
// nibble).  One MFMA takes two blocks of a group: lane (r, q) holds 8 weights
// of each (16 k-slots), and A row 4j + p holds digit p of block j's
// activations at block j's slots (zero elsewhere), so after the group's two
// MFMAs lane (r, q) holds block q's three digit sums of row r, each exact in
// i32.  Per block: D_p - 8 S_p (Q4_0's offset of 8, with S_p the block's sum
// of digits p: exact in integers), the digits recombined in f32, times the
// block's scale d; Q4_1 adds m sum(x).  The products are exact; the roundings
// are x_i's (2^-23 of the row's largest |x|) and the f32 sums.

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// LDS bytes the integer form adds to the streaming kernel's layout: the
// digits (per block, digit and k-group: 8 bytes) and the per-block offsets.
__host__ __device__ constexpr uint32_t i8_lds_bytes(uint32_t nb) { return nb * (3 * 4 * 8 + 16); }

// The digits of the staged items, by the whole workgroup (one thread per
// item: a block's four items on four consecutive lanes), into dg[(b 3 + p) 4 + q]
// (8 bytes: the item's elements in the order of the lane's int8 weights) and
// tb[b] = (8 S_0, 8 S_1, 8 S_2, 8 (S_0 2^16 + S_1 2^8 + S_2) modulo 2^32) for
// Q4_0 (zeros for the other types).  Ends with a barrier.
template <uint32_t QT>
__device__ __forceinline__ void stage_digits(const h8* xs, uint32_t nb, uint64_t* dg, i32x4* tb) {
  const uint32_t NI = nb * 4;
  for (uint32_t i0 = 0; i0 < NI; i0 += blockDim.x) {
    const uint32_t it = i0 + threadIdx.x, ic = min(it, NI - 1);
    const h8 hi = xs[2 * ic], lo = xs[2 * ic + 1];
    // item order (stage_x_from): e(4q), e(4q+2), e(16+4q), e(16+4q+2), e(4q+1), e(4q+3), e(16+4q+1), e(16+4q+3);
    // the int8 weights' order: Q4 e(4q..4q+3), e(16+4q..16+4q+3); Q8_0 the repacked bytes
    // e(4q), e(16+4q), e(4q+2), e(16+4q+2), e(4q+1), e(16+4q+1), e(4q+3), e(16+4q+3)
    constexpr int O4[8] = {0, 4, 1, 5, 2, 6, 3, 7}, O8[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    uint32_t w[3][2] = {{0, 0}, {0, 0}, {0, 0}};
    int sd[3] = {0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int e = QT == LLMHIP_Q8_0 ? O8[i] : O4[i];
      const int v = (int)rintf(((float)hi[e] + (float)lo[e]) * 128.f);
      const int c = (int)(int8_t)(v & 0xff), t = (v - c) >> 8;
      const int b = (int)(int8_t)(t & 0xff), a = (t - b) >> 8;
      const int dgt[3] = {a, b, c};
#pragma unroll
      for (int p = 0; p < 3; p++) {
        w[p][i / 4] |= (uint32_t)(dgt[p] & 0xff) << (8 * (i % 4));
        sd[p] += dgt[p];
      }
    }
#pragma unroll
    for (int p = 0; p < 3; p++) {
      sd[p] += __shfl_xor(sd[p], 1);
      sd[p] += __shfl_xor(sd[p], 2);
    }
    if (it < NI) {
      const uint32_t blk = it / 4, q = it % 4;
#pragma unroll
      for (int p = 0; p < 3; p++) dg[(blk * 3 + p) * 4 + q] = (uint64_t)w[p][0] | (uint64_t)w[p][1] << 32;
      // the last word: the three offsets recombined (modulo 2^32), as group_i8 subtracts them
      const uint32_t tc = ((uint32_t)(8 * sd[0]) << 16) + ((uint32_t)(8 * sd[1]) << 8) + (uint32_t)(8 * sd[2]);
      if (q == 0)
        tb[blk] = QT == LLMHIP_Q4_0 ? i32x4{8 * sd[0], 8 * sd[1], 8 * sd[2], (int32_t)tc} : i32x4{0, 0, 0, 0};
    }
  }
  __syncthreads();
}

// Lane (m, kq)'s A operands of group g's two MFMAs: row m = 4 j + p holds
// digit p (< 3) of block 4 g + j at block j's k-slots (MFMA j / 2, its
// 8-byte half j % 2), zero elsewhere.
__device__ __forceinline__ void i8_operands(const uint64_t* dg, uint32_t g, int lane, i32x4 (&xa)[2]) {
  const uint32_t m = lane & 15, kq = lane >> 4, j = m / 4, p = m % 4;
  const uint64_t v = dg[((4 * g + j) * 3 + min(p, 2u)) * 4 + kq];
  const int32_t lo = p < 3 ? (int32_t)(uint32_t)v : 0, hi = p < 3 ? (int32_t)(uint32_t)(v >> 32) : 0;
#pragma unroll
  for (uint32_t h = 0; h < 2; h++) {
    const bool use = j / 2 == h;
    xa[h] = (j % 2 == 0) ? i32x4{use ? lo : 0, use ? hi : 0, 0, 0} : i32x4{0, 0, use ? lo : 0, use ? hi : 0};
  }
}

// One group of a tile on the integer matrix cores: acc (lane (r, q)) +=
// block 4 g + q's product for row r, times 2^(ex + 7).  T: that block's
// offsets (tb), bsq: Q4_1's 128 sum(x_s) of the block.
template <uint32_t QT>
__device__ __forceinline__ void group_i8(const WUnit& u, const i32x4 (&xa)[2], const i32x4& T, float bsq, int q,
                                         float& acc) {
  i32x4 B0, B1;
  if (QT == LLMHIP_Q8_0) {
    B0 = __builtin_bit_cast(i32x4, u.w0);
    B1 = __builtin_bit_cast(i32x4, u.w1);
  } else {
    auto lo = [](uint32_t w) { return (int32_t)(w & 0x0F0F0F0Fu); };
    auto hi = [](uint32_t w) { return (int32_t)((w >> 4) & 0x0F0F0F0Fu); };
    B0 = i32x4{lo(u.w0.x), hi(u.w0.x), lo(u.w0.y), hi(u.w0.y)};
    B1 = i32x4{lo(u.w0.z), hi(u.w0.z), lo(u.w0.w), hi(u.w0.w)};
  }
  i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[0], B0, i32x4{0, 0, 0, 0}, 0, 0, 0);
  D = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[1], B1, D, 0, 0, 0);
  float t;
  if (QT == LLMHIP_Q8_0) {
    t = fmaf((float)(D[0] - T[0]), 65536.f, fmaf((float)(D[1] - T[1]), 256.f, (float)(D[2] - T[2])));
  } else {
    // the digits recombined in integers: the block's sum times 128 is below
    // 32 * 2^22 * 15 < 2^31 in magnitude (Q4_0 with its offset: * 8), so the
    // sum taken modulo 2^32 is exact, and one conversion rounds it (T[3]: the
    // offsets recombined the same way)
    const uint32_t d = (((uint32_t)D[0] << 8) + (uint32_t)D[1]) << 8;
    t = (float)(int32_t)(d + (uint32_t)D[2] - (uint32_t)T[3]);
  }
  if (QT == LLMHIP_Q4_1) {  // (d, m) of block q
    const uint32_t sw = q == 0 ? u.sv.x : q == 1 ? u.sv.y : q == 2 ? u.sv.z : u.sv.w;
    acc = fmaf(f16_hw(sw & 0xffff), t, acc);
    acc = fmaf(f16_hw(sw >> 16), bsq, acc);
  } else {  // d of blocks 0, 1 in sv.x, of 2, 3 in sv.y
    const uint32_t sw = q < 2 ? u.sv.x : u.sv.y;
    acc = fmaf(f16_hw((q & 1) ? sw >> 16 : sw & 0xffff), t, acc);
  }
}

// Greedy-sampling partials: (max, lowest index) over the rows a workgroup saw
// (NaN never wins, cpu.go:389-397), written to amax_v/amax_i[blockIdx.x];
// argmax_kernel combines the workgroups'.  Called by every thread.
__device__ __forceinline__ void argmax_partial(const GemvArgs& a, float* misc, float bv, uint32_t bi) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const uint32_t nwv = blockDim.x >> 6;
  float* av = misc + 80;
  uint32_t* ai = (uint32_t*)(misc + 96);
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(bv, o);
    uint32_t oi = __shfl_xor(bi, o);
    if (amax_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    av[wave] = bv;
    ai[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (uint32_t w = 1; w < nwv; w++)
      if (amax_better(av[w], ai[w], bv, bi)) {
        bv = av[w];
        bi = ai[w];
      }
    a.amax_v[blockIdx.x] = bv;
    a.amax_i[blockIdx.x] = bi;
  }
}

// Large matrices at one token (the vocabulary head; the 151936-row sweep
// shape; k a multiple of 128, no tail blocks): a grid of a few workgroups per
// CU, the activations staged once per workgroup, and each of the W waves of
// the grid streaming the groups of its tiles w, w + W, w + 2W, ... in order.
// Every refill is issued (those past the wave's last tile read one line for
// the whole wave), so the compiler's wait before each group can count the
// loads issued after it -- on gfx9 stores count too, so the loop is shaped to
// make every count static:
//  NG > 0 (NG groups per tile): one loop iteration is one tile; group g is
//    taken from ring slot g and the slot refilled with group g of the wave's
//    next tile at once, so a whole tile (NG groups) is always in flight; the
//    tile's row epilogue ends the iteration.
//  NG == 0 (any ng): a ring of STREAM_RING groups, the epilogue after a tile's
//    last group (in flight between tiles it drains to the epilogue's stores).
constexpr int STREAM_RING = 4;
template <uint32_t QT, int PRO, int EPI, int NG>
__global__ __launch_bounds__(512) void gemv_stream_kernel(GemvArgs a) {
  constexpr int R = NG > 0 ? NG : STREAM_RING;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const uint32_t nwv = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const uint32_t nb = a.nb, ng = NG > 0 ? NG : a.ng;
  constexpr bool Q8 = (PRO & PRO_Q8) != 0;
  const Lds L = lds_layout(1, QT, nb, nwv, Q8);
  h8* xs = (h8*)(lds + L.xs);
  float* misc = (float*)(lds + L.misc);
  float* bsum = (float*)(lds + L.bsum);
  float* dxs = (float*)(lds + L.dx);
  const int r = lane & 15, q = lane >> 4, slot = lane & 15;
  const uint32_t W = gridDim.x * nwv, gw = blockIdx.x * nwv + wave;
  const uint32_t ntw = gw < a.tiles ? (a.tiles - 1 - gw) / W + 1 : 0;
  const uint32_t U = ntw * ng;
  WUnit w[R];
  float acc0 = 0, acc1 = 0, bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  int ex[1];
  // the row epilogue of the wave's tile j (argmax partials in bv / bi)
  auto finish = [&](uint32_t j) {
    const uint32_t tile = gw + j * W;
    if (NG > 0 && !Q8) {  // group_i8: lane (r, q) holds block q of every group, times 2^7 more
      acc0 += __shfl_xor(acc0, 16);
      acc0 += __shfl_xor(acc0, 32);
    }
    const float v = q == 0 ? ldexpf(acc0, -ex[0] - (NG > 0 && !Q8 ? 7 : 0)) : 0.f;
    row_epilogue<EPI>(a, tile, r, true, 0, q == 0, v, 1, false, 0.f);
    if (EPI == EPI_ARGMAX) {
      const uint32_t lr = row_of_pos(tile * 16 + r, a.map, a.map_hd, a.map_seg0, a.map_seg1, a.ff);
      if (q == 0 && lr < a.rows && v == v && amax_better(v, lr, bv, bi)) {
        bv = v;
        bi = lr;
      }
    }
    acc0 = acc1 = 0;
  };
  if (NG > 0) {
    // The wave's next tile is in flight while it computes the current one:
    // its quants in wt (group g refilled as soon as group g is consumed) and
    // its scales (one load per four groups, handed to the lanes that need
    // them by ds_bpermute) in sc, refilled at the tile's start once the
    // tile's NG groups of scales are extracted.
    constexpr int NS = NG > 0 ? (NG + 3) / 4 : 1;
    constexpr int NGX = NG > 0 ? NG : 1;
    WUnit wt[NGX];
    uint4 sc[NS];
    auto load_sc = [&](uint32_t t, bool real) {
#pragma unroll
      for (int h = 0; h < NS; h++) sc[h] = load_scales4<QT, NG>(a.qs, nb, t, h, lane, real);
    };
    // the activations first (loads return in order), then the first tile
    XItems<1> xi;
    stage_x_load<1, PRO>(a, 0, 1, xi);
    {
      const uint32_t t0 = min(gw, a.tiles - 1);
      load_sc(t0, gw < a.tiles);
#pragma unroll
      for (int g = 0; g < NG; g++) load_group<QT, true, false>(wt[g], a.qs, nb, t0, g, lane, r, gw < a.tiles);
    }
    stage_x_from<QT, 1, PRO>(a, 1, xi, xs, misc, bsum, dxs, ex);
    // f32 activations: the integer form's digits staged once per workgroup,
    // each wave's A operands and per-block offsets in registers
    constexpr int NX = Q8 ? 1 : NGX;
    i32x4 xa[NX][2], tq[NX];
    float bq[NX];
    if (!Q8) {
      uint64_t* dg = (uint64_t*)(lds + L.total);
      i32x4* tb = (i32x4*)(lds + L.total + 96 * nb);
      stage_digits<QT>(xs, nb, dg, tb);
#pragma unroll
      for (int g = 0; g < NX; g++) {
        i8_operands(dg, g, lane, xa[g]);
        tq[g] = tb[4 * g + q];
        bq[g] = QT == LLMHIP_Q4_1 ? 128.f * bsum[4 * g + q] : 0.f;
      }
    }
    for (uint32_t j = 0; j < ntw; j++) {
      const uint32_t next = min(gw + (j + 1) * W, a.tiles - 1);
      const bool more = j + 1 < ntw;
      uint4 sv[NGX];
#pragma unroll
      for (int g = 0; g < NG; g++) sv[g] = group_scales<QT>(sc[g / 4], g, r);
      __builtin_amdgcn_sched_barrier(0);
      load_sc(next, more);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int g = 0; g < NG; g++) {
        wt[g].sv = sv[g];
        if (Q8)
          group_mfma<QT, 1, Q8>(wt[g], g, xs, bsum, dxs, nb, q, slot, acc0, acc1);
        else
          group_i8<QT>(wt[g], xa[g], tq[g], bq[g], q, acc0);
        // the slot's last use before its refill, and the refill issued there:
        // no register copy of a load still in flight (the empty asm keeps the
        // scaled sums from sinking into the epilogue)
        asm volatile("" : "+v"(acc0), "+v"(acc1));
        __builtin_amdgcn_sched_barrier(0);
        load_group<QT, true, false>(wt[g], a.qs, nb, next, g, lane, r, more);
        __builtin_amdgcn_sched_barrier(0);
      }
      finish(j);
    }
  } else {
    uint32_t jf = 0, gf = 0;  // the next group to load: the wave's tile jf, group gf
    auto fetch = [&](WUnit& u, uint32_t i) {
      load_group<QT, true>(u, a.qs, nb, min(gw + jf * W, a.tiles - 1), gf, lane, r, i < U);
      if (++gf == ng) {
        gf = 0;
        jf++;
      }
    };
    XItems<1> xi;
    stage_x_load<1, PRO>(a, 0, 1, xi);
#pragma unroll
    for (int d = 0; d < R; d++) fetch(w[d], d);
    stage_x_from<QT, 1, PRO>(a, 1, xi, xs, misc, bsum, dxs, ex);
    uint32_t jc = 0, gc = 0;  // the group in the MFMA: tile jc, group gc
    for (uint32_t i0 = 0; i0 < U; i0 += R) {
#pragma unroll
      for (int d = 0; d < R; d++) {
        const uint32_t i = i0 + d;
        if (i >= U) break;
        group_mfma<QT, 1, Q8>(w[d], gc, xs, bsum, dxs, nb, q, slot, acc0, acc1);
        fetch(w[d], i + R);
        if (++gc == ng) {  // the tile is complete
          finish(jc);
          gc = 0;
          jc++;
        }
      }
    }
  }
  if (EPI == EPI_ARGMAX) argmax_partial(a, misc, bv, bi);
}


// ------------------------------------------------ prefill: prep + gemm

constexpr int PMAXI = 4;  // items per thread in prep_kernel: k <= 32 * 4 * 256

// One workgroup per token slot: the prologue of the decode kernel for one
// token (plain, RMSNorm, or the attention merge), written once to global
// memory in MFMA operand order for every workgroup of gemm_kernel: item it
// (block it / 4, k-group it % 4) of token t is the operand of lane
// 16 (it % 4) + t % 16 in group t / 16, its f16 hi parts in the block's first
// 64 operands, its lo parts in the next 64.  Slots past ntok (up to a whole
// group of 16) are zero.
template <int PRO>
__global__ __launch_bounds__(256) void prep_kernel(GemvArgs a_in) {
  __shared__ float red[8];  // [0, 4) wave sums of squares, [4, 8) wave maxima
  // the argument lines it reads in one round (as gemv_kernel's touch_args)
  GemvArgs a = a_in;
  asm volatile("" : "+s"(a.rows), "+s"(a.ldx), "+s"(a.msmax), "+s"(a.tg));
  const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const uint32_t nb = a.nb, K = a.k, NI = nb * 4;
  h8* xp = (h8*)a.xp;
  const uint32_t tg = t / 16, slot = t % 16;
  if (t >= a.ntok) {
    for (uint32_t it = tid; it < NI; it += 256) {
      xp[((uint64_t)tg * nb + it / 4) * 128 + (it % 4) * 16 + slot] = h8{};
      xp[((uint64_t)tg * nb + it / 4) * 128 + 64 + (it % 4) * 16 + slot] = h8{};
    }
    for (uint32_t b = tid; b < nb; b += 256) a.xbsum[(uint64_t)t * nb + b] = a.xdx[(uint64_t)t * nb + b] = 0.f;
    if (tid == 0) a.xexp[t] = 0;
    return;
  }
  f4 va[PMAXI], vc[PMAXI], wa[PMAXI], wc[PMAXI];  // x, and the norm weights in the same round trip
  {
#pragma unroll
    for (int k = 0; k < PMAXI; k++) {
      // loads without a condition, so that one wait covers them all (items
      // past the row read the last one; the reductions skip them)
      const uint32_t it = tid + k * 256, ic = min(it, NI - 1);
      const float* xr = a.x + (uint64_t)(a.xrow0 + t) * a.ldx + (ic / 4) * 32 + 4 * (ic % 4);
      va[k] = *(const f4*)xr;
      vc[k] = *(const f4*)(xr + 16);
      if (PRO & PRO_RMS) {
        const float* wr = a.nw + (ic / 4) * 32 + 4 * (ic % 4);
        wa[k] = *(const f4*)wr;
        wc[k] = *(const f4*)(wr + 16);
      }
    }
  }
  // f32 mode with RMSNorm: the largest |x * w| goes through the same barrier
  // as the sum of squares (the exponent below needs only the magnitude of
  // max |x * s * w| = s * max |x * w|, s > 0), so the prep has one barrier
  float mw = 0;
  if (PRO & PRO_RMS) {
    // cpu.go:90-96
    float ss = 0;
#pragma unroll
    for (int k = 0; k < PMAXI; k++)
      if (tid + k * 256 < NI)
        for (int i = 0; i < 4; i++) {
          ss += va[k][i] * va[k][i] + vc[k][i] * vc[k][i];
          mw = fmaxf(mw, fmaxf(fabsf(va[k][i] * wa[k][i]), fabsf(vc[k][i] * wc[k][i])));
        }
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    if (!(PRO & PRO_Q8)) {
      mw = wave_max(mw);
      if (lane == 0) red[4 + wave] = mw;
    }
    __syncthreads();
    // every thread forms the scale from the four wave sums (same order): no second barrier
    const float sc = (float)(1.0 / sqrt((double)((red[0] + red[1] + red[2] + red[3]) / (float)K + a.eps)));
    mw = sc * fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
#pragma unroll
    for (int k = 0; k < PMAXI; k++) {
      uint32_t it = tid + k * 256;
      if (it >= NI) continue;
      for (int i = 0; i < 4; i++) {
        va[k][i] = __fmul_rn(__fmul_rn(va[k][i], sc), wa[k][i]);
        vc[k][i] = __fmul_rn(__fmul_rn(vc[k][i], sc), wc[k][i]);
      }
    }
  }
  if (PRO & PRO_Q8) {  // quantizeQ8 per block, as in stage_x
    if (tid == 0) a.xexp[t] = 0;
#pragma unroll
    for (int k = 0; k < PMAXI; k++) {
      const uint32_t it = tid + k * 256;
      const f4 A = va[k], C = vc[k];
      float am = 0;
      for (int i = 0; i < 4; i++) am = fmaxf(am, fmaxf(fabsf(A[i]), fabsf(C[i])));
      am = fmaxf(am, __shfl_xor(am, 1));
      am = fmaxf(am, __shfl_xor(am, 2));
      const float d = __fdiv_rn(am, 127.f);
      const float id = d != 0.f ? __fdiv_rn(1.f, d) : 0.f;
      const float v[8] = {A[0], A[2], C[0], C[2], A[1], A[3], C[1], C[3]};
      h8 hi;
      int qs = 0;
      for (int i = 0; i < 8; i++) {
        const float qv = roundf(__fmul_rn(v[i], id));
        hi[i] = (_Float16)qv;
        qs += (int)qv;
      }
      qs += __shfl_xor(qs, 1);
      qs += __shfl_xor(qs, 2);
      if (it >= NI) continue;
      h8* dst = xp + ((uint64_t)tg * nb + it / 4) * 128 + (it % 4) * 16 + slot;
      dst[0] = hi;
      dst[64] = h8{};
      if ((it & 3) == 0) {
        a.xdx[(uint64_t)t * nb + it / 4] = (float)to_f16(d);
        a.xbsum[(uint64_t)t * nb + it / 4] = (float)to_f16(__fmul_rn(d, (float)qs));
      }
    }
    return;
  }
  float mm = mw;
  if (!(PRO & PRO_RMS)) {
    float m = 0;
#pragma unroll
    for (int k = 0; k < PMAXI; k++)
      if (tid + k * 256 < NI)
        for (int i = 0; i < 4; i++) m = fmaxf(m, fmaxf(fabsf(va[k][i]), fabsf(vc[k][i])));
    m = wave_max(m);
    if (lane == 0) red[4 + wave] = m;
    __syncthreads();
    // every thread forms the exponent from the four wave maxima: no second barrier
    mm = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
  }
  int ex = 0;
  {
    if (mm > 0 && mm <= 3.0e38f) {
      int E;
      frexpf(mm, &E);
      ex = 15 - E;
    }
  }
  if (tid == 0) a.xexp[t] = ex;
#pragma unroll
  for (int k = 0; k < PMAXI; k++) {
    uint32_t it = tid + k * 256;
    if (it >= NI) continue;
    const f4 A = va[k], C = vc[k];
    const float v[8] = {A[0], A[2], C[0], C[2], A[1], A[3], C[1], C[3]};
    h8 hi, lo;
    for (int i = 0; i < 8; i++) {
      float sv = ldexpf(v[i], ex);
      _Float16 h = (_Float16)sv;
      hi[i] = h;
      lo[i] = (_Float16)(sv - (float)h);
    }
    h8* dst = xp + ((uint64_t)tg * nb + it / 4) * 128 + (it % 4) * 16 + slot;
    dst[0] = hi;
    dst[64] = lo;
    float sx = (A[0] + A[1] + A[2] + A[3]) + (C[0] + C[1] + C[2] + C[3]);
    sx += __shfl_xor(sx, 1);
    sx += __shfl_xor(sx, 2);
    if ((it & 3) == 0) a.xbsum[(uint64_t)t * nb + it / 4] = ldexpf(sx, ex);
  }
}

// Prefill matrix product.  A workgroup owns GT 16-row tiles and one group of
// 16 tokens (grid.y walks the groups); its waves split the block groups of k
// (split-K).  Per block and tile, two MFMAs chained in one accumulator give
// the 16 tokens' products with the block's 16 rows: A = the tokens' f16 hi
// parts, then A = their lo parts (v_mfma_f32_16x16x32_f16: lane l holds
// A[l % 16][8 (l / 16) ..], B[8 (l / 16) ..][l % 16] and D[4 (l / 16) + i][l % 16],
// i < 4: tokens 4 (l / 16) + i of row l % 16), so each lane scales four
// token sums by the block's d.  Each wave pipelines its block groups through
// two register sets: the weights and activation operands of its next group
// are in flight while the current one goes through the MFMA.  Every load in
// that loop is unconditional (indices clamped into the matrix and the
// prepared activations), so the waits count only what is needed.  A weight
// word is dequantised once and feeds both MFMAs of its tile, an activation
// operand GT tiles.  The waves' partials meet in LDS; wave w then adds, in
// wave order, rows w, w + waves, ... (row p: tile p / 2, token pair p % 2 of
// the lane's four) and runs their row epilogues, having loaded the first
// one's inputs with its first operands.
constexpr int GEMM_MAXW = 8;  // waves per workgroup

// The activation side of one block group: 4 blocks x (hi, lo) MFMA operands
// of the workgroup's 16 tokens, and per block the scalars of the lane's four
// tokens where the product needs them (Q8: the activation blocks' d; Q4_1:
// the block sums that meet m).
template <uint32_t QT, bool Q8>
struct XUnit {
  h8 x[4][2];
  float xd[Q8 ? 4 : 1][Q8 ? 4 : 1];
  float xb[QT == LLMHIP_Q4_1 ? 4 : 1][QT == LLMHIP_Q4_1 ? 4 : 1];
};

// Blocks b0 .. b0+3 (clamped to bmax) of token group g.
template <uint32_t QT, bool Q8>
__device__ __forceinline__ void load_xunit(XUnit<QT, Q8>& X, const GemvArgs& a, uint32_t b0, uint32_t bmax,
                                           uint32_t g, int lane, int q) {
  const h8* xp = (const h8*)a.xp;
  const uint32_t nb = a.nb;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t b = min(b0 + j, bmax);
    const h8* xb = xp + ((uint64_t)g * nb + b) * 128 + lane;
    X.x[j][0] = xb[0];
    X.x[j][1] = xb[64];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint64_t it = (uint64_t)(g * 16 + 4 * q + i) * nb + b;
      if (Q8) X.xd[j][i] = a.xdx[it];
      if (QT == LLMHIP_Q4_1) X.xb[j][i] = a.xbsum[it];
    }
  }
}

__device__ __forceinline__ uint32_t u4c(const uint4& v, int j) {
  return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

// Block j of a weight unit: the B operand, d and (Q4_1) m.  A group unit
// holds a 4-block record; the tail unit (TAIL) holds block j in component j.
// RK: the nibble dequantiser on register constants (dq4k).
template <uint32_t QT, bool TAIL, bool RK = false>
__device__ __forceinline__ void unit_block(const WUnit& u, int j, h8& B, float& d, float& m) {
  m = 0.f;
  if (QT == LLMHIP_Q8_0) {
    if (TAIL) {
      B = dq8(u4c(u.w0, j), u4c(u.w1, j));
      d = f16_hw(u4c(u.sv, j) & 0xffff);
    } else {
      const uint4 ww = j < 2 ? u.w0 : u.w1;
      B = (j % 2 == 0) ? dq8(ww.x, ww.y) : dq8(ww.z, ww.w);
      const uint32_t sw = j < 2 ? u.sv.x : u.sv.y;
      d = f16_hw(j % 2 == 0 ? sw & 0xffff : sw >> 16);
    }
  } else if (QT == LLMHIP_Q4_1) {
    B = RK ? dq4k<true>(u4c(u.w0, j), dq4_consts()) : dq4<true>(u4c(u.w0, j));
    const uint32_t sw = u4c(u.sv, j);
    d = f16_hw(sw & 0xffff);
    m = f16_hw(sw >> 16);
  } else {
    B = RK ? dq4k<false>(u4c(u.w0, j), dq4_consts()) : dq4<false>(u4c(u.w0, j));
    if (TAIL) {
      d = f16_hw(u4c(u.sv, j) & 0xffff);
    } else {
      const uint32_t sw = j < 2 ? u.sv.x : u.sv.y;
      d = f16_hw(j % 2 == 0 ? sw & 0xffff : sw >> 16);
    }
  }
}

// The MFMAs of one unit (nblk of its 4 blocks) into acc[tile][token of the lane's four].
template <uint32_t QT, bool Q8, int GT, bool TAIL>
__device__ __forceinline__ void gemm_unit(float (&acc)[GT][4], const WUnit (&w)[GT], const XUnit<QT, Q8>& X,
                                          int nblk) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (j >= nblk) break;
    h8 B[GT];
    float d[GT], mm[GT];
#pragma unroll
    for (int u = 0; u < GT; u++) unit_block<QT, TAIL, true>(w[u], j, B[u], d[u], mm[u]);
#pragma unroll
    for (int u = 0; u < GT; u++) {
      f4 D = __builtin_amdgcn_mfma_f32_16x16x32_f16(X.x[j][0], B[u], f4{0, 0, 0, 0}, 0, 0, 0);
      D = __builtin_amdgcn_mfma_f32_16x16x32_f16(X.x[j][1], B[u], D, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        if (Q8) {  // ggml's block product, as in mfma_block
          float p = __fmul_rn(__fmul_rn(d[u], X.xd[j][i]), D[i]);
          if (QT == LLMHIP_Q4_1) p = __fadd_rn(p, __fmul_rn(mm[u], X.xb[j][i]));
          acc[u][i] += p;
        } else {
          acc[u][i] += d[u] * D[i];
          if (QT == LLMHIP_Q4_1) acc[u][i] += mm[u] * X.xb[j][i];
        }
      }
    }
  }
}

// The activations of one gate/up epilogue row (tile u of the workgroup, tokens
// t and t + 1 of its group; gate row i at lane r < 8, up row i at r + 8) into
// em[token][8 u + i], as EPI_GATEUP forms them.  Every lane calls it.
__device__ __forceinline__ void emit_act(float (&em)[16][33], uint32_t u, uint32_t t, int r, float vA, float vB) {
  const float uA = __shfl_xor(vA, 8), uB = __shfl_xor(vB, 8);
  if (r < 8) {
    em[t][8 * u + r] = vA / (1.f + __expf(-vA)) * uA;
    em[t + 1][8 * u + r] = vB / (1.f + __expf(-vB)) * uB;
  }
}
template <int A, int B>
__device__ __forceinline__ void emit_act(float (&)[A][B], uint32_t, uint32_t, int, float, float) {}

// Block b of the down projection's operands for token group g from em (one
// wave: lane l forms k-group l / 16 of token l % 16).
__device__ __forceinline__ void emit_block(const GemvArgs& a, const float (&em)[16][33], uint32_t g, uint32_t b,
                                           int lane) {
  const uint32_t t16 = lane & 15, kq = lane >> 4;
  const uint32_t col[8] = {0, 2, 16, 18, 1, 3, 17, 19};  // {A0, A2, C0, C2, A1, A3, C1, C3}
  float v[8], mx = 0.f, sm = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    v[i] = em[t16][4 * kq + col[i]];
    mx = fmaxf(mx, fabsf(v[i]));
    sm += v[i];
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16));
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  sm += __shfl_xor(sm, 16);
  sm += __shfl_xor(sm, 32);
  int e = 0;
  if (mx > 0 && mx <= 3.0e38f) {
    int E;
    frexpf(mx, &E);
    e = 15 - E;
  }
  h8 hi, lo;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float sv = ldexpf(v[i], e);
    const _Float16 hh = (_Float16)sv;
    hi[i] = hh;
    lo[i] = (_Float16)(sv - (float)hh);
  }
  h8* dst = (h8*)a.op_xp + ((uint64_t)g * a.op_nb + b) * 128 + lane;
  dst[0] = hi;
  dst[64] = lo;
  if (kq == 0) {
    const uint32_t t = g * 16 + t16;
    a.op_dx[(uint64_t)t * a.op_nb + b] = ldexpf(1.f, -e);
    a.op_bsum[(uint64_t)t * a.op_nb + b] = sm;
    if (b == 0) a.op_exp[t] = 0;
  }
}

// EM (EPI_GATEUP, four tiles: the 32 activations of one block of the down
// projection's input per workgroup): the epilogue rows also put their
// activations into LDS, and wave 0 then forms the block's operands for the
// workgroup's 16 tokens (GemvArgs::op_xp) as the attention's emit_operand
// does: per token the exponent e that puts the block's largest magnitude in
// [2^14, 2^15), hi = f16(v 2^e), lo = f16(v 2^e - hi), lane t + 16 kq holding
// k-group kq of token t.
template <uint32_t QT, int EPI, bool Q8, int GT, bool EM = false>
__global__ __launch_bounds__(64 * GEMM_MAXW) void gemm_kernel(GemvArgs a_in) {
  static_assert(!EM || (EPI == EPI_GATEUP && GT == 4), "the emitting form is four gate/up tiles");
  __shared__ float red[GEMM_MAXW][GT * 4][64];
  __shared__ float em[EM ? 16 : 1][EM ? 33 : 1];
  // the argument lines it reads in one round (as gemv_kernel's touch_args):
  // 0-1 the matrix and output, 2 the epilogue's, 3 up / kparts, 4-5 the prepared operands
  static_assert(offsetof(GemvArgs, xexp) / 64 == 4 && offsetof(GemvArgs, tg) / 64 == 5, "argument lines");
  GemvArgs a = a_in;
  asm volatile("" : "+s"(a.rows), "+s"(a.ldx), "+s"(a.ldy), "+s"(a.kparts), "+s"(a.msmax), "+s"(a.tg));
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int r = lane & 15, q = lane >> 4;
  // W: 4 or 8 waves (gemm_shape), so the counts below are shifts
  const uint32_t W = blockDim.x >> 6, lw = __builtin_ctz(W), nb = a.nb, ng = a.ng;
  const uint32_t g = blockIdx.y, tile0 = blockIdx.x * GT;
  bool tv[GT];
  uint32_t tt[GT];
#pragma unroll
  for (int u = 0; u < GT; u++) {
    tv[u] = tile0 + u < a.tiles;
    tt[u] = tv[u] ? tile0 + u : tile0;
  }
  float acc[GT][4];
#pragma unroll
  for (int u = 0; u < GT; u++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[u][i] = 0.f;

  // groups wave, wave + W, ...: two register sets, A and B, in turn
  const uint32_t cnt = ng > (uint32_t)wave ? (ng - wave + W - 1) >> lw : 0;
  const uint32_t glast = wave + (cnt ? cnt - 1 : 0) * W;
  WUnit wA[GT], wB[GT];
  XUnit<QT, Q8> xA, xB;
  auto load = [&](WUnit (&w)[GT], XUnit<QT, Q8>& X, uint32_t gi) {
#pragma unroll
    for (int u = 0; u < GT; u++) load_group<QT>(w[u], a.qs, nb, tt[u], gi, lane, r);
    load_xunit<QT, Q8>(X, a, 4 * gi, 4 * gi + 3, g, lane, q);
  };
  // wave w runs the epilogues of rows p = w, w + W, ... < 2 GT, row p being
  // (tile p / 2, token pair p % 2 of the lane's four); the inputs of its first
  // (residual, bias, RoPE table, token scales) are loaded with the first
  // group's operands
  const bool epw = (uint32_t)wave < (uint32_t)(GT * 2);
  const uint32_t pu = (uint32_t)wave / 2, ph = (uint32_t)wave % 2;
  bool ptv = tv[0];
#pragma unroll
  for (int u = 1; u < GT; u++) ptv = pu == (uint32_t)u ? tv[u] : ptv;
  const uint32_t tokA = g * 16 + 4 * q + 2 * ph, tokB = tokA + 1;
  const bool okA = tokA < a.ntok, okB = tokB < a.ntok;
  EpiIn ein;
  int exA = 0, exB = 0;
  if (cnt) {
    // no branch between a load and its use, and scheduling barriers, so the
    // loads of the next group stay ahead of the current group's MFMAs
    load(wA, xA, wave);
    if (epw) {
      ein = epi_load<EPI>(a, tile0 + pu, r, ptv, tokA, okA, tokB, okB);
      exA = okA ? a.xexp[tokA] : 0;
      exB = okB ? a.xexp[tokB] : 0;
    }
    uint32_t i = 0;
    for (; i + 1 < cnt; i += 2) {
      load(wB, xB, wave + (i + 1) * W);
      __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
      gemm_unit<QT, Q8, GT, false>(acc, wA, xA, 4);
      load(wA, xA, min(wave + (i + 2) * W, glast));
      __builtin_amdgcn_sched_barrier(0);
      gemm_unit<QT, Q8, GT, false>(acc, wB, xB, 4);
    }
    if (i < cnt) gemm_unit<QT, Q8, GT, false>(acc, wA, xA, 4);
  } else if (epw) {
    ein = epi_load<EPI>(a, tile0 + pu, r, ptv, tokA, okA, tokB, okB);
    exA = okA ? a.xexp[tokA] : 0;
    exB = okB ? a.xexp[tokB] : 0;
  }
  if (a.tail && (ng & (W - 1)) == (uint32_t)wave) {
    WUnit wt[GT];
    XUnit<QT, Q8> xt;
#pragma unroll
    for (int u = 0; u < GT; u++) load_unit<QT>(wt[u], a.qs, nb, tt[u], ng, ng, a.tail, lane, r);
    load_xunit<QT, Q8>(xt, a, 4 * ng, 4 * ng + a.tail - 1, g, lane, q);
    gemm_unit<QT, Q8, GT, true>(acc, wt, xt, (int)a.tail);
  }

  // split-K: every wave's partials into LDS, then each epilogue row is added
  // in wave order by its wave
#pragma unroll
  for (int u = 0; u < GT; u++)
#pragma unroll
    for (int i = 0; i < 4; i++) red[wave][u * 4 + i][lane] = acc[u][i];
  __syncthreads();
  if (epw) {
    const uint32_t o = 4 * pu + 2 * ph;
    float s0 = red[0][o][lane], s1 = red[0][o + 1][lane];
    for (uint32_t w = 1; w < W; w++) {
      s0 += red[w][o][lane];
      s1 += red[w][o + 1][lane];
    }
    const float vA = okA ? ldexpf(s0, -exA) : 0.f;
    const float vB = okB ? ldexpf(s1, -exB) : 0.f;
    row_epilogue<EPI>(a, tile0 + pu, r, ptv, tokA, okA, vA, tokB, okB, vB, &ein);
    if (EM) emit_act(em, pu, 4 * q + 2 * ph, r, vA, vB);
  }
  // rows past the first wave's (GT > W / 2): W is even, so row p's token pair
  // is the wave's own, and so are the token scales loaded with the first row
  for (uint32_t p = wave + W; p < (uint32_t)(GT * 2); p += W) {
    const uint32_t u = p / 2, o = 2 * p, tA = tokA, tB = tokB;
    bool v = tv[0];
#pragma unroll
    for (int k = 1; k < GT; k++) v = u == (uint32_t)k ? tv[k] : v;
    float s0 = red[0][o][lane], s1 = red[0][o + 1][lane];
    for (uint32_t w = 1; w < W; w++) {
      s0 += red[w][o][lane];
      s1 += red[w][o + 1][lane];
    }
    const float vA = okA ? ldexpf(s0, -exA) : 0.f;
    const float vB = okB ? ldexpf(s1, -exB) : 0.f;
    row_epilogue<EPI>(a, tile0 + u, r, v, tA, okA, vA, tB, okB, vB);
    if (EM) emit_act(em, u, 4 * q + 2 * ph, r, vA, vB);
  }
  if constexpr (EM) {
    __syncthreads();
    if (wave == 0) emit_block(a, em, g, tile0 / 4, lane);
  }
}

// ------------------------------------------------------- the decode kernel

// The decode matrix-vector product (1, 2 or 4 tokens).  Waves of a workgroup
// own 16-row tiles; `split` waves share a tile's block groups (split-K, added
// in a fixed order through LDS at the end).  Each wave stages only the
// activations its own units need, in its own part of LDS, with no barrier:
// a batch of up to UB units (groups of four blocks), one DPP row of 16 lanes
// per unit, lane = item (block b, k-group iq: elements 4iq..4iq+3 and
// 16+4iq..16+4iq+3 of the block).  Each unit and token gets its own power of
// two 2^e (the unit's largest magnitude in [2^14, 2^15)), the scaled values are
// split exactly into f16 hi + lo, written to the wave's LDS in MFMA operand
// order and read back by the operand lanes.  RMSNorm (cpu.go:81-98) takes the
// sum of squares of the whole row, which every wave reduces itself.  Loads are
// issued rows, then activation items, then weights: they return in order, so
// the staging overlaps the weights' round trip.
constexpr int UB = 4;  // units per staging batch: one 16-lane DPP row each

// LDS of one wave: A operands [unit][block][k-group][slot] h8 (slots 2t, 2t+1:
// hi, lo of token t), then [unit][block][token] floats: the block sums of x
// (Q4_1) and the activation block scales (PRO_Q8).
template <int NT>
struct WaveLds {
  static constexpr uint32_t S = 2 * NT;
  static constexpr uint32_t OPS = UB * 16 * S * 16;
  static constexpr uint32_t TAB = UB * 4 * NT * 4;
  static constexpr uint32_t BYTES = OPS + 2 * TAB;
};

// Bytes of LDS of a decode-kernel launch: the waves' own staging, the split-K
// partials, and 128 floats of workgroup scratch (the argmax partials).
__host__ __device__ inline uint32_t decode_lds(int nt, uint32_t waves) {
  const uint32_t per = nt == 1 ? WaveLds<1>::BYTES : nt == 2 ? WaveLds<2>::BYTES : WaveLds<4>::BYTES;
  return waves * per + waves * 64 * 2 * 4 + 128 * 4;
}

// One lane's activation item of a staging batch, for each token: x (and the
// norm weights), zero where the item does not exist.  With four units per
// batch a lane loads both halves of its item (elements 4iq..4iq+3 in xa,
// 16+4iq..16+4iq+3 in xc); with two, lanes 0-31 load the first halves of the
// two units' items and lanes 32-63 the second (one load instruction per
// array instead of two), in xa, and staging swaps them across.
// MC chunks (PRO_MERGE, one token): instead of x, each chunk's (max, sum of
// e) of the item's head and its partial sums of e*v for the item's elements;
// P, the chunks below the causal bound; merge_items forms xa / xc from them.
template <int NT, bool RMS, uint32_t MC = 0>
struct Items {
  f4 xa[NT], xc[NT], wa, wc;
  float mc[MC ? MC : 1], lc[MC ? MC : 1];
  f4 oa[MC ? MC : 1], oc[MC ? MC : 1];
  uint32_t P, e0;
  bool ok;
};
template <int NT, int PRO>
using ItemsOf = Items<NT, (PRO & PRO_RMS) != 0, merge_chunks(PRO)>;

// Issue the item loads of the batch whose units start at i0 (group sp +
// i * split for unit i < cnt; with TAILU the tail, blocks < tail).  Absent
// items read one address for the whole wave, so the loads are unconditional.
template <int NT, int PRO, bool TAILU, int NU>
__device__ __forceinline__ void load_items(ItemsOf<NT, PRO>& it, const GemvArgs& a, uint32_t t0, int nt, uint32_t i0,
                                           uint32_t cnt, uint32_t sp, uint32_t split, int lane) {
  const uint32_t u = NU == 4 ? lane >> 4 : (lane >> 4) & 1, b = (lane >> 2) & 3, iq = lane & 3;
  const uint32_t half = NU == 4 ? 0 : lane >> 5;
  const uint32_t i = i0 + u;
  const bool ok = TAILU ? (u == 0 && b < a.tail) : i < cnt;
  const uint32_t g = TAILU ? a.ng : sp + i * split;
  const uint32_t e0 = ok ? (g * 4 + b) * 32 + 4 * iq + 16 * half : 0;
  const f4 z = {0, 0, 0, 0};
  if constexpr ((PRO & PRO_MERGE) != 0) {
    // one token: the head of elements e0.. (and e0 + 16..), its chunks
    static_assert(NT == 1, "merging prologue: one token");
    const uint32_t h = e0 >> __builtin_ctz(a.hd), d = e0 & (a.hd - 1);  // hd: 64 or 128
    const float* ml = a.mml + (uint64_t)h * a.msmax * 2;
    const float* pv = a.mpv + (uint64_t)h * a.msmax * a.hd + d;
#pragma unroll
    for (uint32_t c = 0; c < merge_chunks(PRO); c++) {
      typedef float f2 __attribute__((ext_vector_type(2)));
      const uint32_t cc = min(c, a.msmax - 1);
      const f2 v = *(const f2*)(ml + 2 * cc);
      it.mc[c] = v[0];
      it.lc[c] = v[1];
      it.oa[c] = *(const f4*)(pv + (uint64_t)cc * a.hd);
      if (NU == 4) it.oc[c] = *(const f4*)(pv + (uint64_t)cc * a.hd + 16);
    }
    it.P = (state_pos(a.state) + a.mrows) >> __builtin_ctz(a.mrows);  // chunks holding positions 0 .. pos (mrows: a power of two)
    it.e0 = e0;
    it.ok = ok;
    return;
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const float* xr = a.x + (uint64_t)(a.xrow0 + t0 + min(t, nt - 1)) * a.ldx + e0;
    f4 A = *(const f4*)xr;
    if constexpr ((PRO & PRO_XSUM) != 0) {  // one token: (x + p0) + p1
      static_assert(NT == 1, "PRO_XSUM: one token");
      const f4 P0 = *(const f4*)(a.xpart + e0), P1 = *(const f4*)(a.xpart + a.xpartstride + e0);
      A = (A + P0) + P1;
    }
    it.xa[t] = ok && t < nt ? A : z;
    if (NU == 4) {
      f4 C = *(const f4*)(xr + 16);
      if constexpr ((PRO & PRO_XSUM) != 0) {
        const f4 P0 = *(const f4*)(a.xpart + e0 + 16), P1 = *(const f4*)(a.xpart + a.xpartstride + e0 + 16);
        C = (C + P0) + P1;
      }
      it.xc[t] = ok && t < nt ? C : z;
    }
  }
  if (PRO & PRO_RMS) {
    const f4 A = *(const f4*)(a.nw + e0);
    it.wa = ok ? A : z;
    if (NU == 4) {
      const f4 C = *(const f4*)(a.nw + e0 + 16);
      it.wc = ok ? C : z;
    }
  }
}

// PRO_MERGE: the item's attention outputs from its loaded chunk partials, in
// attn_merge_kernel's order (one batch of chunks from M = -inf, L = o = 0:
// M = max m_c, w_c = e^{m_c - M}, L = sum w_c l_c, o = sum w_c o_c, o / L);
// chunks at or past P are left out.  keep: also store them to matt.
template <int PRO, int NU>
__device__ __forceinline__ void merge_items(ItemsOf<1, PRO>& it, const GemvArgs& a, bool keep) {
  constexpr uint32_t MC = merge_chunks(PRO);
  float M = -INFINITY;
#pragma unroll
  for (uint32_t c = 0; c < MC; c++) M = fmaxf(M, c < it.P ? it.mc[c] : -INFINITY);
  float L = 0;
  f4 oA = {0, 0, 0, 0}, oC = {0, 0, 0, 0};
#pragma unroll
  for (uint32_t c = 0; c < MC; c++) {
    const bool in = c < it.P;
    const float w = in ? __expf(it.mc[c] - M) : 0.f;
    L += w * (in ? it.lc[c] : 0.f);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      oA[k] += w * (in ? it.oa[c][k] : 0.f);
      if (NU == 4) oC[k] += w * (in ? it.oc[c][k] : 0.f);
    }
  }
  const f4 z = {0, 0, 0, 0};
  f4 A, C;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    A[k] = oA[k] / L;
    C[k] = oC[k] / L;
  }
  it.xa[0] = it.ok ? A : z;
  if (NU == 4) it.xc[0] = it.ok ? C : z;
  if (keep && it.ok) {
    *(f4*)(a.matt + it.e0) = A;
    if (NU == 4) *(f4*)(a.matt + it.e0 + 16) = C;
  }
}

// With two units per batch: each lane's other half, from the lane 32 away.
__device__ __forceinline__ f4 other_half(const f4& v, int lane) {
  f4 o;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t x = __float_as_uint(v[k]);
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    o[k] = __uint_as_float(lane < 32 ? r[1] : r[0]);
  }
  return o;
}

// Stage a batch from its loaded items: RMSNorm's h = (x s) w, then per unit
// and token the scale and the f16 hi + lo split (or, for PRO_Q8, quantizeQ8
// per block of 32, cpu.go:117-140), into the wave's LDS.  ex[u][t] receives
// the exponent of unit u, token t (wave-uniform).  Call with the whole wave.
template <uint32_t QT, int NT, int PRO, int NU>
__device__ __forceinline__ void stage_items(const ItemsOf<NT, PRO>& it, const float (&rs)[NT], int lane,
                                            h8* ops, float* sums, float* dxs, int (&ex)[UB][NT]) {
  constexpr int S = 2 * NT;
  const uint32_t u = NU == 4 ? lane >> 4 : (lane >> 4) & 1, b = (lane >> 2) & 3, iq = lane & 3;
  const bool writer = NU == 4 || lane < 32;  // two units: lanes 32-63 hold copies
  h8* dst = ops + ((u * 4 + b) * 4 + iq) * S;
  f4 wA = {0, 0, 0, 0}, wC = {0, 0, 0, 0};
  if (PRO & PRO_RMS) {
    if (NU == 4) {
      wA = it.wa;
      wC = it.wc;
    } else {
      const f4 o = other_half(it.wa, lane);
      wA = lane < 32 ? it.wa : o;
      wC = lane < 32 ? o : it.wa;
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    f4 A = it.xa[t], C = it.xc[t];
    if (NU == 2) {
      const f4 o = other_half(it.xa[t], lane);
      A = lane < 32 ? it.xa[t] : o;
      C = lane < 32 ? o : it.xa[t];
    }
    if (PRO & PRO_RMS) {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        A[k] = __fmul_rn(__fmul_rn(A[k], rs[t]), wA[k]);  // cpu.go:96
        C[k] = __fmul_rn(__fmul_rn(C[k], rs[t]), wC[k]);
      }
    }
    const float v[8] = {A[0], A[2], C[0], C[2], A[1], A[3], C[1], C[3]};
    if (PRO & PRO_Q8) {
      // a block's four items sit in four consecutive lanes
      float am = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) am = fmaxf(am, fabsf(v[k]));
      am = fmaxf(am, __shfl_xor(am, 1));
      am = fmaxf(am, __shfl_xor(am, 2));
      const float d = __fdiv_rn(am, 127.f);
      const float id = d != 0.f ? __fdiv_rn(1.f, d) : 0.f;
      h8 hi;
      int qs = 0;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float qv = roundf(__fmul_rn(v[k], id));
        hi[k] = (_Float16)qv;
        qs += (int)qv;
      }
      qs += __shfl_xor(qs, 1);
      qs += __shfl_xor(qs, 2);
      if (writer) {
        dst[2 * t] = hi;
        dst[2 * t + 1] = h8{};
        if (iq == 0) {
          dxs[(u * 4 + b) * NT + t] = (float)to_f16(d);
          if (QT == LLMHIP_Q4_1) sums[(u * 4 + b) * NT + t] = (float)to_f16(__fmul_rn(d, (float)qs));
        }
      }
#pragma unroll
      for (int w = 0; w < UB; w++) ex[w][t] = 0;
      continue;
    }
    float m = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) m = fmaxf(m, fabsf(v[k]));
    m = row_max16(m);  // the unit's largest magnitude (its 16 lanes)
    int e = 0;
    if (m > 0 && m <= 3.0e38f) {
      int E;
      frexpf(m, &E);
      e = 15 - E;
    }
    h8 hi, lo;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const float sv = ldexpf(v[k], e);
      const _Float16 h = (_Float16)sv;
      hi[k] = h;
      lo[k] = (_Float16)(sv - (float)h);
    }
    if (writer) {
      dst[2 * t] = hi;
      dst[2 * t + 1] = lo;
    }
    if (QT == LLMHIP_Q4_1) {
      // block sums sum_j x_j (cpu.go:196-198), unscaled
      float sx = (A[0] + A[1] + A[2] + A[3]) + (C[0] + C[1] + C[2] + C[3]);
      sx += __shfl_xor(sx, 1);
      sx += __shfl_xor(sx, 2);
      if (writer && iq == 0) sums[(u * 4 + b) * NT + t] = sx;
    }
#pragma unroll
    for (int w = 0; w < UB; w++) ex[w][t] = __builtin_amdgcn_readlane(e, 16 * (w % NU));
  }
}

// The MFMAs of unit u of a staged batch: group blocks 0..3, or the tail's
// blocks 0..tail-1 (TAIL).  Lane (row r, group q) adds to acc0 / acc1 the
// products of tokens 2q / 2q + 1: d_w 2^-e sum_j (hi + lo)_j w_j per block
// (+ m_w sum_j x_j for Q4_1), or for PRO_Q8 ggml's d_w d_x sum_j q_j w_j
// (+ m_w s_x), rounded as cpu.go:174-210 rounds it.
template <uint32_t QT, int NT, bool Q8, bool TAIL>
__device__ __forceinline__ void unit_products(const WUnit& w, uint32_t u, int nblk, const h8* ops, const float* sums,
                                              const float* dxs, const int (&ex)[UB][NT], int q, int slot, float& acc0,
                                              float& acc1) {
  constexpr int S = 2 * NT;
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  const int tA = min(2 * q, NT - 1), tB = min(2 * q + 1, NT - 1);
  const bool okA = 2 * q < NT, okB = 2 * q + 1 < NT;
  float uA = 0, uB = 0, mA = 0, mB = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (j >= nblk) break;
    const u4v X = __builtin_bit_cast(u4v, ops[((u * 4 + j) * 4 + q) * S + min(slot, S - 1)]);
    const h8 A = __builtin_bit_cast(h8, X & (slot < S ? ~0u : 0u));
    h8 B;
    float d, m;
    unit_block<QT, TAIL>(w, j, B, d, m);
    const f4 D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, f4{0, 0, 0, 0}, 0, 0, 0);
    const uint32_t bi = (u * 4 + j) * NT;
    if (Q8) {
      float pA = __fmul_rn(__fmul_rn(d, dxs[bi + tA]), D[0] + D[1]);
      float pB = __fmul_rn(__fmul_rn(d, dxs[bi + tB]), D[2] + D[3]);
      if (QT == LLMHIP_Q4_1) {
        pA = __fadd_rn(pA, __fmul_rn(m, sums[bi + tA]));
        pB = __fadd_rn(pB, __fmul_rn(m, sums[bi + tB]));
      }
      acc0 += okA ? pA : 0.f;
      if (NT > 1) acc1 += okB ? pB : 0.f;
    } else {
      uA += d * (D[0] + D[1]);
      if (NT > 1) uB += d * (D[2] + D[3]);
      if (QT == LLMHIP_Q4_1) {
        mA += m * sums[bi + tA];
        if (NT > 1) mB += m * sums[bi + tB];
      }
    }
  }
  if (!Q8) {
    // undo the unit's scale of each token (ex[u][t] is wave-uniform)
    const int eA = NT == 4 && q == 1 ? ex[u][min(2, NT - 1)] : ex[u][0];
    const int eB = NT == 4 && q == 1 ? ex[u][min(3, NT - 1)] : ex[u][min(1, NT - 1)];
    acc0 += okA ? ldexpf(uA, -eA) + mA : 0.f;
    if (NT > 1) acc1 += okB ? ldexpf(uB, -eB) + mB : 0.f;
  }
}

// (the merging prologue holds every chunk's partials in registers: at most
// 8 waves per workgroup, so that 256 VGPRs are there for it)
// One field of each 64-byte line of the arguments a one-token launch reads,
// routed through an empty asm whose results the kernel then uses, so that
// all of them are loaded in one round at the kernel's start: every first
// touch of a line misses the scalar cache, and left to the compiler the
// loads follow the branches that use them, three or four dependent rounds of
// a few hundred ns before the first activation load is issued.  After this
// round the other fields' loads hit the cache.
// Lines 2 (the epilogue's outputs) and 4 (the merging and summing
// prologues') only where the variant reads them: a line nobody reads costs a
// miss of its own.
template <int PRO, int EPI>
__device__ __forceinline__ void touch_args(GemvArgs& a) {
  static_assert(offsetof(GemvArgs, rows) < 64 && offsetof(GemvArgs, ldx) / 64 == 1 && offsetof(GemvArgs, ldy) / 64 == 2 &&
                    offsetof(GemvArgs, kparts) / 64 == 3 && offsetof(GemvArgs, xout) / 64 == 4 &&
                    offsetof(GemvArgs, msmax) / 64 == 4 && offsetof(GemvArgs, ff) / 64 == 3 &&
                    offsetof(GemvArgs, up) / 64 == 3,
                "one field of each argument line");
  // (integer fields: a pointer that went through the asm would lose its
  // global address space and be read with flat loads)
  constexpr bool L2 = EPI != EPI_GATEUP, L4 = (PRO & (PRO_MERGE | PRO_XSUM)) != 0;
  if constexpr (L2 && L4) asm volatile("" : "+s"(a.rows), "+s"(a.ldx), "+s"(a.ldy), "+s"(a.kparts), "+s"(a.msmax));
  if constexpr (L2 && !L4) asm volatile("" : "+s"(a.rows), "+s"(a.ldx), "+s"(a.ldy), "+s"(a.kparts));
  if constexpr (!L2 && L4) asm volatile("" : "+s"(a.rows), "+s"(a.ldx), "+s"(a.kparts), "+s"(a.msmax));
  if constexpr (!L2 && !L4) asm volatile("" : "+s"(a.rows), "+s"(a.ldx), "+s"(a.kparts));
}

template <uint32_t QT, int NT, int PRO, int EPI, int NU>
__global__ __launch_bounds__((PRO & PRO_MERGE) ? 512 : 1024) void gemv_kernel(GemvArgs a_in) {
  GemvArgs a = a_in;
  if (NT == 1) touch_args<PRO, EPI>(a);
  typedef WaveLds<NT> WL;
  constexpr bool Q8 = (PRO & PRO_Q8) != 0, RMS = (PRO & PRO_RMS) != 0;
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  const uint32_t nwv = a.waves;  // the launch's blockDim.x / 64
  const int lane = threadIdx.x & 63, wave = wave_id();
  const uint32_t t0 = blockIdx.y * NT;
  const int nt = min((int)NT, (int)(a.ntok - t0));
  const uint32_t nb = a.nb, ng = a.ng;
  unsigned char* wl = lds + wave * WL::BYTES;
  h8* ops = (h8*)wl;
  float* sums = (float*)(wl + WL::OPS);
  float* dxs = (float*)(wl + WL::OPS + WL::TAB);
  float* part = (float*)(lds + nwv * WL::BYTES);
  float* misc = part + nwv * 64 * 2;  // [0, 64): RMS partials; [80, 112): argmax partials

  // split and waves are powers of two and kparts is 1 or 2 (gemv_launch
  // checks), so the indices below take shifts and masks, not divisions
  const uint32_t split = a.split, ls = __builtin_ctz(split), tpw = nwv >> ls;
  const uint32_t lt = wave >> ls;
  // k in parts (one token): workgroup x = (tile group) * kparts + part; part p
  // runs block groups [g0, g1), the last one the tail too, into its own row
  const uint32_t lk = a.kparts > 1 ? 1 : 0, kp = 1u << lk, kpart = blockIdx.x & (kp - 1), bx = blockIdx.x >> lk;
  const uint32_t g0 = (kpart * ng) >> lk, g1 = ((kpart + 1) * ng) >> lk;
  const uint32_t tile = min(bx * tpw + lt, a.tiles - 1);
  const bool has_tile = bx * tpw + lt < a.tiles;
  const bool keep = bx * tpw + lt == 0;  // PRO_MERGE: tile 0's waves also store the merged row
  const int r = lane & 15, q = lane >> 4, slot = lane & 15;
  // this wave's units: groups sp = g0 + sw, sp + split, ... below g1, then the
  // tail (the last part's wave (g1 - g0) % split)
  const uint32_t sw = wave & (split - 1), sp = g0 + sw, gn = g1 - g0;
  const uint32_t cnt = has_tile && gn > sw ? (gn - sw + split - 1) >> ls : 0;
  const bool has_tail = has_tile && a.tail && kpart == kp - 1 && (gn & (split - 1)) == sw;

  // RMSNorm's sum of squares: the workgroup's waves load the row between
  // them (two float4s per lane and token at once: rows up to 512 * waves floats)
  constexpr int RV = 2;
  const uint32_t K4 = a.k / 4;
  f4 rv[RMS ? NT : 1][RMS ? RV : 1];
  if (RMS) {
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int v = 0; v < RV; v++) {
        const uint32_t c = min(wave * 64 + lane + 64 * nwv * v, K4 - 1);
        rv[t][v] = *(const f4*)(a.x + (uint64_t)(a.xrow0 + t0 + min(t, nt - 1)) * a.ldx + 4 * c);
        if constexpr ((PRO & PRO_XSUM) != 0)  // one token, k <= 512 * waves (host-checked)
          rv[t][v] = (rv[t][v] + *(const f4*)(a.xpart + 4 * c)) + *(const f4*)(a.xpart + a.xpartstride + 4 * c);
      }
  }
  // the first batch: activation items, then weights (they return in that order)
  ItemsOf<NT, PRO> it, itt;
  WUnit w[NU], wt;
  load_items<NT, PRO, false, NU>(it, a, t0, nt, 0, cnt, sp, split, lane);
#pragma unroll
  for (int u = 0; u < NU; u++) load_group<QT>(w[u], a.qs, nb, tile, sp + u * split, lane, r, (uint32_t)u < cnt);
  if (NT == 1 && has_tail) {  // (several tokens: loaded when the tail comes, to hold fewer registers)
    load_items<NT, PRO, true, NU>(itt, a, t0, nt, 0, cnt, sp, split, lane);
    load_unit<QT>(wt, a.qs, nb, tile, ng, ng, a.tail, lane, r);
  }
  // the epilogue's own inputs (issued after the prologue's: the RoPE rows wait
  // for the position), in flight during the products
  const bool active = sw == 0 && has_tile;
  const int tA = 2 * q, tB = 2 * q + 1;
  const bool okA = tA < nt, okB = NT > 1 && tB < nt;
  const EpiIn pre = epi_load<EPI>(a, tile, r, active, t0 + tA, okA, t0 + tB, okB);
  float rs[NT];
  if (RMS) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
      float ss = 0;
#pragma unroll
      for (int v = 0; v < RV; v++)
        if (wave * 64 + lane + 64 * nwv * v < K4)
          ss += rv[t][v][0] * rv[t][v][0] + rv[t][v][1] * rv[t][v][1] + rv[t][v][2] * rv[t][v][2] +
                rv[t][v][3] * rv[t][v][3];
      for (uint32_t c = wave * 64 + lane + 64 * nwv * RV; c < K4; c += 64 * nwv) {  // longer rows
        const f4 x4 = *(const f4*)(a.x + (uint64_t)(a.xrow0 + t0 + min(t, nt - 1)) * a.ldx + 4 * c);
        ss += x4[0] * x4[0] + x4[1] * x4[1] + x4[2] * x4[2] + x4[3] * x4[3];
      }
      ss = wave_sum_dpp(ss);
      if (lane == 0) misc[wave * NT + t] = ss;
    }
    if constexpr ((PRO & PRO_XSUM) != 0)  // the summed residual row, for the layer's K3
      if (blockIdx.x == 0)
#pragma unroll
        for (int v = 0; v < RV; v++)
          if (wave * 64 + lane + 64 * nwv * v < K4) *(f4*)(a.xout + 4 * (wave * 64 + lane + 64 * nwv * v)) = rv[0][v];
  }
  // cpu.go:90-95, from the waves' partial sums (every thread, the same order)
  auto rms_scales = [&]() {
#pragma unroll
    for (int t = 0; t < NT; t++) {
      float ss = 0;
      for (uint32_t v = 0; v < nwv; v++) ss += misc[v * NT + t];
      rs[t] = t < nt ? rms_scale((double)(ss / (float)a.k + a.eps)) : 0.f;
    }
  };
  // LATE (f32 activations): the units are staged as x * w and the products
  // scaled by each token's 1/rms at the end, so no wave waits for the
  // others' sums before its products.  PRO_Q8 quantises x * s * w itself and
  // needs s first.
  constexpr bool LATE = RMS && !Q8;
  if (RMS && !LATE) {
    __syncthreads();
    rms_scales();
  }
  if (LATE)
#pragma unroll
    for (int t = 0; t < NT; t++) rs[t] = 1.f;

  float acc0 = 0, acc1 = 0;
  int ex[UB][NT];
  for (uint32_t i0 = 0; i0 < cnt; i0 += NU) {
    if (i0 > 0) {
      load_items<NT, PRO, false, NU>(it, a, t0, nt, i0, cnt, sp, split, lane);
#pragma unroll
      for (int u = 0; u < NU; u++) load_group<QT>(w[u], a.qs, nb, tile, sp + (i0 + u) * split, lane, r, i0 + u < cnt);
    }
    if constexpr ((PRO & PRO_MERGE) != 0) merge_items<PRO, NU>(it, a, keep);
    stage_items<QT, NT, PRO, NU>(it, rs, lane, ops, sums, dxs, ex);
#pragma unroll
    for (int u = 0; u < NU; u++)
      if (i0 + u < cnt) unit_products<QT, NT, Q8, false>(w[u], u, 4, ops, sums, dxs, ex, q, slot, acc0, acc1);
  }
  if (has_tail) {
    if (NT > 1) {
      load_items<NT, PRO, true, NU>(itt, a, t0, nt, 0, cnt, sp, split, lane);
      load_unit<QT>(wt, a.qs, nb, tile, ng, ng, a.tail, lane, r);
    }
    if constexpr ((PRO & PRO_MERGE) != 0) merge_items<PRO, NU>(itt, a, keep);
    stage_items<QT, NT, PRO, NU>(itt, rs, lane, ops, sums, dxs, ex);
    unit_products<QT, NT, Q8, true>(wt, 0, (int)a.tail, ops, sums, dxs, ex, q, slot, acc0, acc1);
  }
  if (LATE) {
    __syncthreads();  // every wave's sum of squares is in misc
    rms_scales();
    acc0 *= rs[min(2 * q, NT - 1)];
    acc1 *= rs[min(2 * q + 1, NT - 1)];
  }
  // ---- split-K: partial sums of the waves of a tile, added in a fixed order
  // (every partial read issued before the sums)
  if (split > 1) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    f2* p2 = (f2*)part;
    p2[wave * 64 + lane] = f2{acc0, acc1};
    __syncthreads();
    if (sw == 0) {
      f2 pv[15];
#pragma unroll
      for (int k = 0; k < 15; k++) pv[k] = p2[(wave + min((uint32_t)k + 1, split - 1)) * 64 + lane];
#pragma unroll
      for (int k = 0; k < 15; k++)
        if ((uint32_t)k + 1 < split) {
          acc0 += pv[k][0];
          acc1 += pv[k][1];
        }
    }
  }
  // ---- epilogue: lane holds rows r of the tile for tokens 2q and 2q+1
  const float vA = okA ? acc0 : 0.f;
  const float vB = okB ? acc1 : 0.f;
  row_epilogue<EPI>(a, tile, r, active, t0 + tA, okA, vA, t0 + tB, okB, vB, &pre,
                    kp > 1 ? a.y + kpart * a.pstride : nullptr);
  if (EPI == EPI_ARGMAX) {
    const uint32_t lr = row_of_pos(tile * 16 + r, a.map, a.map_hd, a.map_seg0, a.map_seg1, a.ff);
    const bool ok = active && lr < a.rows && q == 0 && okA && vA == vA;
    argmax_partial(a, misc, ok ? vA : -INFINITY, ok ? lr : 0xffffffffu);
  }
}

// ----------------------------------------------------------- dispatch

template <uint32_t QT, int NT, int PRO, int EPI, int NU>
static int launch_nu(const GemvArgs& a, dim3 grid, uint32_t lds, hipStream_t s) {
  auto k = gemv_kernel<QT, NT, PRO, EPI, NU>;
  static bool big = false;
  if (lds > 65536 && !big) {
    LLM_HIP(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    big = true;
  }
  hipLaunchKernelGGL(k, grid, dim3(64 * a.waves), lds, s, a);
  LLM_HIP(hipGetLastError());
  return 0;
}

// Units a wave stages per batch: two when no wave has more than two groups
// (no load is issued for a third or fourth), else four.
template <uint32_t QT, int NT, int PRO, int EPI>
static int launch_one(const GemvArgs& a, dim3 grid, uint32_t lds, hipStream_t s) {
  const uint32_t kp = a.kparts > 1 ? a.kparts : 1;  // a part's share of the groups
  const uint32_t per_wave = ((a.ng + kp - 1) / kp + a.split - 1) / a.split;
  if (per_wave <= 2) return launch_nu<QT, NT, PRO, EPI, 2>(a, grid, lds, s);
  return launch_nu<QT, NT, PRO, EPI, 4>(a, grid, lds, s);
}

template <uint32_t QT, int NT, int Q>
static int launch_nt_q(const GemvArgs& a, int pro, int epi, dim3 grid, uint32_t lds, hipStream_t s) {
  constexpr int PP = PRO_PLAIN | Q, PR = PRO_RMS | Q;
  if (pro & PRO_XSUM) {
    if constexpr (NT == 1)
      if ((pro & PRO_RMS) && epi == EPI_QKV) {
        if (Q == 0) return launch_one<QT, 1, PRO_RMS | PRO_XSUM, EPI_QKV>(a, grid, lds, s);
        return launch_one<QT, 1, PRO_RMS | PRO_Q8 | PRO_XSUM, EPI_QKV>(a, grid, lds, s);
      }
    return set_error(LLMHIP_ERR_ARG, "llm: gemv: the summing prologue is for one token into EPI_QKV");
  }
  if (pro & PRO_MERGE) {  // two units per staging batch (more would spill the partials)
    if constexpr (Q == 0 && NT == 1)
      if (epi == EPI_ACC && !(pro & (PRO_RMS | PRO_Q8)) && a.waves <= 8 && (a.ng + a.split - 1) / a.split <= 2)
        switch (merge_chunks(pro)) {
          case 2: return launch_nu<QT, 1, merge_pro(2), EPI_ACC, 2>(a, grid, lds, s);
          case 4: return launch_nu<QT, 1, merge_pro(4), EPI_ACC, 2>(a, grid, lds, s);
          case 6: return launch_nu<QT, 1, merge_pro(6), EPI_ACC, 2>(a, grid, lds, s);
          case 8: return launch_nu<QT, 1, merge_pro(8), EPI_ACC, 2>(a, grid, lds, s);
          case 10: return launch_nu<QT, 1, merge_pro(10), EPI_ACC, 2>(a, grid, lds, s);
          case 12: return launch_nu<QT, 1, merge_pro(12), EPI_ACC, 2>(a, grid, lds, s);
          case 14: return launch_nu<QT, 1, merge_pro(14), EPI_ACC, 2>(a, grid, lds, s);
          case 16: return launch_nu<QT, 1, merge_pro(16), EPI_ACC, 2>(a, grid, lds, s);
        }
    return set_error(LLMHIP_ERR_ARG,
                     "llm: gemv: the merging prologue is for one f32 token into EPI_ACC, <= 8 waves, <= 2 units each");
  }
  switch ((pro & PRO_RMS) * 8 + epi) {
    case PRO_PLAIN * 8 + EPI_STORE: return launch_one<QT, NT, PP, EPI_STORE>(a, grid, lds, s);
    case PRO_PLAIN * 8 + EPI_ACC: return launch_one<QT, NT, PP, EPI_ACC>(a, grid, lds, s);
    case PRO_RMS * 8 + EPI_QKV: return launch_one<QT, NT, PR, EPI_QKV>(a, grid, lds, s);
    case PRO_RMS * 8 + EPI_GATEUP: return launch_one<QT, NT, PR, EPI_GATEUP>(a, grid, lds, s);
    case PRO_RMS * 8 + EPI_STORE: return launch_one<QT, NT, PR, EPI_STORE>(a, grid, lds, s);
    case PRO_RMS * 8 + EPI_SWIGLU: return launch_one<QT, NT, PR, EPI_SWIGLU>(a, grid, lds, s);
  }
  if ((pro & PRO_RMS) && epi == EPI_ARGMAX && NT == 1) return launch_one<QT, 1, PR, EPI_ARGMAX>(a, grid, lds, s);
  return set_error(LLMHIP_ERR_ARG, "llm: gemv: unsupported prologue/epilogue %d/%d", pro, epi);
}

template <uint32_t QT, int NT>
static int launch_nt(const GemvArgs& a, int pro, int epi, dim3 grid, uint32_t lds, hipStream_t s) {
  if (pro & PRO_Q8) return launch_nt_q<QT, NT, PRO_Q8>(a, pro, epi, grid, lds, s);
  return launch_nt_q<QT, NT, 0>(a, pro, epi, grid, lds, s);
}

template <uint32_t QT, int PRO, int EPI>
static int launch_stream(const GemvArgs& a, hipStream_t s) {
  const Lds L = lds_layout(1, QT, a.nb, a.swaves, (PRO & PRO_Q8) != 0);
  const dim3 g(a.stream), b(64 * a.swaves);
  switch (a.ng) {  // a whole tile in flight per wave where its groups fit the registers
    case 7:  // (f32 activations: the integer form's digits after the layout)
      hipLaunchKernelGGL((gemv_stream_kernel<QT, PRO, EPI, 7>), g, b,
                         L.total + ((PRO & PRO_Q8) ? 0 : i8_lds_bytes(a.nb)), s, a);
      break;
    default: hipLaunchKernelGGL((gemv_stream_kernel<QT, PRO, EPI, 0>), g, b, L.total, s, a);
  }
  LLM_HIP(hipGetLastError());
  return 0;
}

template <uint32_t QT>
int gemv_launch_qt(const GemvArgs& a, int pro, int epi, hipStream_t s) {
  if (a.stream && a.ntok == 1) {
    // the streaming kernel walks whole groups of four blocks only
    if (a.tail != 0)
      return set_error(LLMHIP_ERR_ARG, "llm: gemv: the streaming kernel takes no tail blocks (k %u)", a.k);
    switch (pro * 8 + epi) {
      case PRO_PLAIN * 8 + EPI_STORE: return launch_stream<QT, PRO_PLAIN, EPI_STORE>(a, s);
      case PRO_PLAIN * 8 + EPI_ACC: return launch_stream<QT, PRO_PLAIN, EPI_ACC>(a, s);
      case PRO_RMS * 8 + EPI_STORE: return launch_stream<QT, PRO_RMS, EPI_STORE>(a, s);
      case PRO_RMS * 8 + EPI_ARGMAX: return launch_stream<QT, PRO_RMS, EPI_ARGMAX>(a, s);
      case (PRO_RMS | PRO_Q8) * 8 + EPI_ARGMAX: return launch_stream<QT, PRO_RMS | PRO_Q8, EPI_ARGMAX>(a, s);
      case (PRO_PLAIN | PRO_Q8) * 8 + EPI_STORE: return launch_stream<QT, PRO_PLAIN | PRO_Q8, EPI_STORE>(a, s);
    }
    return set_error(LLMHIP_ERR_ARG, "llm: gemv: no streaming form of prologue/epilogue %d/%d", pro, epi);
  }
  int nt = a.ntok <= 1 ? 1 : a.ntok <= 2 ? 2 : 4;
  const uint32_t lds = decode_lds(nt, a.waves);
  if (lds > 160 * 1024)
    return set_error(LLMHIP_ERR_ARG, "llm: gemv: %u waves of %d tokens need %u bytes of LDS", a.waves, nt, lds);
  if (epi == EPI_ARGMAX && a.ntok != 1) return set_error(LLMHIP_ERR_ARG, "llm: gemv: argmax epilogue needs one token");
  dim3 grid(gemv_groups(a), (a.ntok + nt - 1) / nt);
  switch (nt) {
    case 1: return launch_nt<QT, 1>(a, pro, epi, grid, lds, s);
    case 2: return launch_nt<QT, 2>(a, pro, epi, grid, lds, s);
    default: return launch_nt<QT, 4>(a, pro, epi, grid, lds, s);
  }
}

template <uint32_t QT>
int repack_launch_qt(const QMat& m, const uint8_t* raw_dev, uint64_t n, uint64_t blk0, uint64_t row_off,
                     uint32_t map, uint32_t hd, uint32_t seg0, uint32_t seg1, uint32_t ff, hipStream_t s) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(repack_kernel<QT>, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, raw_dev, n, blk0,
                     row_off, m.qs, (uint64_t)m.g.tiles, m.g.nb, m.g.ng, m.g.tail, map, hd, seg0, seg1, ff);
  LLM_HIP(hipGetLastError());
  return 0;
}

template <uint32_t QT>
int dequant_launch_qt(const QMat& m, float* out, uint32_t map, uint32_t hd, uint32_t seg0, uint32_t seg1, uint32_t ff,
                      hipStream_t s) {
  uint64_t n = m.g.rows * m.g.nb;
  if (n == 0) return 0;
  hipLaunchKernelGGL(dequant_kernel<QT>, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, m.qs,
                     (uint64_t)m.g.tiles, (uint32_t)m.g.rows, m.g.nb, m.g.ng, m.g.tail, map, hd, seg0, seg1, ff, out);
  LLM_HIP(hipGetLastError());
  return 0;
}

template <uint32_t QT>
int embed_launch_qt(const QMat& m, const int32_t* tokens, const uint32_t* state, float* x, uint32_t ntok,
                    hipStream_t s) {
  hipLaunchKernelGGL(embed_kernel<QT>, dim3(1, ntok), dim3(64), 0, s, m.qs, (uint64_t)m.g.tiles, m.g.nb, m.g.ng,
                     m.g.tail, tokens, state, x);
  LLM_HIP(hipGetLastError());
  return 0;
}

template <uint32_t QT, int EPI, bool Q8, int GT, bool EM = false>
static void gemm_go(const GemvArgs& a, uint32_t waves, hipStream_t s) {
  dim3 grid((a.tiles + GT - 1) / GT, a.tg);
  hipLaunchKernelGGL((gemm_kernel<QT, EPI, Q8, GT, EM>), grid, dim3(64 * waves), 0, s, a);
}

template <uint32_t QT, int EPI>
static void gemm_shape(const GemvArgs& a, hipStream_t s) {
  // Measured on MI355X at 64 tokens (prep + product, Q4_0): 16 tokens per
  // workgroup beat 32 at every layer shape (more workgroups, lower
  // registers: 9728x896 12.6 against 15.2 us, 896x4864 11.8 against 16.6);
  // two tiles per workgroup pay on tall matrices (9728x896: 12.6 against 15.7
  // with one, 14.6 with four); short matrices with many block groups take
  // eight waves, tall ones four.  In the prefill itself (config 3, two
  // chunks at once): long rows (896x4864) take two tiles and eight waves
  // (87.4k -> 89.4k tok/s), the [q; k; v] product two tiles and four waves
  // (-> 90.1k with both); W_o keeps one tile and eight waves.
  const uint32_t units = a.ng + (a.tail ? 1 : 0);
  const bool gt2 = a.tiles >= 256 || units >= 16 || EPI == EPI_QKV;
  const uint32_t waves = units > 4 && (a.tiles < 256 && EPI != EPI_QKV) ? 8 : 4;
  if constexpr (EPI == EPI_GATEUP) {
    if (a.op_xp) {  // the down projection's operands too: four tiles (gemm_launch checked q8 = 0)
      gemm_go<QT, EPI, false, 4, true>(a, 4, s);
      return;
    }
  }
  if (a.q8) {
    if (gt2) gemm_go<QT, EPI, true, 2>(a, waves, s);
    else gemm_go<QT, EPI, true, 1>(a, waves, s);
  } else {
    if (gt2) gemm_go<QT, EPI, false, 2>(a, waves, s);
    else gemm_go<QT, EPI, false, 1>(a, waves, s);
  }
}

template <uint32_t QT>
int gemm_launch_qt(const GemvArgs& a, int epi, hipStream_t s) {
  switch (epi) {
    case EPI_STORE: gemm_shape<QT, EPI_STORE>(a, s); break;
    case EPI_ACC: gemm_shape<QT, EPI_ACC>(a, s); break;
    case EPI_QKV: gemm_shape<QT, EPI_QKV>(a, s); break;
    case EPI_GATEUP: gemm_shape<QT, EPI_GATEUP>(a, s); break;
    case EPI_SWIGLU: gemm_shape<QT, EPI_SWIGLU>(a, s); break;
    default: return set_error(LLMHIP_ERR_ARG, "llm: gemm: unsupported epilogue %d", epi);
  }
  LLM_HIP(hipGetLastError());
  return 0;
}

#define LLMHIP_INSTANTIATE(QT)                                                                                   \
  template int gemv_launch_qt<QT>(const GemvArgs&, int, int, hipStream_t);                                     \
  template int repack_launch_qt<QT>(const QMat&, const uint8_t*, uint64_t, uint64_t, uint64_t, uint32_t,       \
                                    uint32_t, uint32_t, uint32_t, uint32_t, hipStream_t);                      \
  template int dequant_launch_qt<QT>(const QMat&, float*, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,    \
                                     hipStream_t);                                                             \
  template int embed_launch_qt<QT>(const QMat&, const int32_t*, const uint32_t*, float*, uint32_t, hipStream_t); \
  template int gemm_launch_qt<QT>(const GemvArgs&, int, hipStream_t);

}  // namespace llmhip
