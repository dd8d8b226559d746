/*
 * cpuref — TEST INFRASTRUCTURE ONLY. A plain-C restatement of the reference's
 * CPU f32 forward pass, used as the parity oracle for the HIP path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker (or the timed CPU comparator); the
 * product library never links, loads or falls back to it.
 *
 * Every function follows a reference function statement by statement, with
 * f32 arithmetic everywhere the reference uses float32, float64 exactly where
 * the reference widens, and no contraction (build with -ffp-contract=off,
 * no -ffast-math).  Citations are to /root/reference.
 *
 *   cpuref_f16_to_f32    f16.go:6-28      pinned: all 65536 patterns vs numpy, known values
 *   cpuref_f32_to_f16    f16.go:30-66     pinned: all finite f16 round trips, numpy on 2^20
 *                                         random f32 + halfway cases, known values
 *   cpuref_rmsnorm       cpu.go:81-98     pinned: float64 numpy formula, tolerance
 *   cpuref_matvec        cpu.go:143-222   pinned: float64 brute force on dequantised
 *                                         weights; K=32 single-block closed forms
 *   cpuref_dequant       cpu.go:230-254 (embedding) and the per-weight value implied
 *                        by cpu.go:164-215; pinned: closed forms d*(q-8), d*q+m, d*i8
 *   cpuref_rope          cpu.go:371-385   pinned: kernels_test.go:24-58 NEOX invariant
 *                                         (exact), rotation-norm invariant, pos 0 = identity
 *   cpuref_argmax        cpu.go:389-397   pinned: ties, NaN, all-equal special cases
 *   cpuref_forward       cpu.go:225-366   pinned: independent vectorised float64 numpy
 *                                         forward on tiny models (attention weights sum
 *                                         to 1, single-position att = v)
 *   cpuref_matvec_q8     cpu.go:117-140, 166-214  pinned with ExactGGML below
 *   F16KV mode           cpu.go:22-24, 298-299  pinned: the float64 forward with a
 *                                         binary16-rounded cache (numpy RNE), closer to
 *                                         it than to the exact-cache forward
 *   quantize_q8          cpu.go:117-140   pinned: halfway cases (round half away from
 *                                         zero), the amax element at +-127, the Q8_1 sum
 *                                         from the unrounded scale, the half-step bound
 *   ExactGGML mode       cpu.go:15-21     pinned: a float64 forward that quantises every
 *                                         matrix input the same way (f32 ops), integer
 *                                         block dots, binary16 cache: within 1e-6, and
 *                                         1000x closer to it than to the unquantised one
 *   gguf reader / config_from  gguf/gguf.go:292-407, config.go:29-73: pinned by the
 *                        reference's gguf_test.go cases and refusal cases of config.go
 *
 * What cannot be pinned without a Go toolchain (none in this image): the last ulp
 * of Go's math.Exp / math.Pow / math.Sincos against glibc's exp / pow / sincos.
 */
#define _GNU_SOURCE
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

static __thread char g_err[512];

static int fail(const char* fmt, const char* a) {
  snprintf(g_err, sizeof g_err, fmt, a);
  return -1;
}

EXPORT const char* cpuref_error(void) { return g_err; }

/* ---------------------------------------------------------------- f16.go */

static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* F16ToF32, f16.go:6-28: exact, subnormals normalised, NaN payload kept. */
EXPORT float cpuref_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (uint32_t)(h >> 10) & 0x1f;
  uint32_t man = (uint32_t)h & 0x3ff;
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);
    uint32_t e = 127 - 15 + 1;
    while ((man & 0x400) == 0) {
      man <<= 1;
      e--;
    }
    man &= 0x3ff;
    return bits_f32(sign | e << 23 | man << 13);
  }
  if (exp == 31) return bits_f32(sign | 0xffu << 23 | man << 13);
  return bits_f32(sign | (exp + 127 - 15) << 23 | man << 13);
}

/* F32ToF16, f16.go:30-66: round to nearest even. */
EXPORT uint16_t cpuref_f32_to_f16(float f) {
  uint32_t b = f32_bits(f);
  uint16_t sign = (uint16_t)(b >> 16) & 0x8000;
  int32_t exp = (int32_t)(b >> 23) & 0xff;
  uint32_t man = b & 0x7fffff;
  if (exp == 0xff) {
    if (man != 0) return sign | 0x7e00;
    return sign | 0x7c00;
  }
  int32_t e = exp - 127 + 15;
  if (e >= 31) return sign | 0x7c00;
  if (e <= 0) {
    if (e < -10) return sign;
    man |= 0x800000;
    uint32_t shift = (uint32_t)(14 - e);
    uint32_t h = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1) == 1)) h++;
    return sign | (uint16_t)h;
  }
  uint32_t h = (uint32_t)e << 10 | man >> 13;
  uint32_t rem = man & 0x1fff;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1) == 1)) h++;
  return sign | (uint16_t)h;
}

/* RoundF16, f16.go:68. */
EXPORT float cpuref_round_f16(float f) { return cpuref_f16_to_f32(cpuref_f32_to_f16(f)); }

EXPORT void cpuref_f16_to_f32_n(const uint16_t* h, float* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = cpuref_f16_to_f32(h[i]);
}

EXPORT void cpuref_f32_to_f16_n(const float* f, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = cpuref_f32_to_f16(f[i]);
}

/* Go's built-in max for floats: NaN wins, +0 above -0. */
static inline float go_maxf(float a, float b) {
  if (a != a || b != b) return NAN;
  if (a > b) return a;
  if (b > a) return b;
  return signbit(a) ? b : a;
}

/* ------------------------------------------------------------ ggml types */

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q6_K = 14 };

/* gguf.Type.BlockSize, gguf/gguf.go:72-92. */
static int block_size(uint32_t t, uint64_t* elems, uint64_t* bytes) {
  switch (t) {
    case T_F32: *elems = 1; *bytes = 4; return 1;
    case T_F16: *elems = 1; *bytes = 2; return 1;
    case T_Q4_0: *elems = 32; *bytes = 18; return 1;
    case T_Q4_1: *elems = 32; *bytes = 20; return 1;
    case T_Q5_0: *elems = 32; *bytes = 22; return 1;
    case T_Q5_1: *elems = 32; *bytes = 24; return 1;
    case T_Q8_0: *elems = 32; *bytes = 34; return 1;
    case T_Q6_K: *elems = 256; *bytes = 210; return 1;
  }
  return 0;
}

static inline uint16_t u16le(const uint8_t* b) { return (uint16_t)(b[0] | b[1] << 8); }

/* --------------------------------------------------------------- cpu.go */

/* rmsNorm, cpu.go:81-98 (the f32 sum, rmsF64 off). */
EXPORT void cpuref_rmsnorm(float* dst, const float* x, const float* w, int n, float eps) {
  float ss = 0;
  for (int i = 0; i < n; i++) ss += x[i] * x[i];
  float s = (float)(1 / sqrt((double)(ss / (float)n + eps)));
  for (int i = 0; i < n; i++) dst[i] = x[i] * s * w[i];
}

/* quantizeQ8, cpu.go:117-140 (ExactGGML activations). */
typedef struct {
  float* d;
  float* s;
  int8_t* qs;
} q8act;

static void quantize_q8(const float* x, int n, q8act* y) {
  int nb = n / 32;
  for (int i = 0; i < nb; i++) {
    float amax = 0;
    for (int j = 0; j < 32; j++) amax = go_maxf(amax, (float)fabs((double)x[i * 32 + j]));
    float d = amax / 127;
    float id = 0;
    if (d != 0) id = 1 / d;
    y->d[i] = cpuref_round_f16(d);
    int sum = 0;
    for (int j = 0; j < 32; j++) {
      int8_t q = (int8_t)round((double)(x[i * 32 + j] * id));
      y->qs[i * 32 + j] = q;
      sum += q;
    }
    y->s[i] = cpuref_round_f16(d * (float)sum);
  }
}

EXPORT void cpuref_quantize_q8(const float* x, int n, float* d, float* s, int8_t* qs) {
  q8act y = {d, s, qs};
  quantize_q8(x, n, &y);
}

/* One output row of matvec, cpu.go:158-221. */
static float matvec_row(const float* x, uint32_t type, const uint8_t* row, int in, const q8act* qx) {
  float sum = 0;
  int nb = in / 32;
  for (int b = 0; b < nb; b++) {
    switch (type) {
      case T_Q4_0: {
        const uint8_t* blk = row + (size_t)b * 18;
        float d = cpuref_f16_to_f32(u16le(blk));
        if (qx) {
          int si = 0;
          for (int j = 0; j < 16; j++) {
            si += ((int)(blk[2 + j] & 15) - 8) * (int)qx->qs[b * 32 + j];
            si += ((int)(blk[2 + j] >> 4) - 8) * (int)qx->qs[b * 32 + j + 16];
          }
          sum += d * qx->d[b] * (float)si;
        } else {
          float s = 0;
          for (int j = 0; j < 16; j++) {
            s += (float)((int)(blk[2 + j] & 15) - 8) * x[b * 32 + j];
            s += (float)((int)(blk[2 + j] >> 4) - 8) * x[b * 32 + j + 16];
          }
          sum += d * s;
        }
        break;
      }
      case T_Q4_1: {
        const uint8_t* blk = row + (size_t)b * 20;
        float d = cpuref_f16_to_f32(u16le(blk)), mn = cpuref_f16_to_f32(u16le(blk + 2));
        if (qx) {
          int si = 0;
          for (int j = 0; j < 16; j++) {
            si += (int)(blk[4 + j] & 15) * (int)qx->qs[b * 32 + j];
            si += (int)(blk[4 + j] >> 4) * (int)qx->qs[b * 32 + j + 16];
          }
          sum += d * qx->d[b] * (float)si + mn * qx->s[b];
        } else {
          float s = 0, sx = 0;
          for (int j = 0; j < 16; j++) {
            s += (float)(blk[4 + j] & 15) * x[b * 32 + j];
            s += (float)(blk[4 + j] >> 4) * x[b * 32 + j + 16];
          }
          for (int j = 0; j < 32; j++) sx += x[b * 32 + j];
          sum += d * s + mn * sx;
        }
        break;
      }
      case T_Q8_0: {
        const uint8_t* blk = row + (size_t)b * 34;
        float d = cpuref_f16_to_f32(u16le(blk));
        if (qx) {
          int si = 0;
          for (int j = 0; j < 32; j++) si += (int)(int8_t)blk[2 + j] * (int)qx->qs[b * 32 + j];
          sum += d * qx->d[b] * (float)si;
        } else {
          float s = 0;
          for (int j = 0; j < 32; j++) s += (float)(int8_t)blk[2 + j] * x[b * 32 + j];
          sum += d * s;
        }
        break;
      }
    }
  }
  return sum;
}

/* matvec, cpu.go:143-222: dst = W x for a [in, out] tensor. Rows are
 * independent and each keeps its own summation order, so splitting the rows
 * over threads gives bit-identical results. */
static int matvec(float* dst, const float* x, uint32_t type, const uint8_t* data, int in, int out,
                  const q8act* qx, int nthreads) {
  if (type == T_F32) {
    const float* w = (const float*)data; /* little-endian host */
#pragma omp parallel for num_threads(nthreads) if (nthreads > 1) schedule(static)
    for (int o = 0; o < out; o++) {
      float s = 0;
      for (int i = 0; i < in; i++) s += w[(size_t)o * in + i] * x[i];
      dst[o] = s;
    }
    return 0;
  }
  uint64_t be, bb;
  if ((type != T_Q4_0 && type != T_Q4_1 && type != T_Q8_0) || !block_size(type, &be, &bb)) {
    snprintf(g_err, sizeof g_err, "llm: CPU matvec: ggml type %u", type);
    return -1;
  }
  size_t rowBytes = (size_t)(in / 32) * bb;
#pragma omp parallel for num_threads(nthreads) if (nthreads > 1) schedule(static)
  for (int o = 0; o < out; o++) dst[o] = matvec_row(x, type, data + (size_t)o * rowBytes, in, qx);
  return 0;
}

EXPORT int cpuref_matvec(float* dst, const float* x, uint32_t type, const uint8_t* data, int in, int out,
                         int nthreads) {
  return matvec(dst, x, type, data, in, out, NULL, nthreads < 1 ? 1 : nthreads);
}

/* The ExactGGML form of matvec: x quantised by quantizeQ8, then the integer
 * block products (the qx != nil branches of cpu.go:166-214). */
EXPORT int cpuref_matvec_q8(float* dst, const float* x, uint32_t type, const uint8_t* data, int in, int out,
                            int nthreads) {
  if (in % 32) {
    snprintf(g_err, sizeof g_err, "llm: CPU matvec_q8: %d inputs", in);
    return -1;
  }
  int nb = in / 32;
  float* d = (float*)malloc((size_t)nb * 8);
  int8_t* qs = (int8_t*)malloc((size_t)in);
  q8act qx = {d, d + nb, qs};
  quantize_q8(x, in, &qx);
  int rc = matvec(dst, x, type, data, in, out, &qx, nthreads < 1 ? 1 : nthreads);
  free(d);
  free(qs);
  return rc;
}

/* The value of every weight, as the CPU path uses it: the embedding gather
 * (cpu.go:233-251) for Q8_0 and Q4_0, and d*q+m for Q4_1 (the term of
 * cpu.go:199 per element). Used to pin the GPU's dequantisation bit for bit. */
EXPORT int cpuref_dequant(float* out, uint32_t type, const uint8_t* data, uint64_t nblocks) {
  for (uint64_t b = 0; b < nblocks; b++) {
    float* o = out + b * 32;
    switch (type) {
      case T_Q4_0: {
        const uint8_t* blk = data + b * 18;
        float d = cpuref_f16_to_f32(u16le(blk));
        for (int j = 0; j < 16; j++) {
          o[j] = d * (float)((int)(blk[2 + j] & 15) - 8);
          o[j + 16] = d * (float)((int)(blk[2 + j] >> 4) - 8);
        }
        break;
      }
      case T_Q4_1: {
        const uint8_t* blk = data + b * 20;
        float d = cpuref_f16_to_f32(u16le(blk)), m = cpuref_f16_to_f32(u16le(blk + 2));
        for (int j = 0; j < 16; j++) {
          o[j] = d * (float)(blk[4 + j] & 15) + m;
          o[j + 16] = d * (float)(blk[4 + j] >> 4) + m;
        }
        break;
      }
      case T_Q8_0: {
        const uint8_t* blk = data + b * 34;
        float d = cpuref_f16_to_f32(u16le(blk));
        for (int j = 0; j < 32; j++) o[j] = d * (float)(int8_t)blk[2 + j];
        break;
      }
      default:
        snprintf(g_err, sizeof g_err, "llm: dequant: ggml type %u", type);
        return -1;
    }
  }
  return 0;
}

/* rope, cpu.go:371-385. */
EXPORT void cpuref_rope(float* x, int pos, int heads, int dim, float base, int neox) {
  for (int h = 0; h < heads; h++) {
    for (int i = 0; i < dim / 2; i++) {
      double theta = (double)pos * pow((double)base, -(double)(2 * i) / (double)dim);
      double s, c;
      sincos(theta, &s, &c);
      int ia = h * dim + 2 * i, ib = h * dim + 2 * i + 1;
      if (neox) {
        ia = h * dim + i;
        ib = h * dim + i + dim / 2;
      }
      float a = x[ia], b = x[ib];
      x[ia] = a * (float)c - b * (float)s;
      x[ib] = a * (float)s + b * (float)c;
    }
  }
}

/* The host RoPE table of the GPU path, gpu.go:524-534: cs[(pos*hd/2+i)*2+{0,1}]
 * = f32(cos), f32(sin) of the same theta as cpu.go:374. */
EXPORT void cpuref_rope_table(float* cs, int ctx, int hd, float base) {
  int hp = hd / 2;
  for (int pos = 0; pos < ctx; pos++)
    for (int i = 0; i < hp; i++) {
      double theta = (double)pos * pow((double)base, -(double)(2 * i) / (double)hd);
      double s, c;
      sincos(theta, &s, &c);
      cs[(pos * hp + i) * 2] = (float)c;
      cs[(pos * hp + i) * 2 + 1] = (float)s;
    }
}

/* Argmax, cpu.go:389-397: the first index of the maximum; NaN never wins
 * (and a NaN at index 0 is never displaced). */
EXPORT int32_t cpuref_argmax(const float* l, int n) {
  int best = 0;
  for (int i = 0; i < n; i++)
    if (l[i] > l[best]) best = i;
  return best;
}

/* -------------------------------------------------- gguf reader (oracle) */

enum { V_U8, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STRING, V_ARRAY, V_U64, V_I64, V_F64 };

typedef struct {
  char* key;
  int kind; /* 0 uint, 1 int, 2 float, 3 string, 4 bool, 5 array */
  uint64_t u;
  int64_t i;
  double f;
  char* s;
} meta_kv;

typedef struct {
  char* name;
  uint32_t ndims;
  uint64_t dims[4];
  uint32_t type;
  uint64_t offset, size;
  uint8_t* data;
} tensor_t;

typedef struct {
  const uint8_t* p;
  size_t n, pos;
  int bad;
} rd_t;

static int rd(rd_t* r, void* dst, size_t k) {
  if (r->bad || r->pos + k > r->n) {
    r->bad = 1;
    return 0;
  }
  memcpy(dst, r->p + r->pos, k);
  r->pos += k;
  return 1;
}
static uint32_t rd32(rd_t* r) {
  uint32_t v = 0;
  rd(r, &v, 4);
  return v;
}
static uint64_t rd64(rd_t* r) {
  uint64_t v = 0;
  rd(r, &v, 8);
  return v;
}
static char* rdstr(rd_t* r) {
  uint64_t n = rd64(r);
  if (r->bad || n > (1u << 24) || r->pos + n > r->n) {
    r->bad = 1;
    return NULL;
  }
  char* s = (char*)malloc(n + 1);
  memcpy(s, r->p + r->pos, n);
  s[n] = 0;
  r->pos += n;
  return s;
}

/* A metadata value, gguf/gguf.go:210-289 (arrays are skipped: the config
 * reads none). */
static void rdval(rd_t* r, uint32_t t, meta_kv* kv, int depth) {
  uint8_t b1 = 0;
  uint16_t b2 = 0;
  switch (t) {
    case V_U8: rd(r, &b1, 1); kv->kind = 0; kv->u = b1; return;
    case V_I8: rd(r, &b1, 1); kv->kind = 1; kv->i = (int8_t)b1; return;
    case V_BOOL: rd(r, &b1, 1); kv->kind = 4; kv->u = b1 != 0; return;
    case V_U16: rd(r, &b2, 2); kv->kind = 0; kv->u = b2; return;
    case V_I16: rd(r, &b2, 2); kv->kind = 1; kv->i = (int16_t)b2; return;
    case V_U32: kv->kind = 0; kv->u = rd32(r); return;
    case V_I32: kv->kind = 1; kv->i = (int32_t)rd32(r); return;
    case V_F32: { uint32_t v = rd32(r); kv->kind = 2; kv->f = (double)bits_f32(v); return; }
    case V_U64: kv->kind = 0; kv->u = rd64(r); return;
    case V_I64: kv->kind = 1; kv->i = (int64_t)rd64(r); return;
    case V_F64: { uint64_t v = rd64(r); double d; memcpy(&d, &v, 8); kv->kind = 2; kv->f = d; return; }
    case V_STRING: kv->kind = 3; kv->s = rdstr(r); return;
    case V_ARRAY: {
      if (depth > 0) { r->bad = 1; return; }
      uint32_t et = rd32(r);
      uint64_t n = rd64(r);
      if (n > (1u << 22) || n > r->n - r->pos) { r->bad = 1; return; }
      kv->kind = 5;
      for (uint64_t i = 0; i < n && !r->bad; i++) {
        meta_kv tmp = {0};
        rdval(r, et, &tmp, depth + 1);
        free(tmp.s);
      }
      return;
    }
  }
  r->bad = 1;
}

typedef struct {
  int layers, embd, ff, heads, kv_heads, head_dim, vocab, ctx;
  float rope_base, eps;
  int arch_qwen2, rope_neox, bias, tied_output;
} cpuref_config;

struct cpuref_model {
  cpuref_config c;
  int exact_ggml, f16kv, nthreads, max_layers;
  int pos, max_ctx;
  uint8_t* file;
  size_t file_size;
  meta_kv* meta;
  size_t nmeta;
  tensor_t* tensors;
  size_t ntensors;
  float **k, **v;
  float* last_x;
  float* last_h;  /* the head's input of the last token (rmsNorm with output_norm) */
  float* last_u;  /* the up product of the last layer run, last token */
  float* last_a;  /* the attention output of the last layer run, last token */
};
typedef struct cpuref_model cpuref_model;

static meta_kv* find_meta(cpuref_model* m, const char* key) {
  for (size_t i = 0; i < m->nmeta; i++)
    if (strcmp(m->meta[i].key, key) == 0) return &m->meta[i];
  return NULL;
}
static tensor_t* find_tensor(cpuref_model* m, const char* name) {
  for (size_t i = 0; i < m->ntensors; i++)
    if (strcmp(m->tensors[i].name, name) == 0) return &m->tensors[i];
  return NULL;
}
/* File.Uint, gguf/gguf.go:410-420. */
static uint64_t meta_uint(cpuref_model* m, const char* key) {
  meta_kv* kv = find_meta(m, key);
  if (!kv) return 0;
  if (kv->kind == 0) return kv->u;
  if (kv->kind == 1 && kv->i >= 0) return (uint64_t)kv->i;
  return 0;
}

static void model_free(cpuref_model* m) {
  if (!m) return;
  for (size_t i = 0; i < m->nmeta; i++) {
    free(m->meta[i].key);
    free(m->meta[i].s);
  }
  for (size_t i = 0; i < m->ntensors; i++) free(m->tensors[i].name);
  if (m->k)
    for (int l = 0; l < m->c.layers; l++) {
      free(m->k[l]);
      free(m->v[l]);
    }
  free(m->k);
  free(m->v);
  free(m->meta);
  free(m->tensors);
  free(m->file);
  free(m->last_x);
  free(m->last_h);
  free(m->last_u);
  free(m->last_a);
  free(m);
}

EXPORT void cpuref_free(cpuref_model* m) { model_free(m); }

/* ConfigFrom, config.go:29-73. */
static int config_from(cpuref_model* m) {
  cpuref_config* c = &m->c;
  meta_kv* a = find_meta(m, "general.architecture");
  const char* arch = (a && a->kind == 3) ? a->s : "";
  if (strcmp(arch, "llama") != 0 && strcmp(arch, "qwen2") != 0)
    return fail("llm: architecture \"%s\" is not supported (llama and qwen2 only)", arch);
  char key[256];
#define U(k) (snprintf(key, sizeof key, "%s.%s", arch, k), (int)meta_uint(m, key))
  c->arch_qwen2 = strcmp(arch, "qwen2") == 0;
  c->rope_neox = c->arch_qwen2;
  c->layers = U("block_count");
  c->embd = U("embedding_length");
  c->ff = U("feed_forward_length");
  c->heads = U("attention.head_count");
  c->kv_heads = U("attention.head_count_kv");
  c->ctx = U("context_length");
  if (c->kv_heads == 0) c->kv_heads = c->heads;
  if (c->layers <= 0 || c->embd <= 0 || c->ff <= 0 || c->heads <= 0 || c->embd % c->heads != 0 ||
      c->heads % c->kv_heads != 0)
    return fail("llm: implausible %s hyperparameters", arch);
  c->head_dim = c->embd / c->heads;
  int rd = U("rope.dimension_count");
  if (rd != 0 && rd != c->head_dim) return fail("llm: rope.dimension_count differs from the head size (%s)", arch);
  snprintf(key, sizeof key, "%s.rope.scaling.type", arch);
  if (find_meta(m, key)) return fail("llm: rope scaling (%s) is not supported", key);
  snprintf(key, sizeof key, "%s.rope.scaling.factor", arch);
  if (find_meta(m, key)) return fail("llm: rope scaling (%s) is not supported", key);
  snprintf(key, sizeof key, "%s.rope.freq_base", arch);
  meta_kv* rb = find_meta(m, key);
  double rbv = (rb && rb->kind == 2) ? rb->f : 10000;
  snprintf(key, sizeof key, "%s.attention.layer_norm_rms_epsilon", arch);
  meta_kv* ep = find_meta(m, key);
  double epv = (ep && ep->kind == 2) ? ep->f : 0;
  c->rope_base = (float)rbv;
  c->eps = (float)epv;
#undef U
  tensor_t* t = find_tensor(m, "token_embd.weight");
  if (!t) return fail("llm: no token_embd.weight%s", "");
  c->vocab = (int)t->dims[1];
  c->tied_output = find_tensor(m, "output.weight") == NULL;
  c->bias = find_tensor(m, "blk.0.attn_q.bias") != NULL;
  if (c->bias != c->arch_qwen2) return fail("llm: %s with biases of the other architecture is not supported", arch);
  return 0;
}

/* LoadCPU, cpu.go:41-61: the header (gguf/gguf.go:292-407 layout) and every tensor. */
EXPORT int cpuref_load(const char* path, int max_ctx, cpuref_model** out) {
  *out = NULL;
  FILE* fp = fopen(path, "rb");
  if (!fp) return fail("llm: cannot open %s", path);
  fseek(fp, 0, SEEK_END);
  long sz = ftell(fp);
  fseek(fp, 0, SEEK_SET);
  cpuref_model* m = (cpuref_model*)calloc(1, sizeof *m);
  m->file = (uint8_t*)malloc((size_t)sz);
  m->file_size = (size_t)sz;
  if (fread(m->file, 1, (size_t)sz, fp) != (size_t)sz) {
    fclose(fp);
    model_free(m);
    return fail("llm: short read of %s", path);
  }
  fclose(fp);
  m->nthreads = 1;
  rd_t r = {m->file, m->file_size, 0, 0};
  char magic[4];
  rd(&r, magic, 4);
  uint32_t ver = rd32(&r);
  if (r.bad || memcmp(magic, "GGUF", 4) != 0 || ver != 3) {
    model_free(m);
    return fail("gguf: bad magic or version in %s", path);
  }
  uint64_t nt = rd64(&r), nkv = rd64(&r);
  if (nt > (1u << 16) || nkv > (1u << 16)) {
    model_free(m);
    return fail("gguf: too many entries in %s", path);
  }
  m->meta = (meta_kv*)calloc(nkv ? nkv : 1, sizeof(meta_kv));
  for (uint64_t i = 0; i < nkv && !r.bad; i++) {
    meta_kv* kv = &m->meta[m->nmeta++];
    kv->key = rdstr(&r);
    uint32_t t = rd32(&r);
    rdval(&r, t, kv, 0);
  }
  uint64_t align = 32;
  meta_kv* al = find_meta(m, "general.alignment");
  if (al && al->kind == 0 && al->u) align = al->u;
  m->tensors = (tensor_t*)calloc(nt ? nt : 1, sizeof(tensor_t));
  for (uint64_t i = 0; i < nt && !r.bad; i++) {
    tensor_t* t = &m->tensors[m->ntensors++];
    t->name = rdstr(&r);
    t->ndims = rd32(&r);
    if (t->ndims == 0 || t->ndims > 4) r.bad = 1;
    uint64_t elems = 1;
    for (uint32_t j = 0; j < t->ndims && !r.bad; j++) {
      t->dims[j] = rd64(&r);
      elems *= t->dims[j];
    }
    t->type = rd32(&r);
    t->offset = rd64(&r);
    uint64_t be, bb;
    if (!block_size(t->type, &be, &bb)) r.bad = 1;
    else t->size = elems / be * bb;
  }
  if (r.bad) {
    model_free(m);
    return fail("gguf: malformed header in %s", path);
  }
  uint64_t data_off = (r.pos + align - 1) / align * align;
  for (size_t i = 0; i < m->ntensors; i++) {
    tensor_t* t = &m->tensors[i];
    if (data_off + t->offset + t->size > m->file_size) {
      model_free(m);
      return fail("gguf: tensor %s lies past the end of the file", t->name);
    }
    t->data = m->file + data_off + t->offset;
  }
  if (config_from(m) != 0) {
    model_free(m);
    return -1;
  }
  m->max_ctx = max_ctx;
  size_t kv = (size_t)max_ctx * m->c.kv_heads * m->c.head_dim;
  m->k = (float**)calloc((size_t)m->c.layers, sizeof(float*));
  m->v = (float**)calloc((size_t)m->c.layers, sizeof(float*));
  for (int l = 0; l < m->c.layers; l++) {
    m->k[l] = (float*)calloc(kv ? kv : 1, 4);
    m->v[l] = (float*)calloc(kv ? kv : 1, 4);
  }
  m->last_x = (float*)calloc((size_t)m->c.embd, 4);
  m->last_h = (float*)calloc((size_t)m->c.embd, 4);
  m->last_u = (float*)calloc((size_t)m->c.ff, 4);
  m->last_a = (float*)calloc((size_t)m->c.heads * m->c.head_dim, 4);
  *out = m;
  return 0;
}

EXPORT void cpuref_get_config(cpuref_model* m, cpuref_config* out) { *out = m->c; }
EXPORT void cpuref_set_mode(cpuref_model* m, int exact_ggml, int f16kv) {
  m->exact_ggml = exact_ggml;
  m->f16kv = f16kv;
}
EXPORT void cpuref_set_threads(cpuref_model* m, int n) { m->nthreads = n < 1 ? 1 : n; }
EXPORT void cpuref_set_max_layers(cpuref_model* m, int n) { m->max_layers = n; }
EXPORT void cpuref_reset(cpuref_model* m) { m->pos = 0; } /* Reset, cpu.go:64 */
EXPORT int cpuref_pos(cpuref_model* m) { return m->pos; }  /* Pos, cpu.go:67 */
EXPORT void cpuref_last_x(cpuref_model* m, float* out) { memcpy(out, m->last_x, (size_t)m->c.embd * 4); }
/* Intermediate values of the last Forward (copies only; the trace surface the
 * reference's GPU Peek exposes, gpu.go:1015-1043): the head's normed row, the
 * last layer's up product, and a cached K or V row. */
EXPORT void cpuref_last_h(cpuref_model* m, float* out) { memcpy(out, m->last_h, (size_t)m->c.embd * 4); }
EXPORT void cpuref_last_up(cpuref_model* m, float* out) { memcpy(out, m->last_u, (size_t)m->c.ff * 4); }
/* the last layer's attention output (cpu.go:300-334), the reference's Peek("att") */
EXPORT void cpuref_last_att(cpuref_model* m, float* out) {
  memcpy(out, m->last_a, (size_t)m->c.heads * m->c.head_dim * 4);
}
EXPORT int cpuref_kv_row(cpuref_model* m, int layer, int pos, int v, float* out) {
  int kvd = m->c.kv_heads * m->c.head_dim;
  if (layer < 0 || layer >= m->c.layers || pos < 0 || pos >= m->pos) return fail("llm: no cache row%s", "");
  memcpy(out, (v ? m->v[layer] : m->k[layer]) + (size_t)pos * kvd, (size_t)kvd * 4);
  return 0;
}
EXPORT int cpuref_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Raw bytes of a tensor (tests compare uploads against them). */
EXPORT int cpuref_tensor(cpuref_model* m, const char* name, const uint8_t** data, uint64_t* size, uint32_t* type,
                         uint64_t* dims) {
  tensor_t* t = find_tensor(m, name);
  if (!t) return fail("llm: missing tensor %s", name);
  *data = t->data;
  *size = t->size;
  *type = t->type;
  for (int i = 0; i < 4; i++) dims[i] = i < (int)t->ndims ? t->dims[i] : 1;
  return 0;
}

static tensor_t* need(cpuref_model* m, const char* name, int* err) {
  tensor_t* t = find_tensor(m, name);
  if (!t) {
    fail("llm: missing tensor %s", name);
    *err = 1;
  }
  return t;
}

static int mv(cpuref_model* m, float* dst, const float* x, tensor_t* t, const q8act* qx) {
  return matvec(dst, x, t->type, t->data, (int)t->dims[0], (int)t->dims[1], qx, m->nthreads);
}

/* Forward, cpu.go:225-366: one token at the next position. Returns 1 with
 * the logits in `logits`, 0 when MaxLayers stops early (no logits), <0 on error. */
EXPORT int cpuref_forward(cpuref_model* m, int32_t tok, float* logits) {
  cpuref_config c = m->c;
  if (m->pos >= m->max_ctx) return fail("llm: context full%s", "");
  if (tok < 0 || tok >= c.vocab) return fail("llm: token out of range%s", "");
  int err = 0;
  float* x = (float*)calloc((size_t)c.embd, 4);
  tensor_t* emb = need(m, "token_embd.weight", &err);
  if (err) { free(x); return -1; }
  if (emb->type == T_Q8_0) {
    size_t rowBytes = (size_t)(c.embd / 32) * 34;
    const uint8_t* row = emb->data + (size_t)tok * rowBytes;
    for (int b = 0; b < c.embd / 32; b++) {
      float d = cpuref_f16_to_f32(u16le(row + b * 34));
      for (int j = 0; j < 32; j++) x[b * 32 + j] = d * (float)(int8_t)row[b * 34 + 2 + j];
    }
  } else if (emb->type == T_Q4_0) {
    size_t rowBytes = (size_t)(c.embd / 32) * 18;
    const uint8_t* row = emb->data + (size_t)tok * rowBytes;
    for (int b = 0; b < c.embd / 32; b++) {
      float d = cpuref_f16_to_f32(u16le(row + b * 18));
      for (int j = 0; j < 16; j++) {
        x[b * 32 + j] = d * (float)((int)(row[b * 18 + 2 + j] & 15) - 8);
        x[b * 32 + j + 16] = d * (float)((int)(row[b * 18 + 2 + j] >> 4) - 8);
      }
    }
  } else {
    free(x);
    snprintf(g_err, sizeof g_err, "llm: CPU embedding: ggml type %u", emb->type);
    return -1;
  }
  int kvd = c.kv_heads * c.head_dim;
  float* h = (float*)calloc((size_t)c.embd, 4);
  float* q = (float*)calloc((size_t)c.heads * c.head_dim, 4);
  float* kk = (float*)calloc((size_t)kvd, 4);
  float* vv = (float*)calloc((size_t)kvd, 4);
  float* att = (float*)calloc((size_t)c.heads * c.head_dim, 4);
  float* o = (float*)calloc((size_t)c.embd, 4);
  float* g = (float*)calloc((size_t)c.ff, 4);
  float* u = (float*)calloc((size_t)c.ff, 4);
  float* dn = (float*)calloc((size_t)c.embd, 4);
  /* one score row per head, so heads may run on separate threads; each keeps
   * cpu.go's order, so threaded runs are bit-identical */
  float* scores = (float*)calloc((size_t)(m->pos + 1) * c.heads, 4);
  int nmax = c.embd > c.ff ? c.embd : c.ff;
  if (c.heads * c.head_dim > nmax) nmax = c.heads * c.head_dim;
  q8act qa = {(float*)calloc((size_t)nmax / 32 + 1, 4), (float*)calloc((size_t)nmax / 32 + 1, 4),
              (int8_t*)calloc((size_t)nmax, 1)};
#define PREP(v, n) (m->exact_ggml ? (quantize_q8((v), (n), &qa), &qa) : (const q8act*)NULL)
  int nl = c.layers;
  if (m->max_layers != 0) {
    int ml = m->max_layers > 0 ? m->max_layers : 0;
    nl = nl < ml ? nl : ml;
  }
  char p[96];
  int rc = 0;
  for (int l = 0; l < nl && !err; l++) {
#define T(suffix) (snprintf(p, sizeof p, "blk.%d." suffix, l), need(m, p, &err))
    tensor_t* an = T("attn_norm.weight");
    if (err) break;
    cpuref_rmsnorm(h, x, (const float*)an->data, c.embd, c.eps);
    const q8act* qh = PREP(h, c.embd);
    tensor_t *wq = T("attn_q.weight"), *wk = T("attn_k.weight"), *wv = T("attn_v.weight");
    if (err) break;
    if (mv(m, q, h, wq, qh) || mv(m, kk, h, wk, qh) || mv(m, vv, h, wv, qh)) { err = 1; break; }
    if (c.bias) {
      tensor_t *bq = T("attn_q.bias"), *bk = T("attn_k.bias"), *bv = T("attn_v.bias");
      if (err) break;
      const float* b = (const float*)bq->data;
      for (uint64_t i = 0; i < bq->dims[0]; i++) q[i] += b[i];
      b = (const float*)bk->data;
      for (uint64_t i = 0; i < bk->dims[0]; i++) kk[i] += b[i];
      b = (const float*)bv->data;
      for (uint64_t i = 0; i < bv->dims[0]; i++) vv[i] += b[i];
    }
    cpuref_rope(q, m->pos, c.heads, c.head_dim, c.rope_base, c.rope_neox);
    cpuref_rope(kk, m->pos, c.kv_heads, c.head_dim, c.rope_base, c.rope_neox);
    for (int i = 0; i < kvd; i++) {
      if (m->exact_ggml || m->f16kv) {
        m->k[l][(size_t)m->pos * kvd + i] = cpuref_round_f16(kk[i]);
        m->v[l][(size_t)m->pos * kvd + i] = cpuref_round_f16(vv[i]);
      } else {
        m->k[l][(size_t)m->pos * kvd + i] = kk[i];
        m->v[l][(size_t)m->pos * kvd + i] = vv[i];
      }
    }
    float scale = (float)(1 / sqrt((double)c.head_dim));
    int grp = c.heads / c.kv_heads;
    const float* kl = m->k[l];
    const float* vl = m->v[l];
    int pos = m->pos;
#pragma omp parallel for num_threads(m->nthreads) if (m->nthreads > 1 && pos >= 64) schedule(static)
    for (int hd = 0; hd < c.heads; hd++) {
      int kvh = hd / grp;
      float* sc = scores + (size_t)hd * (pos + 1);
      const float* qv = q + hd * c.head_dim;
      float mx = -INFINITY;
      for (int t = 0; t <= pos; t++) {
        const float* kr = kl + (size_t)t * kvd + kvh * c.head_dim;
        float s = 0;
        for (int i = 0; i < c.head_dim; i++) s += qv[i] * kr[i];
        sc[t] = s * scale;
        mx = go_maxf(mx, sc[t]);
      }
      float sum = 0;
      for (int t = 0; t <= pos; t++) {
        sc[t] = (float)exp((double)(sc[t] - mx));
        sum += sc[t];
      }
      float* outv = att + hd * c.head_dim;
      for (int i = 0; i < c.head_dim; i++) outv[i] = 0;
      for (int t = 0; t <= pos; t++) {
        const float* vr = vl + (size_t)t * kvd + kvh * c.head_dim;
        float w = sc[t] / sum;
        for (int i = 0; i < c.head_dim; i++) outv[i] += w * vr[i];
      }
    }
    tensor_t* wo = T("attn_output.weight");
    if (err) break;
    if (mv(m, o, att, wo, PREP(att, c.heads * c.head_dim))) { err = 1; break; }
    for (int i = 0; i < c.embd; i++) x[i] += o[i];
    tensor_t* fn = T("ffn_norm.weight");
    if (err) break;
    cpuref_rmsnorm(h, x, (const float*)fn->data, c.embd, c.eps);
    qh = PREP(h, c.embd);
    tensor_t *wg = T("ffn_gate.weight"), *wu = T("ffn_up.weight"), *wd = T("ffn_down.weight");
    if (err) break;
    if (mv(m, g, h, wg, qh) || mv(m, u, h, wu, qh)) { err = 1; break; }
    for (int i = 0; i < c.ff; i++) g[i] = g[i] / (1 + (float)exp((double)(-g[i]))) * u[i];
    if (mv(m, dn, g, wd, PREP(g, c.ff))) { err = 1; break; }
    for (int i = 0; i < c.embd; i++) x[i] += dn[i];
#undef T
  }
  if (err) {
    rc = -1;
  } else {
    memcpy(m->last_x, x, (size_t)c.embd * 4);
    if (nl > 0) memcpy(m->last_u, u, (size_t)c.ff * 4);
    if (nl > 0) memcpy(m->last_a, att, (size_t)c.heads * c.head_dim * 4);
    if (m->max_layers != 0 && m->max_layers < c.layers) {
      m->pos++;
      rc = 0;
    } else {
      tensor_t* on = need(m, "output_norm.weight", &err);
      tensor_t* out = c.tied_output ? emb : need(m, "output.weight", &err);
      if (err) {
        rc = -1;
      } else {
        cpuref_rmsnorm(h, x, (const float*)on->data, c.embd, c.eps);
        memcpy(m->last_h, h, (size_t)c.embd * 4);
        if (mv(m, logits, h, out, PREP(h, c.embd))) rc = -1;
        else {
          m->pos++;
          rc = 1;
        }
      }
    }
  }
#undef PREP
  free(x); free(h); free(q); free(kk); free(vv); free(att); free(o); free(g); free(u); free(dn); free(scores);
  free(qa.d); free(qa.s); free(qa.qs);
  return rc;
}
