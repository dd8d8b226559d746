// The non-matrix kernels of the forward pass: attention over the f32 KV cache
// in chunks of positions (flash-decoding partials, merged by the O-projection
// prologue), greedy sampling and the state advance.
#include "layer.h"
#include "wave.h"

namespace llmhip {

// One workgroup per (chunk of CH positions, KV head, token): the GQ query heads
// that share the KV head read its keys and values once (the reference's K2
// reads them once per query head, kernels_fused.go:82-146).  Writes the
// chunk's softmax statistics (max m, sum l of exp(s - m)) and sum_p e_p v_p.
// A chunk wholly past the causal bound writes nothing: the merge never reads it.
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const uint32_t c = blockIdx.x, g = blockIdx.y, t = blockIdx.z;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t HD = a.hd, GQ = a.heads / a.kv_heads, CH = a.chunk;
  const uint32_t pos = a.state[0] + t, n = pos + 1;
  const uint32_t p0 = c * CH;
  if (p0 >= n) return;
  const uint32_t L = min(CH, n - p0);
  const uint32_t KS = HD + 1;  // padded row: lanes reading different rows hit different banks
  float* qs = sm;               // [GQ][HD]
  float* ks = qs + GQ * HD;     // [CH][HD+1]
  float* vs = ks + CH * KS;     // [CH][HD]
  float* sc = vs + CH * HD;     // [GQ][CH]
  const float* qg = a.q + (uint64_t)t * a.heads * HD + (uint64_t)g * GQ * HD;
  const float* kb = a.kv + (uint64_t)p0 * a.kvd + g * HD;
  const float* vb = a.kv + (uint64_t)a.ctx * a.kvd + (uint64_t)p0 * a.kvd + g * HD;
  // every load of the workgroup in flight at once: q rows, then K and V rows as float4
  typedef float f4 __attribute__((ext_vector_type(4)));
  const uint32_t HD4 = HD / 4, NQ4 = GQ * HD4, NK4 = L * HD4;
  constexpr int U = 8;  // float4 of K (and of V) per thread: CH*HD/4 <= 8*256
  f4 qr[2], kr[U], vr[U];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    uint32_t i = tid + u * blockDim.x;
    if (i < NQ4) qr[u] = ((const f4*)qg)[i];
  }
#pragma unroll
  for (int u = 0; u < U; u++) {
    uint32_t i = tid + u * blockDim.x;
    if (i < NK4) {
      uint32_t p = i / HD4, d = i % HD4;
      kr[u] = *(const f4*)(kb + (uint64_t)p * a.kvd + 4 * d);
      vr[u] = *(const f4*)(vb + (uint64_t)p * a.kvd + 4 * d);
    }
  }
#pragma unroll
  for (int u = 0; u < 2; u++) {
    uint32_t i = tid + u * blockDim.x;
    if (i < NQ4) ((f4*)qs)[i] = qr[u];
  }
#pragma unroll
  for (int u = 0; u < U; u++) {
    uint32_t i = tid + u * blockDim.x;
    if (i < NK4) {
      uint32_t p = i / HD4, d = i % HD4;
      for (int j = 0; j < 4; j++) ks[p * KS + 4 * d + j] = kr[u][j];
      ((f4*)vs)[p * HD4 + d] = vr[u];
    }
  }
  __syncthreads();
  // scores: s = (q . k) * scale, the dot product in index order (cpu.go:312-316)
  for (uint32_t i = tid; i < GQ * L; i += blockDim.x) {
    uint32_t h = i / L, p = i % L;
    const float* qq = qs + h * HD;
    const float* kk = ks + p * KS;
    float s = 0;
    for (uint32_t d = 0; d < HD; d++) s += qq[d] * kk[d];
    sc[h * CH + p] = s * a.scale;
  }
  __syncthreads();
  // per head: m = max, e = exp(s - m), l = sum e (one wave per head)
  for (uint32_t h = wave; h < GQ; h += 4) {
    float m = -INFINITY;
    for (uint32_t p = lane; p < L; p += 64) m = fmaxf(m, sc[h * CH + p]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float l = 0;
    for (uint32_t p = lane; p < L; p += 64) {
      float e = expf(sc[h * CH + p] - m);
      sc[h * CH + p] = e;
      l += e;
    }
    for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
    if (lane == 0) {
      float* mlp = a.ml + (((uint64_t)t * a.heads + g * GQ + h) * a.smax + c) * 2;
      mlp[0] = m;
      mlp[1] = l;
    }
  }
  __syncthreads();
  // o = sum_p e_p v_p
  for (uint32_t i = tid; i < GQ * HD; i += blockDim.x) {
    uint32_t h = i / HD, d = i % HD;
    const float* e = sc + h * CH;
    float o = 0;
    for (uint32_t p = 0; p < L; p++) o += e[p] * vs[p * HD + d];
    a.pv[(((uint64_t)t * a.heads + g * GQ + h) * a.smax + c) * HD + d] = o;
  }
}

// Short-context attention (every position of the pass below ATTN_FULL_MAX =
// 256), one 512-thread workgroup per (query head, token) and no split, so the
// softmax uses the exact maximum over all positions (cpu.go:306-334) and the
// head's output goes straight to att[t][h*64 + d] for a plain O-projection
// prologue.  Lane (r, c) of a wave's four 16-lane rows holds float4 c of key
// and value rows slot + 32j (slot = 4*wave + r, j < 8): loads are coalesced
// 256-byte rows, q is one float4 per lane, a score is a 16-lane DPP sum that
// lands in the lanes holding the matching value row, and the weighted value
// sums are reduced over rows by two shuffles and over waves through LDS.  All
// global loads are issued before anything waits; a.rows (host-chosen, >= every
// position count of the pass) bounds the rows read, the rest are masked.
// Workgroups go to the 8 XCDs round-robin (block b on XCD b % 8), so the query
// heads of one (token, KV head) instance get blocks on one XCD and read its
// rows through one L2, and the instances spread over the XCDs: block b serves
// instance 8*(s / GQ) + b % 8 (= t * kv_heads + g), query head s % GQ of it,
// with s = b / 8; blocks past the last instance exit at once.
__global__ __launch_bounds__(512) void attn_full_kernel(AttnArgs a, uint32_t ntok) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  constexpr uint32_t HD = 64, J = ATTN_FULL_MAX / 32;
  __shared__ float red_m[8], red_l[8];
  __shared__ __attribute__((aligned(16))) float red_o[8 * HD];
  const uint32_t GQ = a.heads / a.kv_heads, sb = blockIdx.x / 8;
  const uint32_t inst = 8 * (sb / GQ) + blockIdx.x % 8;
  if (inst >= ntok * a.kv_heads) return;
  const uint32_t t = inst / a.kv_heads, g = inst % a.kv_heads;
  const uint32_t h = g * GQ + sb % GQ, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t c = lane & 15, slot = tid >> 4;
  const float* kb = a.kv + g * HD + 4 * c;
  const float* vb = a.kv + (uint64_t)a.ctx * a.kvd + g * HD + 4 * c;
  const f4 q = *(const f4*)(a.q + (uint64_t)t * a.heads * HD + h * HD + 4 * c);
  f4 kr[J], vr[J];
#pragma unroll
  for (uint32_t j = 0; j < J; j++) {
    const uint32_t p = slot + 32 * j;
    if (p < a.rows) {
      kr[j] = *(const f4*)(kb + (uint64_t)p * a.kvd);
      vr[j] = *(const f4*)(vb + (uint64_t)p * a.kvd);
    }
  }
  const uint32_t n = a.state[0] + t + 1;
  // scores s = (q . k) * scale (cpu.go:312-316), masked past the causal bound
  float sj[J], m = -INFINITY;
#pragma unroll
  for (uint32_t j = 0; j < J; j++) {
    const uint32_t p = slot + 32 * j;
    float d = 0;
    if (p < a.rows) d = q[0] * kr[j][0] + q[1] * kr[j][1] + q[2] * kr[j][2] + q[3] * kr[j][3];
    d = row_sum16(d);
    sj[j] = p < n ? d * a.scale : -INFINITY;
    m = fmaxf(m, sj[j]);
  }
  m = rows_max4(m);
  if (lane == 0) red_m[wave] = m;
  __syncthreads();
  float M = red_m[0];
#pragma unroll
  for (uint32_t w = 1; w < 8; w++) M = fmaxf(M, red_m[w]);
  // e = exp(s - max); l = sum e; o = sum e v
  f4 acc = f4{0, 0, 0, 0};
  float l = 0;
#pragma unroll
  for (uint32_t j = 0; j < J; j++) {
    const uint32_t p = slot + 32 * j;
    if (p < n) {
      const float e = expf(sj[j] - M);
      l += e;
      acc += e * vr[j];
    }
  }
  l = rows_sum4(l);
#pragma unroll
  for (int k = 0; k < 4; k++) {
    acc[k] += __shfl_xor(acc[k], 16);
    acc[k] += __shfl_xor(acc[k], 32);
  }
  if (lane < 16) ((f4*)red_o)[wave * 16 + c] = acc;
  if (lane == 0) red_l[wave] = l;
  __syncthreads();
  if (tid < HD) {
    float L = 0, o = 0;
#pragma unroll
    for (uint32_t w = 0; w < 8; w++) {
      L += red_l[w];
      o += red_o[w * HD + tid];
    }
    a.att[(uint64_t)t * a.heads * HD + h * HD + tid] = o / L;
  }
}

bool attn_full_ok(uint32_t heads, uint32_t kv_heads, uint32_t hd) {
  (void)heads;
  (void)kv_heads;
  return hd == 64;
}

// Rows the short-context kernel reads for a pass whose last position is
// last_pos: the next multiple of 64 (one of four graph variants).
uint32_t attn_full_rows(uint32_t last_pos) { return (last_pos / 64 + 1) * 64; }

int attn_full_launch(const AttnArgs& a, uint32_t ntok, hipStream_t s) {
  if (ntok == 0) return 0;
  if (!attn_full_ok(a.heads, a.kv_heads, a.hd) || !a.att || a.rows > ATTN_FULL_MAX || a.rows > a.ctx)
    return set_error(LLMHIP_ERR_ARG, "llm: attention: head size %u or %u rows not supported by the short-context kernel",
                     a.hd, a.rows);
  const uint32_t gq = a.heads / a.kv_heads, blocks = 8 * gq * ((ntok * a.kv_heads + 7) / 8);
  hipLaunchKernelGGL(attn_full_kernel, dim3(blocks), dim3(512), 0, s, a, ntok);
  LLM_HIP(hipGetLastError());
  return 0;
}

uint32_t attn_lds_bytes(uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t chunk) {
  uint32_t gq = heads / kv_heads;
  return 4 * (gq * hd + chunk * (hd + 1) + chunk * hd + gq * chunk);
}

int attn_launch(const AttnArgs& a, uint32_t ntok, hipStream_t s) {
  if (ntok == 0) return 0;
  const uint32_t gq = a.heads / a.kv_heads;
  if (a.hd % 4 || gq * a.hd / 4 > 2 * 256 || a.chunk * a.hd / 4 > 8 * 256)
    return set_error(LLMHIP_ERR_ARG, "llm: attention: %u heads per KV head of %u, chunk %u not supported", gq, a.hd,
                     a.chunk);
  uint32_t lds = attn_lds_bytes(a.heads, a.kv_heads, a.hd, a.chunk);
  hipLaunchKernelGGL(attn_kernel, dim3(a.smax, a.kv_heads, ntok), dim3(256), lds, s, a);
  LLM_HIP(hipGetLastError());
  return 0;
}

// Greedy sampling (cpu.go:389-397): the lowest index of the largest logit,
// NaN never wins, and a NaN logit 0 is never displaced.  Combines the
// per-workgroup partials of the head's matvec (all loads in flight at once),
// writes the token to tokens[step + adv] and out[0] (kernels.go:389-392),
// then advances (pos, step) by adv (kernels.go:397-415).
__device__ __forceinline__ bool amax_better(float v, uint32_t i, float bv, uint32_t bi) {
  return i != 0xffffffffu && (bi == 0xffffffffu || v > bv || (v == bv && i < bi));
}

__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ pv, const uint32_t* __restrict__ pi,
                                                      uint32_t n, const float* __restrict__ logits,
                                                      int32_t* __restrict__ tokens, int32_t* __restrict__ outb,
                                                      uint32_t* __restrict__ state, uint32_t adv) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  constexpr int U = 8;
  float v[U];
  uint32_t ix[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    uint32_t i = tid + u * blockDim.x;
    v[u] = -INFINITY;
    ix[u] = 0xffffffffu;
    if (i < n) {
      v[u] = pv[i];
      ix[u] = pi[i];
    }
  }
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
#pragma unroll
  for (int u = 0; u < U; u++)
    if (amax_better(v[u], ix[u], bv, bi)) {
      bv = v[u];
      bi = ix[u];
    }
  for (uint32_t i = tid + U * blockDim.x; i < n; i += blockDim.x)
    if (amax_better(pv[i], pi[i], bv, bi)) {
      bv = pv[i];
      bi = pi[i];
    }
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(bv, o);
    uint32_t oi = __shfl_xor(bi, o);
    if (amax_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (uint32_t w = 1; w < nw; w++)
      if (amax_better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    float l0 = logits[0];
    if (bi == 0xffffffffu || l0 != l0) bi = 0;
    uint32_t step = state[1];
    tokens[step + adv] = (int32_t)bi;
    outb[0] = (int32_t)bi;
    state[0] += adv;
    state[1] = step + adv;
  }
}

int argmax_launch(const float* pv, const uint32_t* pi, uint32_t n, const float* logits, int32_t* tokens,
                  int32_t* outb, uint32_t* state, uint32_t adv, hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, pv, pi, n, logits, tokens, outb, state, adv);
  LLM_HIP(hipGetLastError());
  return 0;
}

// state += n (kernels.go:407-415)
__global__ void advance_kernel(uint32_t* state, uint32_t n) {
  if (threadIdx.x == 0) {
    state[0] += n;
    state[1] += n;
  }
}

int advance_launch(uint32_t* state, uint32_t n, hipStream_t s) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, s, state, n);
  LLM_HIP(hipGetLastError());
  return 0;
}

}  // namespace llmhip
