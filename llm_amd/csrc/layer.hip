// The non-matrix kernels of the forward pass: attention over the f32 KV cache
// (one chunk, or chunks of positions merged by a second kernel), greedy
// sampling and the state advance.
#include "attn_core.h"
#include "gemv_impl.h"
#include "layer.h"
#include "wave.h"

namespace llmhip {

// The block-scaled operand form of att (AttnOps): v = att[t][col],
// col = h * HD + d, held by lane d % 64 of whole waves.  Per 32-element block
// (half a wave): the exponent e that puts the block's max magnitude in
// [2^14, 2^15) (0 for an all-zero or non-finite block), hi = f16(v 2^e),
// lo = f16(v 2^e - hi); item i of the block (elements 4i..4i+3 and
// 16+4i..16+4i+3) is written by the block's lane 4i as the product's 16-byte
// operands (hi, then lo 64 operands on) for token t % 16 of group t / 16, in
// the order {A0, A2, C0, C2, A1, A3, C1, C3} of prep_kernel.
__device__ __forceinline__ void emit_operand(const AttnOps& a, uint32_t t, uint32_t col, float v) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const uint32_t lane = threadIdx.x & 63, j = lane & 31, b = col / 32;
  float mx = fabsf(v), sum = v;
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o));
    sum += __shfl_xor(sum, o);
  }
  int e = 0;
  if (mx > 0 && mx <= 3.0e38f) {
    int E;
    frexpf(mx, &E);
    e = 15 - E;
  }
  const float sv = ldexpf(v, e);
  const uint32_t base = lane - j;  // the block's first lane
  float g[8];
  const uint32_t src[8] = {0, 2, 16, 18, 1, 3, 17, 19};
#pragma unroll
  for (int i = 0; i < 8; i++) g[i] = __shfl(sv, (int)(base + (j & ~3u) + src[i]));
  if ((j & 3) == 0 && j < 16) {
    h8 hi, lo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const _Float16 hh = (_Float16)g[i];
      hi[i] = hh;
      lo[i] = (_Float16)(g[i] - (float)hh);
    }
    h8* dst = (h8*)a.xp + ((uint64_t)(t / 16) * a.onb + b) * 128 + (j / 4) * 16 + t % 16;
    dst[0] = hi;
    dst[64] = lo;
  }
  if (j == 0) {
    a.xdx[(uint64_t)t * a.onb + b] = ldexpf(1.f, -e);
    a.xbsum[(uint64_t)t * a.onb + b] = sum;
    if (col == 0) a.xexp[t] = 0;
  }
}

// Attention over the KV cache (cpu.go:300-334), one query head per
// workgroup of 512 threads over C = 32*J cache rows (attn_core.h).  Every
// global load is issued before anything waits; a.rows (host-chosen, >= every
// position count of the pass, <= ctx) bounds the rows read.
//
// Work units are (token t, KV head g, chunk c) = (u % NI / kv, u % NI % kv,
// u / NI), NI = ntok * kv_heads.  Workgroups go to the 8 XCDs round-robin
// (block b on XCD b % 8): block b serves unit 8*(s / GQ) + b % 8, query head
// s % GQ of it (s = b / 8), so the GQ query heads of a unit read its rows
// through one L2 and the units spread over the XCDs; blocks past the last
// unit exit at once.
//   SPLIT = false: one chunk (all positions < C); writes att[t][h*HD + d].
//   SPLIT = true: chunk c covers rows [c*C, c*C + C); writes the partials
//     (m, l) and o = sum e v for attn_merge_kernel; chunks past the causal
//     bound write nothing.
template <uint32_t HD, uint32_t J, bool SPLIT, bool KVH, bool EMIT = false>
__global__ __launch_bounds__(512) void attn_kernel(AttnArgs a_in, uint32_t ntok, uint32_t units, AttnOps ops) {
  // both lines of the arguments it reads in one round of scalar loads (as gemv_kernel's touch_args)
  static_assert(offsetof(AttnArgs, heads) < 64 && offsetof(AttnArgs, rows) / 64 == 1 &&
                    offsetof(AttnArgs, dkv) / 64 == 1,
                "argument lines");
  AttnArgs a = a_in;
  asm volatile("" : "+s"(a.heads), "+s"(a.rows));
  typedef AttnChunk<HD, J, 8, KVH> AC;
  __shared__ AttnLds<HD, 8> sm;
  const uint32_t GQ = a.dgq.d, sb = blockIdx.x / 8, sq = fdiv(sb, a.dgq);
  const uint32_t u = 8 * sq + blockIdx.x % 8;
  if (u >= units) return;
  const uint32_t NI = a.dni.d, c = fdiv(u, a.dni), inst = u - c * NI;
  const uint32_t t = fdiv(inst, a.dkv), g = inst - t * a.kv_heads, h = g * GQ + (sb - sq * GQ);
  const uint32_t tid = threadIdx.x, cl = tid & 15;
  const uint32_t row0 = c * AC::C;
  const float* qp = a.q + (uint64_t)t * a.heads * HD + h * HD + 4 * cl;
  f4 q[AC::V4];
#pragma unroll
  for (uint32_t v = 0; v < AC::V4; v++) q[v] = *(const f4*)(qp + 64 * v);
  AC rows;
  rows.load(a.kv, a.kvd, a.ctx, g, row0, a.rows);
  const uint32_t n = state_pos(a.state) + t + 1;
  if (SPLIT && row0 >= n) return;  // uniform over the workgroup
  float M, L, o;
  rows.reduce(q, row0, n, a.scale, sm, &M, &L, &o);
  if (tid < HD) {
    if (SPLIT) {
      const uint64_t th = (uint64_t)t * a.heads + h;
      a.pv[(th * a.smax + c) * HD + tid] = o;
      if (tid == 0) {
        a.ml[(th * a.smax + c) * 2] = M;
        a.ml[(th * a.smax + c) * 2 + 1] = L;
      }
    } else {
      a.att[(uint64_t)t * a.heads * HD + h * HD + tid] = o / L;
    }
  }
  if (EMIT && tid < HD) emit_operand(ops, t, h * HD + tid, o / L);
}

// The one-chunk attention for QN tokens of a pass at once: a workgroup per
// (token group of QN, KV head) and query head, as attn_kernel maps units to
// XCDs, loads the rows once for its QN queries (AttnChunk::reduce_n), each
// with its own causal bound; outputs (and, EMIT, the O product's operands)
// as attn_kernel<SPLIT = false> writes them.
template <uint32_t HD, uint32_t J, bool KVH, bool EMIT, uint32_t QN>
__global__ __launch_bounds__(512) void attn_multi_kernel(AttnArgs a_in, uint32_t ntok, uint32_t units, AttnOps ops) {
  typedef AttnChunk<HD, J, 8, KVH> AC;
  __shared__ AttnLds<HD, 8, QN> sm;
  // both argument lines in one round (as gemv_kernel's touch_args); divisions by multiplies (FastDiv)
  AttnArgs a = a_in;
  asm volatile("" : "+s"(a.heads), "+s"(a.rows));
  const uint32_t GQ = a.dgq.d, sb = blockIdx.x / 8, sq = fdiv(sb, a.dgq);
  const uint32_t u = 8 * sq + blockIdx.x % 8;
  if (u >= units) return;
  const uint32_t tp = fdiv(u, a.dkv), g = u - tp * a.kv_heads, h = g * GQ + (sb - sq * GQ);
  const uint32_t tid = threadIdx.x, cl = tid & 15;
  f4 q[QN][AC::V4];
  uint32_t n[QN];
#pragma unroll
  for (uint32_t i = 0; i < QN; i++) {
    const uint32_t t = min(tp * QN + i, ntok - 1);
    const float* qp = a.q + (uint64_t)t * a.heads * HD + h * HD + 4 * cl;
#pragma unroll
    for (uint32_t v = 0; v < AC::V4; v++) q[i][v] = *(const f4*)(qp + 64 * v);
    n[i] = state_pos(a.state) + t + 1;
  }
  AC rows;
  rows.load(a.kv, a.kvd, a.ctx, g, 0, a.rows);
  float M[QN], L[QN], o[QN];
  rows.template reduce_n<QN>(q, 0, n, a.scale, sm, M, L, o);
#pragma unroll
  for (uint32_t i = 0; i < QN; i++) {
    const uint32_t t = tp * QN + i;
    if (t >= ntok) break;  // uniform
    if (tid < HD) a.att[(uint64_t)t * a.heads * HD + h * HD + tid] = o[i] / L[i];
    if (EMIT && tid < HD) emit_operand(ops, t, h * HD + tid, o[i] / L[i]);
  }
}

// Prefill attention over chunks of 128 cache rows on the matrix cores (head
// size 64, several tokens): a workgroup per (KV head g, chunk c, group of 64
// queries), the queries of KV head g numbered token * GQ + (head - g * GQ).
// The chunk's key and value rows are staged in LDS once; each of the four
// waves owns 16 queries and forms, with v_mfma_f32_16x16x4_f32,
//   S = Q K^T (16 queries x 128 rows, 16 steps of 4 dimensions),
// then per query the chunk max M over its causal rows, e = exp(s*scale - M),
// L = sum e, and O = e V (P goes through LDS into the A layout).  (M, L, O)
// are the chunk partials attn_merge_kernel combines, as attn_kernel<SPLIT>
// writes them; chunks at or past a query's causal bound write nothing.
// Operand layouts of the 16x16x4 f32 MFMA: lane l holds A[l % 16][l / 16],
// B[l / 16][l % 16] and D[4 (l / 16) + i][l % 16], i < 4.
constexpr uint32_t AMMA_KS = 65, AMMA_VS = 80, AMMA_PS = 132;  // LDS row strides (bank-conflict free)

template <bool KVH>
__global__ __launch_bounds__(256) void attn_mma_kernel(AttnArgs a_in, uint32_t ntok, FastDiv dch) {
  constexpr uint32_t HD = 64, C = ATTN_SPLIT_ROWS;
  __shared__ float Ks[C * AMMA_KS], Vs[C * AMMA_VS], Ps[4][16 * AMMA_PS];
  // both argument lines in one round (as gemv_kernel's touch_args); divisions by multiplies (FastDiv)
  AttnArgs a = a_in;
  asm volatile("" : "+s"(a.heads), "+s"(a.rows));
  const uint32_t GQ = a.dgq.d, nq = ntok * GQ;
  const uint32_t rest = fdiv(blockIdx.x, dch), c = blockIdx.x - rest * dch.d;
  const uint32_t qg = fdiv(rest, a.dkv), g = rest - qg * a.kv_heads, q0 = qg * 64;
  const uint32_t row0 = c * C, pos0 = state_pos(a.state);
  const uint32_t tlast = fdiv(min(q0 + 64, nq) - 1, a.dgq);
  if (q0 >= nq || row0 >= pos0 + tlast + 1) return;  // uniform: no query of the group reaches the chunk
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, grp = lane >> 4, r = lane & 15;

  // stage the chunk's rows below lim (zeros past it: masked, and 0 * V stays 0)
  // (every load first, rows clamped below lim, so that one wait covers them)
  const uint32_t lim = min(a.rows, pos0 + tlast + 1);  // > row0
  constexpr uint32_t NL = C * HD / 4 / 256;
  f4 kk[NL], vv[NL];
#pragma unroll
  for (uint32_t k = 0; k < NL; k++) {
    const uint32_t idx = tid + 256 * k, p = min(row0 + idx / 16, lim - 1), c4 = idx % 16;
    kk[k] = kv_load4<KVH>(a.kv, (uint64_t)p * a.kvd + g * HD + 4 * c4);
    vv[k] = kv_load4<KVH>(a.kv, (uint64_t)a.ctx * a.kvd + (uint64_t)p * a.kvd + g * HD + 4 * c4);
  }
#pragma unroll
  for (uint32_t k = 0; k < NL; k++) {
    const uint32_t idx = tid + 256 * k, row = idx / 16, c4 = idx % 16;
    const bool in = row0 + row < lim;
    const f4 z = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; i++) Ks[row * AMMA_KS + 4 * c4 + i] = in ? kk[k][i] : 0.f;
    *(f4*)&Vs[row * AMMA_VS + 4 * c4] = in ? vv[k] : z;
  }

  // this lane's A rows: query m = r of the wave, dimensions 16 grp .. 16 grp + 15
  const uint32_t qa = min(q0 + 16 * wave + r, nq - 1), ta = fdiv(qa, a.dgq), ha = g * GQ + (qa - ta * GQ);
  f4 aq[4];
  const float* qp = a.q + (uint64_t)ta * a.heads * HD + ha * HD + 16 * grp;
#pragma unroll
  for (int v = 0; v < 4; v++) aq[v] = *(const f4*)(qp + 4 * v);
  // the causal bound of this lane's D rows: queries 4 grp + i of the wave
  uint32_t nd[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t qd = q0 + 16 * wave + 4 * grp + i;
    nd[i] = qd < nq ? pos0 + fdiv(qd, a.dgq) + 1 : 0;
  }
  __syncthreads();

  f4 S[C / 16];
#pragma unroll
  for (uint32_t nt = 0; nt < C / 16; nt++) S[nt] = f4{0, 0, 0, 0};
  // batches of 4 dimension steps: the batch's key operands are read from LDS
  // before its MFMAs (scheduling barriers keep the compiler from interleaving
  // each read with its use)
#pragma unroll
  for (uint32_t jb = 0; jb < 16; jb += 4) {
    float kb[4][C / 16];
#pragma unroll
    for (uint32_t jj = 0; jj < 4; jj++)
#pragma unroll
      for (uint32_t nt = 0; nt < C / 16; nt++) kb[jj][nt] = Ks[(16 * nt + r) * AMMA_KS + 16 * grp + jb + jj];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t jj = 0; jj < 4; jj++)
#pragma unroll
      for (uint32_t nt = 0; nt < C / 16; nt++)
        S[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[jb / 4][jj], kb[jj][nt], S[nt], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  float M[4], L[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float m = -INFINITY;
#pragma unroll
    for (uint32_t nt = 0; nt < C / 16; nt++) {
      const bool ok = row0 + 16 * nt + r < nd[i];
      S[nt][i] = ok ? S[nt][i] * a.scale : -INFINITY;
      m = fmaxf(m, S[nt][i]);
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    M[i] = m;
    float l = 0;
#pragma unroll
    for (uint32_t nt = 0; nt < C / 16; nt++) {
      const bool ok = row0 + 16 * nt + r < nd[i];
      const float e = ok ? __expf(S[nt][i] - m) : 0.f;
      l += e;
      Ps[wave][(4 * grp + i) * AMMA_PS + 16 * nt + r] = e;
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) l += __shfl_xor(l, o);
    L[i] = l;
  }
  __syncthreads();

  f4 O[HD / 16];
#pragma unroll
  for (uint32_t dt = 0; dt < HD / 16; dt++) O[dt] = f4{0, 0, 0, 0};
  // batches of 8 row steps: the batch's operands are read from LDS before its MFMAs
  for (uint32_t jb = 0; jb < C / 4; jb += 8) {
    float pa[8], vb[8][HD / 16];
#pragma unroll
    for (uint32_t jj = 0; jj < 8; jj++) {
      const uint32_t j = jb + jj;
      pa[jj] = Ps[wave][r * AMMA_PS + 4 * j + grp];
#pragma unroll
      for (uint32_t dt = 0; dt < HD / 16; dt++) vb[jj][dt] = Vs[(4 * j + grp) * AMMA_VS + 16 * dt + r];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t jj = 0; jj < 8; jj++)
#pragma unroll
      for (uint32_t dt = 0; dt < HD / 16; dt++)
        O[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[jj], vb[jj][dt], O[dt], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t qd = q0 + 16 * wave + 4 * grp + i;
    if (qd >= nq || row0 >= nd[i]) continue;
    const uint32_t t = fdiv(qd, a.dgq), h = g * GQ + (qd - t * GQ);
    const uint64_t th = (uint64_t)t * a.heads + h;
#pragma unroll
    for (uint32_t dt = 0; dt < HD / 16; dt++) a.pv[(th * a.smax + c) * HD + 16 * dt + r] = O[dt][i];
    if (r == 0) {
      a.ml[(th * a.smax + c) * 2] = M[i];
      a.ml[(th * a.smax + c) * 2 + 1] = L[i];
    }
  }
}

// The chunks of one (token, head) merged (the flash-decoding combine of
// kernels_fused.go:150-170): M = max m_c, att = sum_c e^{m_c-M} o_c / sum_c
// e^{m_c-M} l_c, over the chunks below the causal bound.  One thread per
// output dimension; the partials of up to 16 chunks are loaded at once.
template <uint32_t HD, bool EMIT = false>
__global__ __launch_bounds__(HD) void attn_merge_kernel(AttnArgs a, AttnOps ops, uint32_t crows) {
  const uint32_t h = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
  const uint32_t n = state_pos(a.state) + t + 1, P = (n + crows - 1) / crows;
  const uint64_t th = (uint64_t)t * a.heads + h;
  const float* ml = a.ml + th * a.smax * 2;
  const float* pv = a.pv + th * a.smax * HD + d;
  constexpr uint32_t B = 16;
  float M = -INFINITY, L = 0, o = 0;
  for (uint32_t c0 = 0; c0 < P; c0 += B) {
    // every load of the batch issued before any is used (chunk clamped below
    // P; the chunks past it are skipped below), so that one wait covers them
    float mc[B], lc[B], oc[B];
#pragma unroll
    for (uint32_t i = 0; i < B; i++) {
      const uint32_t c = min(c0 + i, P - 1);
      mc[i] = ml[2 * c];
      lc[i] = ml[2 * c + 1];
      oc[i] = pv[(uint64_t)c * HD];
    }
    float M2 = M;
#pragma unroll
    for (uint32_t i = 0; i < B; i++) M2 = fmaxf(M2, c0 + i < P ? mc[i] : -INFINITY);
    const float r = __expf(M - M2);  // 0 on the first batch (M = -inf)
    L *= r;
    o *= r;
#pragma unroll
    for (uint32_t i = 0; i < B; i++) {
      const float w = c0 + i < P ? __expf(mc[i] - M2) : 0.f;
      L += w * lc[i];
      o += w * oc[i];
    }
    M = M2;
  }
  a.att[(uint64_t)t * a.heads * HD + h * HD + d] = o / L;
  if (EMIT) emit_operand(ops, t, h * HD + d, o / L);
}

bool attn_ok(uint32_t hd) { return hd == 64 || hd == 128; }

uint32_t attn_full_max(uint32_t hd) { return hd == 64 ? 256 : 128; }

template <uint32_t HD, uint32_t J, bool SPLIT>
static void attn_go(const AttnArgs& a0, uint32_t ntok, uint32_t units, hipStream_t s, const AttnOps& ops) {
  AttnArgs a = a0;
  a.dgq = fast_div(a.heads / a.kv_heads);
  a.dni = fast_div(ntok * a.kv_heads);
  a.dkv = fast_div(a.kv_heads);
  const uint32_t gq = a.heads / a.kv_heads, blocks = 8 * gq * ((units + 7) / 8);
  const dim3 g(blocks), b(512);
  if (!SPLIT && ops.xp) {  // prefill: also the output projection's operands
    if (a.kv16) hipLaunchKernelGGL((attn_kernel<HD, J, false, true, true>), g, b, 0, s, a, ntok, units, ops);
    else hipLaunchKernelGGL((attn_kernel<HD, J, false, false, true>), g, b, 0, s, a, ntok, units, ops);
    return;
  }
  if (a.kv16) hipLaunchKernelGGL((attn_kernel<HD, J, SPLIT, true>), g, b, 0, s, a, ntok, units, ops);
  else hipLaunchKernelGGL((attn_kernel<HD, J, SPLIT, false>), g, b, 0, s, a, ntok, units, ops);
}

// The one-chunk attention at head size 64 over 32 * J rows: one token as
// attn_kernel, several two tokens per workgroup (attn_multi_kernel; measured:
// prefill 53.8k -> 54.8k tok/s, four tokens 53.4k).
template <uint32_t J>
static void attn_one_chunk64(const AttnArgs& a, uint32_t ntok, uint32_t NI, hipStream_t s, const AttnOps& ops) {
  if (ntok == 1) return attn_go<64, J, false>(a, ntok, NI, s, ops);
  constexpr uint32_t QN = 2;
  const uint32_t units = (ntok + QN - 1) / QN * a.kv_heads, gq = a.heads / a.kv_heads;
  const dim3 g(8 * gq * ((units + 7) / 8)), b(512);
  AttnArgs m = a;
  m.dgq = fast_div(gq);
  m.dkv = fast_div(a.kv_heads);
  if (a.kv16) {
    if (ops.xp) hipLaunchKernelGGL((attn_multi_kernel<64, J, true, true, QN>), g, b, 0, s, m, ntok, units, ops);
    else hipLaunchKernelGGL((attn_multi_kernel<64, J, true, false, QN>), g, b, 0, s, m, ntok, units, ops);
  } else {
    if (ops.xp) hipLaunchKernelGGL((attn_multi_kernel<64, J, false, true, QN>), g, b, 0, s, m, ntok, units, ops);
    else hipLaunchKernelGGL((attn_multi_kernel<64, J, false, false, QN>), g, b, 0, s, m, ntok, units, ops);
  }
}

int attn_launch(const AttnArgs& a, uint32_t ntok, hipStream_t s, const AttnOps* ops_in, bool merge) {
  if (ntok == 0) return 0;
  const AttnOps ops = ops_in ? *ops_in : AttnOps{nullptr, nullptr, nullptr, nullptr, 0};
  if (!attn_ok(a.hd) || a.rows == 0 || a.rows > a.ctx || a.kv_heads == 0 || a.heads % a.kv_heads)
    return set_error(LLMHIP_ERR_ARG, "llm: attention: head size %u, %u rows of %u not supported", a.hd, a.rows,
                     a.ctx);
  const uint32_t NI = ntok * a.kv_heads;
  if (!a.split) {
    if (a.rows > attn_full_max(a.hd)) return set_error(LLMHIP_ERR_ARG, "llm: attention: %u rows in one chunk", a.rows);
    if (a.hd == 64) {
      // 32 * J rows per workgroup, J the least even count covering a.rows
      // (a graph variant's multiple of 64), so that few loads repeat the last row
      const uint32_t J = (a.rows + 63) / 64 * 2;
      if (J <= 2) attn_one_chunk64<2>(a, ntok, NI, s, ops);
      else if (J <= 4) attn_one_chunk64<4>(a, ntok, NI, s, ops);
      else if (J <= 6) attn_one_chunk64<6>(a, ntok, NI, s, ops);
      else attn_one_chunk64<8>(a, ntok, NI, s, ops);
    } else {
      attn_go<128, 4, false>(a, ntok, NI, s, ops);
    }
    LLM_HIP(hipGetLastError());
    return 0;
  }
  const uint32_t crows = ntok == 1 ? ATTN_DECODE_ROWS : ATTN_SPLIT_ROWS;
  const uint32_t chunks = (a.rows + crows - 1) / crows;
  if (chunks > a.smax) return set_error(LLMHIP_ERR_ARG, "llm: attention: %u chunks of %u", chunks, a.smax);
  if (ntok == 1) {
    if (a.hd == 64) attn_go<64, ATTN_DECODE_ROWS / 32, true>(a, ntok, NI * chunks, s, ops);
    else attn_go<128, ATTN_DECODE_ROWS / 32, true>(a, ntok, NI * chunks, s, ops);
  } else if (a.hd == 64) {
    // several tokens: the matrix-core form, 64 queries of a KV head per workgroup
    const uint32_t blocks = chunks * a.kv_heads * ((ntok * (a.heads / a.kv_heads) + 63) / 64);
    AttnArgs b = a;
    b.dgq = fast_div(a.heads / a.kv_heads);
    b.dkv = fast_div(a.kv_heads);
    const FastDiv dch = fast_div(chunks);
    if (a.kv16) hipLaunchKernelGGL((attn_mma_kernel<true>), dim3(blocks), dim3(256), 0, s, b, ntok, dch);
    else hipLaunchKernelGGL((attn_mma_kernel<false>), dim3(blocks), dim3(256), 0, s, b, ntok, dch);
  } else {
    attn_go<128, ATTN_SPLIT_ROWS / 32, true>(a, ntok, NI * chunks, s, ops);
  }
  LLM_HIP(hipGetLastError());
  if (!merge) {
    if (ntok != 1 || ops.xp) return set_error(LLMHIP_ERR_ARG, "llm: attention: only one token's merge is left out");
    return 0;
  }
  const dim3 mg(a.heads, ntok);
  if (a.hd == 64) {
    if (ops.xp) hipLaunchKernelGGL((attn_merge_kernel<64, true>), mg, dim3(64), 0, s, a, ops, crows);
    else hipLaunchKernelGGL((attn_merge_kernel<64, false>), mg, dim3(64), 0, s, a, ops, crows);
  } else {
    if (ops.xp) hipLaunchKernelGGL((attn_merge_kernel<128, true>), mg, dim3(128), 0, s, a, ops, crows);
    else hipLaunchKernelGGL((attn_merge_kernel<128, false>), mg, dim3(128), 0, s, a, ops, crows);
  }
  LLM_HIP(hipGetLastError());
  return 0;
}

// Greedy sampling (cpu.go:389-397): the lowest index of the largest logit
// (amax_better), NaN never wins, and a NaN logit 0 is never displaced.
// Combines the per-workgroup partials of the head's matvec (all loads in
// flight at once), writes the token to tokens[step + adv] and out[0]
// (kernels.go:389-392), then advances (pos, step) by adv (kernels.go:397-415).
// QT (the embedding's type; 0: none): then the sampled token's embedding row
// (kernels.go:19-73) also goes to xn, for the next one-token pass.
template <uint32_t QT>
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ pv, const uint32_t* __restrict__ pi,
                                                      uint32_t n, const float* __restrict__ logits,
                                                      int32_t* __restrict__ tokens, int32_t* __restrict__ outb,
                                                      uint32_t* __restrict__ state, uint32_t adv,
                                                      const uint8_t* __restrict__ eq, uint64_t etiles, uint32_t enb,
                                                      uint32_t eng, uint32_t etail, float* __restrict__ xn,
                                                      uint32_t* __restrict__ epoch) {
  __shared__ float sv[16];
  __shared__ uint32_t si[16];
  __shared__ uint32_t tok;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id(), nw = blockDim.x >> 6;
  // what thread 0 reads besides the partials, loaded with them rather than
  // after the reduction (one dependent round trip fewer)
  float l0 = 0.f;
  uint32_t pos = 0, step = 0, ep = 0;
  if (tid == 0) {
    l0 = logits[0];
    pos = state[0];
    step = state[1];
    if (epoch) ep = epoch[0];
  }
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
    if (bi == 0xffffffffu || l0 != l0) bi = 0;
    tokens[step + adv] = (int32_t)bi;
    outb[0] = (int32_t)bi;
    state[0] = pos + adv;
    state[1] = step + adv;
    tok = bi;
    if (epoch) epoch[0] = ep + 1;  // the fused decode pass's flags (pass.h): a new value after every head pass
  }
  if (QT != 0) {
    __syncthreads();
    const uint32_t row = tok;
    for (uint32_t b = tid; b < enb; b += blockDim.x) {
      float v[32];
      dequant_block<QT>(eq, etiles, enb, eng, etail, row, b, v);
      for (int j = 0; j < 32; j++) xn[b * 32 + j] = v[j];
    }
  }
}

int argmax_launch(const float* pv, const uint32_t* pi, uint32_t n, const float* logits, int32_t* tokens,
                  int32_t* outb, uint32_t* state, uint32_t adv, hipStream_t s, const QMat* e, float* xn,
                  uint32_t* epoch) {
  const dim3 g(1), b(1024);
  if (!e || !xn) {
    hipLaunchKernelGGL(argmax_kernel<0>, g, b, 0, s, pv, pi, n, logits, tokens, outb, state, adv, nullptr, 0ull, 0u,
                       0u, 0u, nullptr, epoch);
  } else if (e->g.q.type == LLMHIP_Q4_0) {
    hipLaunchKernelGGL(argmax_kernel<LLMHIP_Q4_0>, g, b, 0, s, pv, pi, n, logits, tokens, outb, state, adv, e->qs,
                       (uint64_t)e->g.tiles, e->g.nb, e->g.ng, e->g.tail, xn, epoch);
  } else if (e->g.q.type == LLMHIP_Q8_0) {
    hipLaunchKernelGGL(argmax_kernel<LLMHIP_Q8_0>, g, b, 0, s, pv, pi, n, logits, tokens, outb, state, adv, e->qs,
                       (uint64_t)e->g.tiles, e->g.nb, e->g.ng, e->g.tail, xn, epoch);
  } else {
    return set_error(LLMHIP_ERR_TYPE, "llm: embedding type %u", e->g.q.type);
  }
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

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                      uint32_t n, float eps, float* __restrict__ out) {
  __shared__ float part[4];
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  float ss = 0;
  for (uint32_t i = tid; i < n; i += 256) ss += x[i] * x[i];
  ss = rows_sum4(row_sum16(ss));
  if (lane == 0) part[wave] = ss;
  __syncthreads();
  const float t = (part[0] + part[1]) + (part[2] + part[3]);
  const float sc = (float)(1.0 / sqrt((double)(t / (float)n + eps)));
  for (uint32_t i = tid; i < n; i += 256) out[i] = __fmul_rn(__fmul_rn(x[i], sc), w[i]);
}

int rmsnorm_launch(const float* x, const float* w, uint32_t n, float eps, float* out, hipStream_t s) {
  if (n == 0 || n > 16384) return set_error(LLMHIP_ERR_ARG, "llm: rmsnorm of %u elements", n);
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(256), 0, s, x, w, n, eps, out);
  LLM_HIP(hipGetLastError());
  return 0;
}

// state = (p, p): a prefill chunk's first position, on its own lane
__global__ void set_state_kernel(uint32_t* state, uint32_t p) {
  if (threadIdx.x == 0) {
    state[0] = p;
    state[1] = p;
  }
}

int set_state_launch(uint32_t* state, uint32_t p, hipStream_t s) {
  hipLaunchKernelGGL(set_state_kernel, dim3(1), dim3(64), 0, s, state, p);
  LLM_HIP(hipGetLastError());
  return 0;
}

int advance_launch(uint32_t* state, uint32_t n, hipStream_t s) {
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, s, state, n);
  LLM_HIP(hipGetLastError());
  return 0;
}

}  // namespace llmhip
