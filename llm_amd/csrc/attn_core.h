// The attention of one query head over one chunk of cache rows, by a
// workgroup of NW waves (cpu.go:300-334): s = (q . k) * scale, the chunk's
// max, e = exp(s - max), l = sum e, o = sum e v.  Lane c of a 16-lane row
// holds float4 c (and c+16 for HD 128) of key and value rows; slot = tid / 16
// serves rows row0 + slot + S*j (S = 4*NW slots, j < J), so a chunk is
// C = S*J rows.  Loads are coalesced rows, a score is a 16-lane DPP sum that
// lands in the lanes holding the matching value row, and the weighted value
// sums are reduced over rows by two shuffles and over waves through LDS.
// attn_kernel (layer.hip) runs one chunk per workgroup with it.
#pragma once

#include "wave.h"

namespace llmhip {

typedef float f4 __attribute__((ext_vector_type(4)));

// Four consecutive cache elements as f32: an f32 cache, or binary16 (F16KV)
// widened exactly.
template <bool KVH>
__device__ __forceinline__ f4 kv_load4(const float* kv, uint64_t i) {
  if (!KVH) return *(const f4*)(kv + i);
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 h = *(const h4*)((const _Float16*)kv + i);
  return f4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

template <uint32_t HD, uint32_t NW, uint32_t QN = 1>
struct AttnLds {
  float m[QN][NW], l[QN][NW];
  f4 o[QN][NW * 16 * (HD / 64)];
};

template <uint32_t HD, uint32_t J, uint32_t NW, bool KVH>
struct AttnChunk {
  static constexpr uint32_t V4 = HD / 64, S = 4 * NW, C = S * J;
  f4 kr[J][V4], vr[J][V4];

  // Issue the loads of rows row0 + slot + S*j of KV head g (the cache is
  // [2][ctx][kvd]); a row at or past lim (1 <= lim <= ctx) loads row lim - 1
  // instead, which reduce masks out with the rest past the causal bound.
  // The loads are unconditional and all key rows go out before the value
  // rows: loads complete in issue order, so the scores wait for the keys
  // only, and the values arrive under the score, max and barrier phase.
  __device__ __forceinline__ void load(const float* kv, uint32_t kvd, uint32_t ctx, uint32_t g, uint32_t row0,
                                       uint32_t lim) {
    const uint32_t cl = threadIdx.x & 15, slot = threadIdx.x >> 4;
    const uint64_t kb = g * HD + 4 * cl, vb = (uint64_t)ctx * kvd + g * HD + 4 * cl;  // element offsets
    uint32_t p[J];
#pragma unroll
    for (uint32_t j = 0; j < J; j++) p[j] = min(row0 + slot + S * j, lim - 1);
#pragma unroll
    for (uint32_t j = 0; j < J; j++)
#pragma unroll
      for (uint32_t v = 0; v < V4; v++) kr[j][v] = kv_load4<KVH>(kv, kb + (uint64_t)p[j] * kvd + 64 * v);
#pragma unroll
    for (uint32_t j = 0; j < J; j++)
#pragma unroll
      for (uint32_t v = 0; v < V4; v++) vr[j][v] = kv_load4<KVH>(kv, vb + (uint64_t)p[j] * kvd + 64 * v);
    __builtin_amdgcn_sched_barrier(0);  // no arithmetic (and no wait) scheduled between the loads
  }

  // The rows below n (all of them loaded or set), with q the lane's float4
  // slice of the query: returns the chunk's max M in every thread, and its
  // sum L and o = sum e v[d] for d = tid < HD.  Each wave weighs its rows by
  // its own max m_w (e = exp(s - m_w), l_w = sum e, o_w = sum e v); one
  // barrier shares them, and the output's threads combine them in wave order
  // with the weights exp(m_w - M), M = max m_w.  Call with the whole
  // workgroup; at least one row below n.
  __device__ __forceinline__ void reduce(const f4 (&q)[V4], uint32_t row0, uint32_t n, float scale,
                                         AttnLds<HD, NW>& sm, float* M_out, float* L_out, float* o_out) const {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id(), cl = lane & 15, slot = tid >> 4;
    float sj[J], m = -INFINITY;
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
      const uint32_t p = row0 + slot + S * j;
      float d = 0;
      if (p < n)
#pragma unroll
        for (uint32_t v = 0; v < V4; v++)
          d += q[v][0] * kr[j][v][0] + q[v][1] * kr[j][v][1] + q[v][2] * kr[j][v][2] + q[v][3] * kr[j][v][3];
      d = row_sum16(d);
      sj[j] = p < n ? d * scale : -INFINITY;
      m = fmaxf(m, sj[j]);
    }
    m = rows_max4(m);  // the wave's max (-inf if none of its rows is below n)
    f4 acc[V4];
#pragma unroll
    for (uint32_t v = 0; v < V4; v++) acc[v] = f4{0, 0, 0, 0};
    float l = 0;
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
      const uint32_t p = row0 + slot + S * j;
      if (p < n) {
        const float e = __expf(sj[j] - m);  // v_exp_f32: a few ulp, inside the parity bounds
        l += e;
#pragma unroll
        for (uint32_t v = 0; v < V4; v++) acc[v] += e * vr[j][v];
      }
    }
    l = rows_sum4(l);
#pragma unroll
    for (uint32_t v = 0; v < V4; v++)
#pragma unroll
      for (int k = 0; k < 4; k++) {
        acc[v][k] += xor16(acc[v][k], lane);
        acc[v][k] += xor32(acc[v][k], lane);
      }
    if (lane < 16)
#pragma unroll
      for (uint32_t v = 0; v < V4; v++) sm.o[0][(wave * 16 + cl) * V4 + v] = acc[v];
    if (lane == 0) {
      sm.m[0][wave] = m;
      sm.l[0][wave] = l;
    }
    __syncthreads();
    float mw[NW], M = -INFINITY;
#pragma unroll
    for (uint32_t w = 0; w < NW; w++) {
      mw[w] = sm.m[0][w];
      M = fmaxf(M, mw[w]);
    }
    *M_out = M;
    float L = 0, o = 0;
    if (tid < HD) {
      const uint32_t fi = tid / 4, ci = fi % 16, vi = fi / 16, k = tid % 4;
#pragma unroll
      for (uint32_t w = 0; w < NW; w++) {
        const float c = mw[w] == -INFINITY ? 0.f : __expf(mw[w] - M);
        L += c * sm.l[0][w];
        o += c * sm.o[0][(w * 16 + ci) * V4 + vi][k];
      }
    }
    *L_out = L;
    *o_out = o;
  }

  // reduce for QN queries of one head over the same rows (several tokens of a
  // prefill chunk): query i has its slice q[i] and its causal bound n[i]; out
  // per query as reduce's, but with the chunk's max shared first (a barrier)
  // and every row weighed by it: two barriers for all QN.
  template <uint32_t QN>
  __device__ __forceinline__ void reduce_n(const f4 (&q)[QN][V4], uint32_t row0, const uint32_t (&n)[QN],
                                           float scale, AttnLds<HD, NW, QN>& sm, float (&M_out)[QN],
                                           float (&L_out)[QN], float (&o_out)[QN]) const {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = wave_id(), cl = lane & 15, slot = tid >> 4;
    float sj[QN][J], m[QN];
#pragma unroll
    for (uint32_t i = 0; i < QN; i++) {
      m[i] = -INFINITY;
#pragma unroll
      for (uint32_t j = 0; j < J; j++) {
        const uint32_t p = row0 + slot + S * j;
        float d = 0;
#pragma unroll
        for (uint32_t v = 0; v < V4; v++)
          d += q[i][v][0] * kr[j][v][0] + q[i][v][1] * kr[j][v][1] + q[i][v][2] * kr[j][v][2] +
               q[i][v][3] * kr[j][v][3];
        d = row_sum16(d);
        sj[i][j] = p < n[i] ? d * scale : -INFINITY;
        m[i] = fmaxf(m[i], sj[i][j]);
      }
      m[i] = rows_max4(m[i]);
      if (lane == 0) sm.m[i][wave] = m[i];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t i = 0; i < QN; i++) {
      float M = sm.m[i][0];
#pragma unroll
      for (uint32_t w = 1; w < NW; w++) M = fmaxf(M, sm.m[i][w]);
      M_out[i] = M;
      f4 acc[V4];
#pragma unroll
      for (uint32_t v = 0; v < V4; v++) acc[v] = f4{0, 0, 0, 0};
      float l = 0;
#pragma unroll
      for (uint32_t j = 0; j < J; j++) {
        const uint32_t p = row0 + slot + S * j;
        if (p < n[i]) {
          const float e = __expf(sj[i][j] - M);
          l += e;
#pragma unroll
          for (uint32_t v = 0; v < V4; v++) acc[v] += e * vr[j][v];
        }
      }
      l = rows_sum4(l);
#pragma unroll
      for (uint32_t v = 0; v < V4; v++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
          acc[v][k] += xor16(acc[v][k], lane);
          acc[v][k] += xor32(acc[v][k], lane);
        }
      if (lane < 16)
#pragma unroll
        for (uint32_t v = 0; v < V4; v++) sm.o[i][(wave * 16 + cl) * V4 + v] = acc[v];
      if (lane == 0) sm.l[i][wave] = l;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t i = 0; i < QN; i++) {
      float L = 0, o = 0;
      if (tid < HD) {
        const uint32_t fi = tid / 4, ci = fi % 16, vi = fi / 16, k = tid % 4;
#pragma unroll
        for (uint32_t w = 0; w < NW; w++) {
          L += sm.l[i][w];
          o += sm.o[i][(w * 16 + ci) * V4 + vi][k];
        }
      }
      L_out[i] = L;
      o_out[i] = o;
    }
  }
};

}  // namespace llmhip
