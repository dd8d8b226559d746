// The fused decode pass: every layer of a one-token pass in one persistent
// launch of one workgroup per CU (cpu.go:277-351 per layer; the reference
// records five dispatches per layer, fused.go:259-265).
//
// Each workgroup has a fixed share of each phase of a layer:
//   K1  a tile of [q; k; v]: RMSNorm(x) (attn_norm), the product, bias, RoPE,
//       q out, K and V appended to the cache (kernels_fused.go:47-73);
//   K2  one query head's attention over the cache rows of the pass
//       (kernels_fused.go:82-146, one chunk: every position below
//       attn_full_max);
//   K3  a tile of W_o att plus the residual (kernels_fused.go:150-170);
//   K4  tiles of [gate; up]: RMSNorm (ffn_norm), the product, SwiGLU;
//   K5  a tile of W_down act plus the residual.
// The boundaries between the phases are not kernel boundaries: a phase's
// result goes out as flag-carrying words (PassArgs) and the next phase's
// workgroups poll for the words they need, so a hand-off costs a round trip
// through the memory system instead of a dependent launch.  Every workgroup
// issues its weight loads for a phase before it waits for the phase's input
// (K1, K3 and K4 at the layer's start, K5 after K3), and the attention
// workgroups load the cache rows of earlier positions there too; the row of
// the current position comes from K1's words.
//
// The products are those of the decode tile kernel (gemv_impl.h): weights
// dequantised exactly to f16, activations per unit of 128 elements scaled by
// a power of two and split into f16 hi + lo, v_mfma_f32_16x16x32_f16, the
// block scale in f32; RMSNorm's 1/rms applied to the sums at the end.  The
// waves of a workgroup split a tile's units (split-K) and add their partial
// sums through LDS in wave order, so every result is deterministic.
#include "attn_core.h"
#include "gemv_impl.h"
#include "layer.h"
#include "pass.h"

namespace llmhip {

__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_store(uint64_t* p, float v, uint32_t flag) {
  __hip_atomic_store(p, ((uint64_t)flag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A thread's bounded waits: after `limit` polls of one wait it counts a
// timeout in *err and waits no more (its later reads take whatever is there),
// so the launch always ends.
struct Waiter {
  uint32_t* err;
  uint32_t limit;
  bool dead;
};

// Words base[idx[i]] (those with need[i]) polled until each carries `flag`;
// their f32 values in v (0 where not needed).
template <int N>
__device__ __forceinline__ void ll_wait(const uint64_t* base, const uint32_t (&idx)[N], const bool (&need)[N],
                                        uint32_t flag, float (&v)[N], Waiter& w) {
  uint64_t x[N];
  const uint64_t none = (uint64_t)flag << 32;
#pragma unroll
  for (int i = 0; i < N; i++) x[i] = need[i] ? ll_load(base + idx[i]) : none;
  uint32_t spins = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; i++) ok = ok && (uint32_t)(x[i] >> 32) == flag;
    if (ok || w.dead) break;
    if (++spins > w.limit) {
      w.dead = true;
      atomicOr(w.err, 1u);
      break;
    }
#pragma unroll
    for (int i = 0; i < N; i++)
      if ((uint32_t)(x[i] >> 32) != flag) x[i] = ll_load(base + idx[i]);
  }
#pragma unroll
  for (int i = 0; i < N; i++) v[i] = __uint_as_float((uint32_t)x[i]);
}

template <uint32_t HD>
struct PassLds {
  float xin[PASS_MAX_EMBD];  // a phase's input row
  float misc[16];            // the waves' sums of squares
  float part[PASS_K4_TILES][PASS_WAVES][64];  // split-K partials
  unsigned char wl[PASS_WAVES][WaveLds<1>::BYTES];  // each wave's staged operands
  AttnLds<HD, PASS_WAVES> am;
};

constexpr uint32_t RPT = PASS_MAX_EMBD / (64 * PASS_WAVES);  // row elements per thread

// The phase's input row (n <= PASS_MAX_EMBD floats) into LDS: from
// flag-carrying words (ll) or plain memory (at layer 0, the row the sampling
// kernel wrote).  RMS: returns the row's sum of squares (the waves' partial
// sums added in wave order, the same in every thread).  Ends with a barrier.
template <bool RMS>
__device__ __forceinline__ float stage_row(float* xin, float* misc, const uint64_t* ll, const float* plain, uint32_t n,
                                           uint32_t flag, Waiter& w, uint32_t tid, uint32_t wave) {
  const uint32_t lane = tid & 63;
  float v[RPT];
  if (ll) {
    uint32_t idx[RPT];
    bool need[RPT];
#pragma unroll
    for (uint32_t k = 0; k < RPT; k++) {
      idx[k] = tid + 64 * PASS_WAVES * k;
      need[k] = idx[k] < n;
    }
    ll_wait<RPT>(ll, idx, need, flag, v, w);
  } else {
#pragma unroll
    for (uint32_t k = 0; k < RPT; k++) {
      const uint32_t e = tid + 64 * PASS_WAVES * k;
      v[k] = e < n ? plain[e] : 0.f;
    }
  }
  float ss = 0;
#pragma unroll
  for (uint32_t k = 0; k < RPT; k++) {
    const uint32_t e = tid + 64 * PASS_WAVES * k;
    if (e < n) {
      xin[e] = v[k];
      ss += v[k] * v[k];
    }
  }
  if (RMS) {
    ss = wave_sum_dpp(ss);
    if (lane == 0) misc[wave] = ss;
  }
  __syncthreads();
  float tot = 0;
  if (RMS)
#pragma unroll
    for (uint32_t k = 0; k < PASS_WAVES; k++) tot += misc[k];
  return tot;
}

// Units of a wave in a phase: u = wave + PASS_WAVES * i (a unit is a group of
// four blocks, or the tail of nb % 4 blocks: u == ng), for the workgroup's
// tiles tile[j] (clamped into the matrix; tv[j]: the tile is the
// workgroup's).  Absent units read one line of their tile, so the loads need
// no branch.
template <uint32_t QT, int MT, int MU>
__device__ __forceinline__ void units_load(WUnit (&W)[MT][MU], const PassMat& M, const uint32_t (&tile)[MT],
                                           const bool (&tv)[MT], uint32_t wave, int lane) {
  const int r = lane & 15;
  const uint32_t U = M.ng + (M.tail ? 1u : 0u);
#pragma unroll
  for (int j = 0; j < MT; j++)
#pragma unroll
    for (int i = 0; i < MU; i++) {
      const uint32_t u = wave + PASS_WAVES * i;
      const bool real = tv[j] && u < U;
      if (real && u == M.ng)
        load_unit<QT>(W[j][i], M.qs, M.nb, tile[j], M.ng, M.ng, M.tail, lane, r);
      else
        load_group<QT>(W[j][i], M.qs, M.nb, tile[j], M.ng ? min(u, M.ng - 1) : 0, lane, r, real);
    }
}

// Q8: a Q8_0 matrix may come (else every layer matrix is Q4_0 or Q4_1, and
// the second quant word of WUnit is never live).
template <bool Q8, int MT, int MU>
__device__ __forceinline__ void units_load_any(WUnit (&W)[MT][MU], const PassMat& M, const uint32_t (&tile)[MT],
                                               const bool (&tv)[MT], uint32_t wave, int lane) {
  if (Q8 && M.type == LLMHIP_Q8_0) units_load<LLMHIP_Q8_0, MT, MU>(W, M, tile, tv, wave, lane);
  else if (M.type == LLMHIP_Q4_1) units_load<LLMHIP_Q4_1, MT, MU>(W, M, tile, tv, wave, lane);
  else units_load<LLMHIP_Q4_0, MT, MU>(W, M, tile, tv, wave, lane);
}

// The norm weights of a wave's first batch of items (RMS phases: every unit
// of the wave in one batch), loaded before the wait for the row.
struct NormItems {
  f4 wa, wc;
};
__device__ __forceinline__ NormItems norm_load(const PassMat& M, const float* nw, uint32_t wave, int lane) {
  const uint32_t ub = lane >> 4, b = (lane >> 2) & 3, iq = lane & 3, unit = wave + PASS_WAVES * ub;
  const bool ok = unit < M.ng || (unit == M.ng && b < M.tail);
  const uint32_t e0 = ok ? (unit * 4 + b) * 32 + 4 * iq : 0;
  NormItems n;
  n.wa = *(const f4*)(nw + e0);
  n.wc = *(const f4*)(nw + e0 + 16);
  if (!ok) n.wa = n.wc = f4{0, 0, 0, 0};
  return n;
}

// A wave's partial sums for the workgroup's tiles (acc[j]: lanes of q == 0
// hold row r's sum; see unit_products), its units staged in batches of four
// from the row in LDS (xin; RMS: times the norm weights, nrm) or, FROM_LL,
// straight from flag-carrying words.
template <uint32_t QT, int MT, int MU, bool RMS, bool FROM_LL>
__device__ __forceinline__ void units_products(const WUnit (&W)[MT][MU], const PassMat& M, const float* xin,
                                               const NormItems& nrm, const uint64_t* ll, uint32_t flag, Waiter& wt,
                                               unsigned char* wl, uint32_t wave, int lane, float (&acc)[MT]) {
  constexpr int PRO = RMS ? PRO_RMS : PRO_PLAIN;
  h8* ops = (h8*)wl;
  float* sums = (float*)(wl + WaveLds<1>::OPS);
  float* dxs = (float*)(wl + WaveLds<1>::OPS + WaveLds<1>::TAB);
  const uint32_t U = M.ng + (M.tail ? 1u : 0u);
  const uint32_t nu = U > wave ? (U - 1 - wave) / PASS_WAVES + 1 : 0;
  const int q = lane >> 4, slot = lane & 15;
  const uint32_t ub = lane >> 4, b = (lane >> 2) & 3, iq = lane & 3;
  static_assert(!RMS || MU <= 4, "an RMS phase stages its units in one batch");
#pragma unroll
  for (int i0 = 0; i0 < MU; i0 += 4) {
    if ((uint32_t)i0 >= nu) break;
    ItemsOf<1, PRO> it;
    const uint32_t i = i0 + ub, unit = wave + PASS_WAVES * i;
    const bool ok = i < nu && (unit < M.ng || b < M.tail);
    const uint32_t e0 = ok ? (unit * 4 + b) * 32 + 4 * iq : 0;
    if (FROM_LL) {
      uint32_t idx[8];
      bool need[8];
      float v[8];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        idx[c] = e0 + c;
        idx[4 + c] = e0 + 16 + c;
        need[c] = need[4 + c] = ok;
      }
      ll_wait<8>(ll, idx, need, flag, v, wt);
      it.xa[0] = f4{v[0], v[1], v[2], v[3]};
      it.xc[0] = f4{v[4], v[5], v[6], v[7]};
    } else {
      const f4 z = {0, 0, 0, 0};
      const f4 A = *(const f4*)(xin + e0), C = *(const f4*)(xin + e0 + 16);
      it.xa[0] = ok ? A : z;
      it.xc[0] = ok ? C : z;
    }
    if constexpr (RMS) {
      it.wa = nrm.wa;
      it.wc = nrm.wc;
    }
    const float rs1[1] = {1.f};
    int ex[UB][1];
    stage_items<QT, 1, PRO, 4>(it, rs1, lane, ops, sums, dxs, ex);
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int ii = i0 + u;
      if (ii >= MU || (uint32_t)ii >= nu) break;
      const uint32_t un = wave + PASS_WAVES * ii;
      float dummy = 0;
#pragma unroll
      for (int j = 0; j < MT; j++) {
        if (un == M.ng)
          unit_products<QT, 1, false, true>(W[j][ii], u, (int)M.tail, ops, sums, dxs, ex, q, slot, acc[j], dummy);
        else
          unit_products<QT, 1, false, false>(W[j][ii], u, 4, ops, sums, dxs, ex, q, slot, acc[j], dummy);
      }
    }
  }
}

template <bool Q8, int MT, int MU, bool RMS, bool FROM_LL>
__device__ __forceinline__ void units_products_any(const WUnit (&W)[MT][MU], const PassMat& M, const float* xin,
                                                   const NormItems& nrm, const uint64_t* ll, uint32_t flag,
                                                   Waiter& wt, unsigned char* wl, uint32_t wave, int lane,
                                                   float (&acc)[MT]) {
  if (Q8 && M.type == LLMHIP_Q8_0)
    units_products<LLMHIP_Q8_0, MT, MU, RMS, FROM_LL>(W, M, xin, nrm, ll, flag, wt, wl, wave, lane, acc);
  else if (M.type == LLMHIP_Q4_1)
    units_products<LLMHIP_Q4_1, MT, MU, RMS, FROM_LL>(W, M, xin, nrm, ll, flag, wt, wl, wave, lane, acc);
  else
    units_products<LLMHIP_Q4_0, MT, MU, RMS, FROM_LL>(W, M, xin, nrm, ll, flag, wt, wl, wave, lane, acc);
}

// The waves' partial sums into LDS, a barrier, and for tile j < MT the sum
// in wave order (every lane of wave j; call with the whole workgroup).
template <int MT>
__device__ __forceinline__ float split_sum(float (*part)[PASS_WAVES][64], const float (&acc)[MT], uint32_t wave,
                                           int lane) {
#pragma unroll
  for (int j = 0; j < MT; j++) part[j][wave][lane] = acc[j];
  __syncthreads();
  float v = 0;
  if (wave < (uint32_t)MT)
#pragma unroll
    for (uint32_t w = 0; w < PASS_WAVES; w++) v += part[wave][w][lane];
  return v;
}

template <uint32_t HD, bool KVH, bool Q8>
__global__ __launch_bounds__(512) void pass_kernel(PassArgs a) {
  constexpr uint32_t V4 = HD / 64, JM = HD == 64 ? 8 : 4, S = 4 * PASS_WAVES;
  typedef AttnChunk<HD, JM, PASS_WAVES, KVH> AC;
  __shared__ PassLds<HD> L;
  const uint32_t wg = blockIdx.x, G = gridDim.x;
  const uint32_t E = a.embd, nq = a.embd, nk = a.kvd, hp = HD / 2;
  const uint32_t pos = state_pos(a.state);
  const uint32_t epoch = *(const __attribute__((address_space(4))) uint32_t*)a.ctrl;
  Waiter wt{a.ctrl + 1, a.ctrl[2] ? a.ctrl[2] : PASS_SPIN_DEFAULT, false};
  float* xin = L.xin;
// The thread's indices, redefined at each phase's start: per-lane offsets
// formed from them stay inside the phase (hoisted out of the layer loop, every
// phase's would hold registers through all the others).
#define PHASE_IDS                                      \
  uint32_t tid = threadIdx.x, wave = wave_id();        \
  asm volatile("" : "+v"(tid), "+s"(wave));            \
  const uint32_t lane = tid & 63;                      \
  const int r = lane & 15, q = lane >> 4;              \
  unsigned char* wl = L.wl[wave];                      \
  (void)r;                                             \
  (void)q;                                             \
  (void)wl

  // this workgroup's share (the same for every layer)
  const uint32_t T1 = (E + 2 * a.kvd + 15) / 16, T3 = (E + 15) / 16, T5 = (E + 15) / 16;
  const bool has1 = wg >= a.b1 && wg - a.b1 < T1, has3 = wg >= a.b3 && wg - a.b3 < T3,
             has5 = wg >= a.b5 && wg - a.b5 < T5;
  const uint32_t t1 = has1 ? wg - a.b1 : 0, t3 = has3 ? wg - a.b3 : 0, t5 = has5 ? wg - a.b5 : 0;
  const uint32_t GQ = a.heads / a.kv_heads;
  bool hasA = false;
  uint32_t hg = 0, hh = 0;  // attention: KV head and query head
  if (wg >= a.batt) {  // head h = g GQ + s on workgroup batt + 8 (GQ (g / 8) + s) + g % 8 (one XCD per KV head)
    const uint32_t rel = wg - a.batt, y = rel / 8;
    hg = (y / GQ) * 8 + rel % 8;
    hh = hg * GQ + y % GQ;
    hasA = hg < a.kv_heads;
  }
  const uint32_t rw4 = (wg + G - a.b4 % G) % G;

  for (uint32_t l = 0; l < a.nlayers; l++) {
    const PassLayer& Y = a.layers[l];
    const bool last = l + 1 == a.nlayers;
    const uint32_t F = epoch * a.nlayers + l + 1, Fp = F - 1;  // this layer's flag, the previous layer's
    // the flag-word pointers, redefined in every iteration: addresses formed
    // from them stay inside the iteration (hoisted out of the layer loop they
    // would hold registers through every phase)
    uint64_t *llx = a.llx, *llb = a.llb, *llq = a.llq, *llatt = a.llatt, *llact = a.llact;
    asm volatile("" : "+s"(llx), "+s"(llb), "+s"(llq), "+s"(llatt), "+s"(llact));

    // ---- K1: h = RMSNorm(x) attn_norm; [q; k; v] = W h (+ b); RoPE; K, V appended at pos
    if (has1) {
      const PassMat& M = Y.qkv;
      PHASE_IDS;
      WUnit w1[1][1];
      const uint32_t tt1[1] = {min(t1, M.tiles - 1)};
      const bool v1[1] = {true};
      units_load_any<Q8, 1, 1>(w1, M, tt1, v1, wave, lane);
      const NormItems n1 = norm_load(M, Y.attn_norm, wave, lane);
      const float ss = stage_row<true>(xin, L.misc, l ? llx : nullptr, a.xn, E, Fp, wt, tid, wave);
      float acc[1] = {0};
      units_products_any<Q8, 1, 1, true, false>(w1, M, xin, n1, nullptr, 0, wt, wl, wave, lane, acc);
      float v = split_sum<1>(L.part, acc, wave, lane);
      if (wave == 0) {
        const float rs = rms_scale((double)(ss / (float)E + a.eps));
        v *= rs;
        const uint32_t lr = row_of_pos(t1 * 16 + r, M.map, M.map_hd, M.map_seg0, M.map_seg1, M.ff);
        const bool rv = q == 0 && lr < M.rows;
        if (Y.bias && rv) v += Y.bias[lr];
        const float o = __shfl_xor(v, a.neox ? 8 : 1);
        if (rv) {
          if (lr < nq + nk) {
            const uint32_t j = lr < nq ? lr : lr - nq, w = j & (HD - 1);
            const bool first = a.neox ? w < hp : (w % 2) == 0;
            const uint32_t i = a.neox ? w & (hp - 1) : w / 2;
            const uint64_t co = ((uint64_t)pos * hp + i) * 2;
            const float c = a.cs[co], sn = a.cs[co + 1];
            const float x = first ? v : o, z = first ? o : v;
            const float res = first ? __fsub_rn(__fmul_rn(x, c), __fmul_rn(z, sn))   // cpu.go:381
                                    : __fadd_rn(__fmul_rn(x, sn), __fmul_rn(z, c));  // cpu.go:382
            if (lr < nq) {
              ll_store(llq + lr, res, F);
              if (last) a.q[lr] = res;
            } else {
              const uint64_t ci = (uint64_t)pos * a.kvd + j;
              float kvv = res;
              if (KVH) {
                const _Float16 hv = to_f16(res);
                ((_Float16*)Y.kv)[ci] = hv;
                kvv = (float)hv;
              } else {
                Y.kv[ci] = res;
              }
              ll_store(llq + nq + j, kvv, F);
            }
          } else {
            const uint32_t j = lr - nq - nk;
            const uint64_t ci = (uint64_t)a.ctx * a.kvd + (uint64_t)pos * a.kvd + j;
            float kvv = v;
            if (KVH) {
              const _Float16 hv = to_f16(v);
              ((_Float16*)Y.kv)[ci] = hv;
              kvv = (float)hv;
            } else {
              Y.kv[ci] = v;
            }
            ll_store(llq + nq + nk + j, kvv, F);
          }
        }
      }
    }

    // ---- K2: one query head over rows 0 .. pos (cpu.go:300-334): the rows of
    // earlier positions from the cache, the position's row from K1's words
    if (hasA) {
      PHASE_IDS;
      const uint32_t cl = tid & 15, slot = tid >> 4;
      AC rows;
      {
        // 32-bit element offsets (the cache holds 2 ctx kvd < 2^31 elements)
        const uint32_t lim = max(pos, 1u), Jr = a.rows / S;
        const uint32_t kb = hg * HD + 4 * cl, vb = a.ctx * a.kvd + hg * HD + 4 * cl;
#pragma unroll
        for (uint32_t j = 0; j < JM; j++) {
          if (j >= Jr) break;
          const uint32_t p = min(slot + S * j, lim - 1) * a.kvd;
#pragma unroll
          for (uint32_t v = 0; v < V4; v++) {
            rows.kr[j][v] = kv_load4<KVH>(Y.kv, kb + p + 64 * v);
            rows.vr[j][v] = kv_load4<KVH>(Y.kv, vb + p + 64 * v);
          }
        }
      }
      f4 qv[V4];
      {
        uint32_t idx[4 * V4];
        bool need[4 * V4];
        float v[4 * V4];
#pragma unroll
        for (uint32_t k = 0; k < 4 * V4; k++) {
          idx[k] = hh * HD + 4 * cl + 64 * (k / 4) + k % 4;
          need[k] = true;
        }
        ll_wait<4 * V4>(llq, idx, need, F, v, wt);
#pragma unroll
        for (uint32_t k = 0; k < V4; k++) qv[k] = f4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
      }
      if (slot == pos % S) {  // this thread's rows hold the position's row: K1's words
        uint32_t idx[8 * V4];
        bool need[8 * V4];
        float v[8 * V4];
#pragma unroll
        for (uint32_t k = 0; k < 4 * V4; k++) {
          idx[k] = nq + hg * HD + 4 * cl + 64 * (k / 4) + k % 4;
          idx[4 * V4 + k] = nq + nk + hg * HD + 4 * cl + 64 * (k / 4) + k % 4;
          need[k] = need[4 * V4 + k] = true;
        }
        ll_wait<8 * V4>(llq, idx, need, F, v, wt);
        const uint32_t jp = pos / S;
#pragma unroll
        for (uint32_t j = 0; j < JM; j++)
          if (j == jp)
#pragma unroll
            for (uint32_t k = 0; k < V4; k++) {
              rows.kr[j][k] = f4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
              rows.vr[j][k] = f4{v[4 * V4 + 4 * k], v[4 * V4 + 4 * k + 1], v[4 * V4 + 4 * k + 2],
                                 v[4 * V4 + 4 * k + 3]};
            }
      }
      float M_, L_, o;
      rows.reduce(qv, 0, pos + 1, a.scale, L.am, &M_, &L_, &o);
      if (tid < HD) {
        const float att = o / L_;
        ll_store(llatt + hh * HD + tid, att, F);
        if (last) a.att[hh * HD + tid] = att;
      }
    }

    // ---- K3: x + W_o att
    if (has3) {
      const PassMat& M = Y.o;
      PHASE_IDS;
      WUnit w3[1][1];
      const uint32_t tt3[1] = {min(t3, M.tiles - 1)};
      const bool v3[1] = {true};
      units_load_any<Q8, 1, 1>(w3, M, tt3, v3, wave, lane);
      stage_row<false>(xin, L.misc, llatt, nullptr, E, F, wt, tid, wave);
      float acc[1] = {0};
      const NormItems none = {};
      units_products_any<Q8, 1, 1, false, false>(w3, M, xin, none, nullptr, 0, wt, wl, wave, lane, acc);
      const float v = split_sum<1>(L.part, acc, wave, lane);
      if (wave == 0) {
        const uint32_t lr = t3 * 16 + r;
        const bool rv = q == 0 && lr < M.rows;
        float res = 0;
        if (l == 0) {
          res = rv ? a.xn[lr] : 0.f;
        } else {
          const uint32_t idx[1] = {lr};
          const bool need[1] = {rv};
          float x[1];
          ll_wait<1>(llx, idx, need, Fp, x, wt);
          res = x[0];
        }
        if (rv) ll_store(llb + lr, res + v, F);
      }
    }

    // ---- K4: h = RMSNorm(x) ffn_norm; act = silu(W_gate h) * (W_up h).
    // K5's weights are issued here too (its workgroups take part in K4).
    WUnit w5[1][PASS_K5_UNITS];
    {
      const PassMat& M = Y.gu;
      if (rw4 < M.tiles) {
        PHASE_IDS;
        WUnit w4[PASS_K4_TILES][1];
        uint32_t tt4[PASS_K4_TILES];
        bool v4[PASS_K4_TILES];
#pragma unroll
        for (uint32_t j = 0; j < PASS_K4_TILES; j++) {
          const uint32_t t = rw4 + G * j;
          v4[j] = t < M.tiles;
          tt4[j] = v4[j] ? t : 0;
        }
        units_load_any<Q8, PASS_K4_TILES, 1>(w4, M, tt4, v4, wave, lane);
        const NormItems n4 = norm_load(M, Y.ffn_norm, wave, lane);
        if (has5) {
          const uint32_t tt5[1] = {min(t5, Y.down.tiles - 1)};
          const bool v5[1] = {true};
          units_load_any<Q8, 1, PASS_K5_UNITS>(w5, Y.down, tt5, v5, wave, lane);
        }
        const float ss = stage_row<true>(xin, L.misc, llb, nullptr, E, F, wt, tid, wave);
        float acc[PASS_K4_TILES] = {};
        units_products_any<Q8, PASS_K4_TILES, 1, true, false>(w4, M, xin, n4, nullptr, 0, wt, wl, wave, lane, acc);
        float v = split_sum<PASS_K4_TILES>(L.part, acc, wave, lane);
        const uint32_t tile = rw4 + G * wave;
        if (wave < PASS_K4_TILES && tile < M.tiles) {
          v *= rms_scale((double)(ss / (float)E + a.eps));
          // gate row i at lane r < 8, up row i at r + 8 (MAP_GATEUP)
          const float u = __shfl_xor(v, 8);
          const uint32_t i = 8 * tile + (r & 7);
          if (q == 0 && i < a.ff) {
            if (r < 8) {
              const float act = v / (1.f + __expf(-v)) * u;  // cpu.go:345
              ll_store(llact + i, act, F);
              if (last) a.act[i] = act;
            } else if (last) {
              a.up[i] = v;
            }
          }
        }
      } else if (has5) {
        PHASE_IDS;
        const uint32_t tt5[1] = {min(t5, Y.down.tiles - 1)};
        const bool v5[1] = {true};
        units_load_any<Q8, 1, PASS_K5_UNITS>(w5, Y.down, tt5, v5, wave, lane);
      }
    }

    // ---- K5: x + W_down act
    if (has5) {
      const PassMat& M = Y.down;
      PHASE_IDS;
      __syncthreads();  // K4's epilogue has read the partials (K5 stages no row, whose barrier would order it)
      float acc[1] = {0};
      const NormItems none = {};
      units_products_any<Q8, 1, PASS_K5_UNITS, false, true>(w5, M, nullptr, none, llact, F, wt, wl, wave, lane, acc);
      const float v = split_sum<1>(L.part, acc, wave, lane);
      if (wave == 0) {
        const uint32_t lr = t5 * 16 + r;
        const bool rv = q == 0 && lr < M.rows;
        const uint32_t idx[1] = {lr};
        const bool need[1] = {rv};
        float x[1];
        ll_wait<1>(llb, idx, need, F, x, wt);
        if (rv) {
          if (last) a.x[lr] = x[0] + v;
          else ll_store(llx + lr, x[0] + v, F);
        }
      }
    }
  }
}

#undef PHASE_IDS

// ------------------------------------------------------------------ host

const char* pass_unfit(const llmhip_config& c, uint32_t kvd, const PassMat& qkv, const PassMat& o, const PassMat& gu,
                       const PassMat& down, uint32_t grid) {
  if (grid == 0) return "no co-resident grid";
  if (c.head_dim != 64 && c.head_dim != 128) return "head size";
  if ((uint32_t)c.embd > PASS_MAX_EMBD) return "embedding above the staged row";
  const uint32_t E = (uint32_t)c.embd, GQ = (uint32_t)(c.heads / c.kv_heads);
  if ((E + 2 * kvd + 15) / 16 > grid || (E + 15) / 16 > grid) return "more tiles than workgroups";
  if (8 * GQ * ((uint32_t)(c.kv_heads + 7) / 8) > grid) return "more heads than workgroups";
  auto units = [](const PassMat& m) { return m.ng + (m.tail ? 1u : 0u); };
  if (units(qkv) > PASS_WAVES || units(o) > PASS_WAVES || units(gu) > PASS_WAVES)
    return "more units per tile than waves";
  if (units(down) > PASS_WAVES * PASS_K5_UNITS) return "down projection too long";
  if (gu.tiles > PASS_K4_TILES * grid) return "gate/up too tall";
  if (gu.map != MAP_GATEUP || o.map != MAP_IDENT || down.map != MAP_IDENT) return "row maps";
  if (qkv.rows != E + 2 * kvd || o.rows != E || down.rows != E || gu.rows != 2 * (uint32_t)c.ff) return "shapes";
  return nullptr;
}

template <uint32_t HD, bool KVH>
static uint32_t grid_of(int device) {
  int n = 0, n8 = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, pass_kernel<HD, KVH, false>, 64 * PASS_WAVES, 0) !=
          hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&n8, pass_kernel<HD, KVH, true>, 64 * PASS_WAVES, 0) != hipSuccess)
    return 0;
  n = std::min(n, n8);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
  return n >= 1 && cus > 0 ? (uint32_t)cus : 0;
}

uint32_t pass_grid(int device, uint32_t hd, bool kv16) {
  // (the Q8 form holds more registers: its occupancy bounds both)
  if (hd == 64) return kv16 ? grid_of<64, true>(device) : grid_of<64, false>(device);
  if (hd == 128) return kv16 ? grid_of<128, true>(device) : grid_of<128, false>(device);
  return 0;
}

// K1's tiles from workgroup 0, the attention heads after them (from a
// multiple of 8: a KV head's query heads on one XCD), K3's tiles after those
// where they fit, K5's at the end (their weights are the largest share a
// workgroup holds), K4 round robin over the whole grid.  Where the grid is
// too small for disjoint ranges they overlap (the phases run in turn).
void pass_place(PassArgs* a, uint32_t grid, uint32_t t1, uint32_t t3, uint32_t t5, uint32_t natt) {
  a->b1 = 0;
  a->batt = (t1 + 7) / 8 * 8;
  if (a->batt + natt > grid) a->batt = 0;
  a->b5 = grid - t5;
  const uint32_t e = std::max(t1, a->batt + natt);
  a->b3 = e + t3 <= grid - t5 ? e : 0;
  a->b4 = 0;
}

template <uint32_t HD, bool KVH>
static void go(const PassArgs& a, uint32_t grid, bool q8, hipStream_t s) {
  if (q8) hipLaunchKernelGGL((pass_kernel<HD, KVH, true>), dim3(grid), dim3(64 * PASS_WAVES), 0, s, a);
  else hipLaunchKernelGGL((pass_kernel<HD, KVH, false>), dim3(grid), dim3(64 * PASS_WAVES), 0, s, a);
}

int pass_launch(const PassArgs& a, uint32_t grid, bool q8, hipStream_t s) {
  if (a.hd == 64) {
    if (a.kv16) go<64, true>(a, grid, q8, s);
    else go<64, false>(a, grid, q8, s);
  } else if (a.hd == 128) {
    if (a.kv16) go<128, true>(a, grid, q8, s);
    else go<128, false>(a, grid, q8, s);
  } else {
    return set_error(LLMHIP_ERR_ARG, "llm: decode pass: head size %u", a.hd);
  }
  LLM_HIP(hipGetLastError());
  return 0;
}

}  // namespace llmhip
