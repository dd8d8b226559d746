// The fused decode pass: every layer of a one-token pass in one persistent
// launch of one workgroup per CU (cpu.go:277-351 per layer; the reference
// records five dispatches per layer, fused.go:259-265).
//
// Each workgroup has a fixed share of each phase of a layer:
//   K1  a tile of [q; k; v]: RMSNorm(x) (attn_norm, its scale applied to the
//       product), the product, bias, RoPE, q out, K and V appended to the
//       cache (kernels_fused.go:47-73);
//   K2  one query head over one chunk of 128 cache rows: the chunk's max
//       score, sum of e and sum of e v (kernels_fused.go:82-146; every
//       position is below attn_full_max, so there are one or two chunks);
//       the second chunk's workgroup merges the first's sums into its own as
//       attn_merge_kernel merges chunks and writes the head's output;
//   K3  a tile of W_o att plus the residual (kernels_fused.go:150-170);
//   K4  tiles of [gate; up]: RMSNorm (ffn_norm, as K1's), the product, SwiGLU;
//   K5  one of kp k-parts of a tile of W_down act; the next layer adds the
//       parts to the residual, in order.
// The boundaries between the phases are not kernel boundaries: a phase's
// result goes out as flag-carrying words (PassArgs) and the next phase's
// workgroups poll for the words they need, so a hand-off costs a round trip
// through the memory system instead of a dependent launch.  Every workgroup
// issues a phase's weight loads, and the loads of the inputs its epilogue
// needs, before it waits for the phase's input; the attention workgroups load
// the cache rows of earlier positions before waiting for K1's row of the
// position.
//
// The products run on v_mfma_f32_16x16x32_f16 as the decode kernels' do
// (gemv_impl.h): weights dequantised exactly to f16, the staged row scaled by
// a power of two and split into f16 hi + lo, the block scale in f32.  The
// waves of a workgroup split a tile's units (split-K) and add their partial
// sums through LDS in wave order; the k-parts are added in part order: every
// result is deterministic.
#include "attn_core.h"
#include "gemv_impl.h"
#include "layer.h"
#include "pass.h"

namespace llmhip {

// The flag-carrying words are device memory: their atomics take the global
// address space (global_load / global_store with sc1), not the generic one,
// whose flat instructions also count in the LDS and scalar wait counter.
typedef __attribute__((address_space(1))) uint64_t gword;
__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
  return __hip_atomic_load((const gword*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_store(uint64_t* p, float v, uint32_t flag) {
  __hip_atomic_store((gword*)p, ((uint64_t)flag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// A thread's bounded waits: after `limit` polls of one wait it counts a
// timeout in *err and waits no more (its later reads take whatever is there),
// so the launch always ends.
struct Waiter {
  uint32_t* err;
  uint32_t limit;
  bool dead;
};

// Words at(i) (those with need(i)) polled until each carries `flag`; their
// f32 values in v (0 where not needed).  Every load is issued before the first
// wait; a retry follows a short pause.  The addresses and conditions are
// formed again where used (a thread holds only the words, not N addresses).
template <int N, class At, class Need>
__device__ __forceinline__ void ll_wait_f(At at, Need need, uint32_t flag, float (&v)[N], Waiter& w) {
  uint64_t x[N];
  const uint64_t none = (uint64_t)flag << 32;
#pragma unroll
  for (int i = 0; i < N; i++) x[i] = need(i) ? ll_load(at(i)) : none;
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
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; i++)
      if ((uint32_t)(x[i] >> 32) != flag) x[i] = ll_load(at(i));
  }
#pragma unroll
  for (int i = 0; i < N; i++) v[i] = __uint_as_float((uint32_t)x[i]);
}

constexpr int PASS_GATE_STAGGER = 6;  // s_sleep units (64 cycles) between the gate's two first polls

// ll_wait_f preceded by a gate: the wave's first lane polls its word `gate`
// alone until it carries the flag (a word of the input's last producers).  A workgroup that reaches a phase long
// before the phase's input is produced then waits with one load in flight
// per wave instead of its whole input's, which leaves the memory system to
// the phases still running.
template <int N, class At, class Need>
__device__ __forceinline__ void ll_wait_gated(At at, Need need, uint32_t flag, float (&v)[N], Waiter& w,
                                              int gate = 0) {
  // lane 0's word `gate`, polled by the whole wave at one address (one
  // request), two polls in flight started PASS_GATE_STAGGER apart: each check
  // waits for the older one only (loads return in order), so a word that
  // lands between two polls is seen about half a round trip sooner
  const uint64_t gp = (uint64_t)at(gate);
  const uint64_t* p0 = (const uint64_t*)(((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(gp >> 32)) << 32) |
                                         (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)gp));
  if (__builtin_amdgcn_readfirstlane(need(gate) ? 1 : 0) && !w.dead) {
    uint64_t x0 = ll_load(p0);
    __builtin_amdgcn_s_sleep(PASS_GATE_STAGGER);
    uint64_t x1 = ll_load(p0);
    uint32_t spins = 0;
    auto done = [&](uint64_t x) {
      if (__builtin_amdgcn_readfirstlane((uint32_t)(x >> 32)) == flag) return true;
      if (++spins > w.limit) {  // (spins: the same in every lane)
        atomicOr(w.err, 1u);
        w.dead = true;
        return true;
      }
      return false;
    };
    for (;;) {
      if (done(x0)) break;
      x0 = ll_load(p0);
      if (done(x1)) break;
      x1 = ll_load(p0);
    }
  }
  ll_wait_f<N>(at, need, flag, v, w);
}

// ll_wait_gated or, where the input is expected soon, ll_wait_f.
template <int N, class At, class Need>
__device__ __forceinline__ void ll_wait_row(bool gate, At at, Need need, uint32_t flag, float (&v)[N], Waiter& w,
                                            int gate_word = 0) {
  if (gate) ll_wait_gated<N>(at, need, flag, v, w, gate_word);
  else ll_wait_f<N>(at, need, flag, v, w);
}

// ll_wait_f over base[idx[i]] where need[i].
template <int N>
__device__ __forceinline__ void ll_wait(const uint64_t* base, const uint32_t (&idx)[N], const bool (&need)[N],
                                        uint32_t flag, float (&v)[N], Waiter& w) {
  ll_wait_f<N>([&](int i) { return base + idx[i]; }, [&](int i) { return need[i]; }, flag, v, w);
}

// The value of a flag-carrying word loaded earlier (x, from p), polled again
// until it carries `flag` (bounded).
__device__ __forceinline__ float ll_settle(const uint64_t* p, uint64_t x, uint32_t flag, Waiter& w) {
  uint32_t spins = 0;
  while ((uint32_t)(x >> 32) != flag && !w.dead) {
    if (++spins > w.limit) {
      w.dead = true;
      atomicOr(w.err, 1u);
      break;
    }
    x = ll_load(p);
  }
  return __uint_as_float((uint32_t)x);
}

constexpr uint32_t PASS_MAX_ITEMS = PASS_MAX_FF / 8;  // items of 8 elements of the longest staged row

template <uint32_t HD>
struct PassLds {
  float row[PASS_MAX_FF];         // the phase's input row as polled (f32)
  float nw[PASS_MAX_EMBD];        // RMS phases: the norm weights
  h8 xs[2 * PASS_MAX_ITEMS];      // the phase's A operands: item it at 2 it (hi) and 2 it + 1 (lo)
  float bsum[PASS_MAX_ITEMS / 4];  // Q4_1: each block's sum, scaled like the operands
  // The RMSNorm phases' partial sums of squares ([0] K1, [1] K4) and split-K
  // partials, one copy per layer parity: no barrier precedes a phase's
  // products, so a wave may write a layer's while another still reads those
  // of the layer before; two layers back, the phase's own barrier has passed.
  float ss[2][2][PASS_WAVES];
  float part1[2][1][PASS_WAVES][64];
  float part4[2][PASS_K4_TILES][PASS_WAVES][64];
  float part2[1][PASS_WAVES][64];  // K3's and K5's: the phases between them have barriers
  AttnLds<HD, PASS_WAVES> am;
  float mrg[PASS_LONG_CHUNKS][HD + 2];  // the long form's merge: each chunk's o, m and l
};

// Where an RMSNorm phase's input row comes from (stage_rms_wave).
enum PassSrc : int {
  SRC_LL,     // one vector of flag-carrying words
  SRC_PLAIN,  // plain memory (layer 0's input, which the sampling kernel wrote)
  SRC_XSUM,   // x = ((xb + p_0) + p_1) + ...: the attention's residual and the down projection's k-parts
};

struct StageIn {
  const uint64_t* ll;  // SRC_LL: the vector; SRC_XSUM: xb, then part p at (1 + p) E
  const float* plain;  // SRC_PLAIN
  uint32_t flag, kp, E;
  bool gate;           // wait behind a gate word (ll_wait_gated): the input is expected late
};

// The wave's units' items (those of units_load: u = u0 + wave + 8 i < u1,
// i < MU) from the row in LDS: item it = (block it / 4, k-group it % 4:
// elements 4 (it % 4) + 0..3 and 16 + 4 (it % 4) + 0..3 of the block) in MFMA
// element order, RMS: h = (x s) w (cpu.go:96), scaled by 2^ex and split
// exactly into f16 hi (xs[2 it]) + lo (xs[2 it + 1]); the blocks' sums (Q4_1:
// cpu.go:196-198) scaled alike.  Only the wave reads them.
template <bool RMS, int MU, uint32_t HD>
__device__ __forceinline__ void form_items(PassLds<HD>& L, uint32_t nb, uint32_t u0, uint32_t u1, float s, int ex,
                                           uint32_t wave, uint32_t lane) {
  static_assert(16 * MU <= 64, "a wave forms its units' items in one pass");
  const uint32_t NI = nb * 4;
  // lane: item lane % 16 of the wave's unit lane / 16
  const uint32_t i = lane / 16, u = u0 + wave + PASS_WAVES * i;
  const uint32_t it = 16 * (u - u0) + (lane & 15);
  const bool ok = (int)i < MU && u < u1 && it < NI;
  const uint32_t e0 = (it / 4) * 32 + 4 * (it % 4);
  f4 a = {0, 0, 0, 0}, c = {0, 0, 0, 0};
  if (ok) {
    a = *(const f4*)&L.row[e0];
    c = *(const f4*)&L.row[e0 + 16];
    if (RMS) {
      const f4 wa = *(const f4*)&L.nw[e0], wc = *(const f4*)&L.nw[e0 + 16];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        a[k] = __fmul_rn(__fmul_rn(a[k], s), wa[k]);  // cpu.go:96
        c[k] = __fmul_rn(__fmul_rn(c[k], s), wc[k]);
      }
    }
  }
  const float vv[8] = {a[0], a[2], c[0], c[2], a[1], a[3], c[1], c[3]};
  h8 hi, lo;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const float sv = ldexpf(vv[k], ex);
    const _Float16 h = (_Float16)sv;
    hi[k] = h;
    lo[k] = (_Float16)(sv - (float)h);
  }
  float sx = (a[0] + a[1] + a[2] + a[3]) + (c[0] + c[1] + c[2] + c[3]);
  sx += __shfl_xor(sx, 1);  // a block's four items: four consecutive lanes
  sx += __shfl_xor(sx, 2);
  if (ok) {
    L.xs[2 * it] = hi;
    L.xs[2 * it + 1] = lo;
    if ((it & 3) == 0) L.bsum[it / 4] = ldexpf(sx, ex);
  }
  __builtin_amdgcn_wave_barrier();
}

// An RMSNorm phase's input (K1, K4: a row of nb blocks of 32) staged by each
// wave for its own units only, with no workgroup barrier, as stage_wave
// stages K3's and K5's: the wave reads its units' elements (SRC_XSUM: the
// residual, then the k-parts added in order) and their norm weights (loaded
// before the wait), puts y = x w into its part of the row in LDS and forms its
// items from it scaled by its own 2^ex (its largest |y| in [2^14, 2^15)); its
// partial sum of x^2 goes to ss[wave].  The product is then formed as
// s (W y), s from the waves' sums (rms_of), for cpu.go:90-96's W ((x s) w).
// Returns the wave's ex.
template <int SRC, int MU, uint32_t HD>
__device__ __forceinline__ int stage_rms_wave(PassLds<HD>& L, const StageIn& in, uint32_t nb, uint32_t u0,
                                              uint32_t u1, const float* nw, float* ss, Waiter& w, uint32_t wave,
                                              uint32_t lane) {
  constexpr int NE = 2 * MU;
  const uint32_t n = nb * 32;
  // element j: 128 (u - u0) + 64 (j % 2) + lane of unit u = u0 + wave + 8 (j / 2)
  auto el = [&](int j) { return 128 * (wave + PASS_WAVES * (j / 2)) + 64 * (j % 2) + lane; };
  auto need = [&](int j) { return u0 + wave + PASS_WAVES * (j / 2) < u1 && el(j) < n; };
  float wv[NE], x[NE];
#pragma unroll
  for (int j = 0; j < NE; j++) wv[j] = need(j) ? nw[el(j)] : 0.f;
  if constexpr (SRC == SRC_PLAIN) {
#pragma unroll
    for (int j = 0; j < NE; j++) x[j] = need(j) ? in.plain[el(j)] : 0.f;
  } else if constexpr (SRC == SRC_LL) {
    ll_wait_row<NE>(in.gate, [&](int j) { return in.ll + el(j); }, need, in.flag, x, w);
  } else if constexpr (SRC == SRC_XSUM) {
    constexpr uint32_t NP = 1 + PASS_MAX_KP;
    float u[NE * NP];
    // word i: vector i / NE (xb, then the parts), element i % NE; the gate:
    // the wave's word of the last k-part, whose producers finish last
    ll_wait_row<NE * NP>(in.gate, [&](int i) { return in.ll + (i / NE) * in.E + el(i % NE); },
                         [&](int i) { return (uint32_t)(i / NE) <= in.kp && need(i % NE); }, in.flag, u, w,
                         (int)(in.kp * NE));
#pragma unroll
    for (int k = 0; k < NE; k++) {
      x[k] = u[k];
#pragma unroll
      for (uint32_t q = 1; q < NP; q++)
        if (q <= in.kp) x[k] += u[q * NE + k];
    }
  }
  float s2 = 0, mx = 0;
#pragma unroll
  for (int j = 0; j < NE; j++) {
    const float y = __fmul_rn(x[j], wv[j]);
    if (need(j)) L.row[el(j)] = y;
    s2 += x[j] * x[j];  // (0 where not needed)
    mx = fmaxf(mx, fabsf(y));
  }
  s2 = wave_sum_dpp(s2);
  mx = wave_max_dpp(mx);  // (the same in every lane)
  if (lane == 0) ss[wave] = s2;
  __builtin_amdgcn_wave_barrier();
  int ex = 0;
  if (mx > 0 && mx <= 3.0e38f) {
    int E;
    frexpf(mx, &E);
    ex = 15 - E;
  }
  form_items<false, MU>(L, nb, u0, u1, 1.f, ex, wave, lane);
  return ex;
}

// The RMS scale s = f32(1/sqrt(f64(sum x^2 / n + eps))) (cpu.go:90-96) from
// the waves' partial sums (stage_rms_wave), added in wave order; read after
// a barrier that follows every wave's stage.
__device__ __forceinline__ float rms_of(const float* ss, uint32_t n, float eps) {
  float tot = 0;
#pragma unroll
  for (uint32_t k = 0; k < PASS_WAVES; k++) tot += ss[k];
  return rms_scale((double)(tot / (float)n + eps));
}

// The phase's input row (one vector of flag-carrying words, nb blocks of 32
// from block nb0 on) staged by each wave for its own units only, with no
// workgroup barrier: the wave polls its units' elements (unit u: blocks
// 4 (u - u0) .. 4 (u - u0) + 3 of the row) into its part of the row in LDS
// and forms their items scaled by its own 2^ex (its largest |x| in
// [2^14, 2^15)).  A wave whose input is in starts its products while the
// others still wait; each wave scales its sums back by 2^-ex (exact) before
// the waves' sums are added.  Returns the wave's ex.
template <int MU, bool ACT, uint32_t HD>
__device__ __forceinline__ int stage_wave(PassLds<HD>& L, const StageIn& in, uint32_t nb0, uint32_t nb, uint32_t u0,
                                          uint32_t u1, Waiter& w, uint32_t wave, uint32_t lane) {
  const uint32_t n = nb * 32;
  // word j: element 128 (u - u0) + 64 (j % 2) + lane of unit u = u0 + wave + 8 (j / 2)
  auto el = [&](int j) { return 128 * (wave + PASS_WAVES * (j / 2)) + 64 * (j % 2) + lane; };
  auto need = [&](int j) { return u0 + wave + PASS_WAVES * (j / 2) < u1 && el(j) < n; };
  auto at = [&](int j) {
    const uint32_t e = 32 * nb0 + el(j);
    return in.ll + (ACT ? e + (e & ~7u) : e);  // ACT: 8 of every 16 words
  };
  float v[2 * MU];
  ll_wait_row<2 * MU>(in.gate, at, need, in.flag, v, w);
  float mx = 0;
#pragma unroll
  for (int j = 0; j < 2 * MU; j++) {
    if (need(j)) L.row[el(j)] = v[j];
    mx = fmaxf(mx, fabsf(v[j]));
  }
  mx = wave_max_dpp(mx);  // (the same in every lane)
  __builtin_amdgcn_wave_barrier();
  int ex = 0;
  if (mx > 0 && mx <= 3.0e38f) {
    int E;
    frexpf(mx, &E);
    ex = 15 - E;
  }
  form_items<false, MU>(L, nb, u0, u1, 1.f, ex, wave, lane);
  return ex;
}

// Units of a wave in a phase: u = u0 + wave + PASS_WAVES * i < u1 (a unit is a
// group of four blocks, or the tail of nb % 4 blocks: u == ng), for the
// workgroup's tiles tile[j] (clamped into the matrix; tv[j]: the tile is the
// workgroup's).  Absent units read one line of their tile, so the loads need
// no branch.
template <uint32_t QT, int MT, int MU>
__device__ __forceinline__ void units_load(WUnit (&W)[MT][MU], const PassMat& M, const uint32_t (&tile)[MT],
                                           const bool (&tv)[MT], uint32_t u0, uint32_t u1, uint32_t wave, int lane) {
  const int r = lane & 15;
#pragma unroll
  for (int j = 0; j < MT; j++)
#pragma unroll
    for (int i = 0; i < MU; i++) {
      const uint32_t u = u0 + wave + PASS_WAVES * i;
      const bool real = tv[j] && u < u1;
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
                                               const bool (&tv)[MT], uint32_t u0, uint32_t u1, uint32_t wave,
                                               int lane) {
  if (Q8 && M.type == LLMHIP_Q8_0) units_load<LLMHIP_Q8_0, MT, MU>(W, M, tile, tv, u0, u1, wave, lane);
  else if (M.type == LLMHIP_Q4_1) units_load<LLMHIP_Q4_1, MT, MU>(W, M, tile, tv, u0, u1, wave, lane);
  else units_load<LLMHIP_Q4_0, MT, MU>(W, M, tile, tv, u0, u1, wave, lane);
}

// A wave's units dequantised (B operands and block scales; m: Q4_1's block
// minima), ahead of the wait for the phase's input: after the wait only the
// MFMAs remain.
template <int MT, int MU>
struct UnitsB {
  h8 B[MT][MU][4];
  float d[MT][MU][4], m[MT][MU][4];
};

template <uint32_t QT, int MT, int MU>
__device__ __forceinline__ void units_deq(const WUnit (&W)[MT][MU], const PassMat& M, uint32_t u0, uint32_t wave,
                                          UnitsB<MT, MU>& ub) {
#pragma unroll
  for (int i = 0; i < MU; i++) {
    const uint32_t u = u0 + wave + PASS_WAVES * i;
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        ub.B[t][i][j] = h8{};
        ub.d[t][i][j] = ub.m[t][i][j] = 0.f;
        if (u < M.ng) unit_block<QT, false>(W[t][i], j, ub.B[t][i][j], ub.d[t][i][j], ub.m[t][i][j]);
        else if (j < 3) unit_block<QT, true>(W[t][i], j, ub.B[t][i][j], ub.d[t][i][j], ub.m[t][i][j]);
      }
  }
}

template <bool Q8, int MT, int MU>
__device__ __forceinline__ void units_deq_any(const WUnit (&W)[MT][MU], const PassMat& M, uint32_t u0, uint32_t wave,
                                              UnitsB<MT, MU>& ub) {
  if (Q8 && M.type == LLMHIP_Q8_0) units_deq<LLMHIP_Q8_0, MT, MU>(W, M, u0, wave, ub);
  else if (M.type == LLMHIP_Q4_1) units_deq<LLMHIP_Q4_1, MT, MU>(W, M, u0, wave, ub);
  else units_deq<LLMHIP_Q4_0, MT, MU>(W, M, u0, wave, ub);
}

// A wave's products for the workgroup's tiles from the staged operands (block
// b of the matrix at staged block b - 4 u0): its units of units_load, ub.B[j][i]
// of tile j.  acc[j]: lanes of q == 0 hold row r's sum times 2^ex
// (d (hi + lo) . w per block, + m s_x for Q4_1, added block by block).  Every
// A operand is read before the first MFMA and the MFMAs issue back to back
// (a block outside the wave's units reads staged block 0 and adds nothing).
template <uint32_t QT, int MT, int MU>
__device__ __forceinline__ void units_mac(const UnitsB<MT, MU>& ub, const PassMat& M, const h8* xs,
                                          const float* bsum, uint32_t u0, uint32_t u1, uint32_t wave, int lane,
                                          float (&acc)[MT]) {
  typedef uint32_t u4v __attribute__((ext_vector_type(4)));
  const int q = lane >> 4, slot = lane & 15;
  const u4v keep = slot < 2 ? ~0u : 0u;
  h8 A[MU][4];
  float bs[MU][4];
  bool on[MU][4];
#pragma unroll
  for (int i = 0; i < MU; i++) {
    const uint32_t u = u0 + wave + PASS_WAVES * i;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      on[i][j] = u < u1 && (u < M.ng || j < (int)M.tail);
      const uint32_t b = on[i][j] ? 4 * (u - u0) + j : 0;
      A[i][j] = __builtin_bit_cast(h8, __builtin_bit_cast(u4v, xs[(b * 4 + q) * 2 + min(slot, 1)]) & keep);
      bs[i][j] = QT == LLMHIP_Q4_1 ? bsum[b] : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < MU; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int t = 0; t < MT; t++) {
        const f4 D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i][j], ub.B[t][i][j], f4{0, 0, 0, 0}, 0, 0, 0);
        if (on[i][j]) {
          acc[t] += ub.d[t][i][j] * (D[0] + D[1]);
          if (QT == LLMHIP_Q4_1) acc[t] += ub.m[t][i][j] * bs[i][j];
        }
      }
}

template <bool Q8, int MT, int MU>
__device__ __forceinline__ void units_mac_any(const UnitsB<MT, MU>& ub, const PassMat& M, const h8* xs,
                                              const float* bsum, uint32_t u0, uint32_t u1, uint32_t wave, int lane,
                                              float (&acc)[MT]) {
  if (Q8 && M.type == LLMHIP_Q8_0) units_mac<LLMHIP_Q8_0, MT, MU>(ub, M, xs, bsum, u0, u1, wave, lane, acc);
  else if (M.type == LLMHIP_Q4_1) units_mac<LLMHIP_Q4_1, MT, MU>(ub, M, xs, bsum, u0, u1, wave, lane, acc);
  else units_mac<LLMHIP_Q4_0, MT, MU>(ub, M, xs, bsum, u0, u1, wave, lane, acc);
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

typedef const __attribute__((address_space(4))) PassMat CMat;
// A matrix of the layer table (written by the host before the launch), field
// by field: scalar loads, which do not wait behind the vector loads in flight.
__device__ __forceinline__ PassMat cmat(CMat* c) {
  PassMat m;
  m.qs = c->qs;
  m.type = c->type;
  m.rows = c->rows;
  m.nb = c->nb;
  m.ng = c->ng;
  m.tail = c->tail;
  m.tiles = c->tiles;
  m.map = c->map;
  m.map_hd = c->map_hd;
  m.map_seg0 = c->map_seg0;
  m.map_seg1 = c->map_seg1;
  m.ff = c->ff;
  return m;
}

// LONG: positions past attn_full_max (the split attention's range): chunks
// of PASS_LONG_ROWS rows, one workgroup per (query head, chunk), the last
// chunk's workgroup merging the others.
template <uint32_t HD, bool KVH, bool Q8, bool LONG>
__global__ __launch_bounds__(512) void pass_kernel(PassArgs a) {
  static_assert(!LONG || HD == 64, "the long form holds 256 rows of a 64-wide head per workgroup");
  constexpr uint32_t RC = LONG ? PASS_LONG_ROWS : PASS_CHUNK_ROWS;  // cache rows of a chunk
  constexpr uint32_t V4 = HD / 64, S = 4 * PASS_WAVES, JC = RC / S;
  typedef AttnChunk<HD, JC, PASS_WAVES, KVH> AC;
  __shared__ PassLds<HD> L;
  const uint32_t wg = blockIdx.x, G = gridDim.x;
  const uint32_t E = a.embd, nq = a.embd, nk = a.kvd, hp = HD / 2;
  const uint32_t pos = state_pos(a.state);
  const uint32_t epoch = *(const __attribute__((address_space(4))) uint32_t*)a.ctrl;
  Waiter wt{a.ctrl + 1, a.ctrl[2] ? a.ctrl[2] : PASS_SPIN_DEFAULT, false};
  const uint32_t NCH = pass_chunks(HD), P = pos / RC + 1;  // chunks; those holding rows 0 .. pos
// The thread's indices, redefined at each phase's start: per-lane offsets
// formed from them stay inside the phase (hoisted out of the layer loop, every
// phase's would hold registers through all the others).
#define PHASE_IDS                                      \
  uint32_t tid = threadIdx.x, wave = wave_id();        \
  asm volatile("" : "+v"(tid), "+s"(wave));            \
  const uint32_t lane = tid & 63;                      \
  const int r = lane & 15, q = lane >> 4;              \
  (void)r;                                             \
  (void)q

  // this workgroup's share (the same for every layer)
  const uint32_t T1 = (E + 2 * a.kvd + 15) / 16, T3 = (E + 15) / 16, T5 = (E + 15) / 16;
  const bool has1 = wg >= a.b1 && wg - a.b1 < T1, has3 = wg >= a.b3 && wg - a.b3 < T3,
             has5 = wg >= a.b5 && wg - a.b5 < a.kp * T5;
  const uint32_t t1 = has1 ? wg - a.b1 : 0, t3 = has3 ? wg - a.b3 : 0;
  const uint32_t t5 = has5 ? (wg - a.b5) % T5 : 0, p5 = has5 ? (wg - a.b5) / T5 : 0;  // K5 tile and part
  const uint32_t GQ = a.heads / a.kv_heads, natt1 = 8 * GQ * ((a.kv_heads + 7) / 8);
  bool hasA = false;
  uint32_t hg = 0, hh = 0, hc = 0;  // attention: KV head, query head, chunk
  if (LONG) {
    // (query head, chunk)s for the chunks of the rows this launch may read,
    // grouped by (chunk, KV head) pair p = c kv_heads + g: pair p's GQ query
    // heads on XCD p % 8 (workgroup w runs on XCD w % 8), so that the pair's
    // rows are read through one L2; XCD x's units (pairs x, x + 8, ..., GQ
    // each) on its workgroups from the grid's end down: unit k of XCD x on
    // workgroup G - 8 (k + 1) + x (G a multiple of 8: pass_long_fits)
    const uint32_t PM = (a.rows + RC - 1) / RC, x = wg % 8, k = (G + x - wg) / 8 - 1;
    const uint32_t p = x + 8 * (k / GQ);
    if (p < PM * a.kv_heads) {
      hc = p / a.kv_heads;
      hg = p % a.kv_heads;
      hh = hg * GQ + k % GQ;
      hasA = hc < P;
    }
  } else if (wg >= a.batt && wg - a.batt < NCH * natt1) {
    // head h = g GQ + s, chunk c on workgroup batt + c natt1 + 8 (GQ (g / 8) + s) + g % 8 (a KV head's
    // query heads on one XCD)
    const uint32_t rel0 = wg - a.batt, rel = rel0 % natt1, y = rel / 8;
    hc = rel0 / natt1;
    hg = (y / GQ) * 8 + rel % 8;
    hh = hg * GQ + y % GQ;
    hasA = hg < a.kv_heads && hc < P;  // a chunk past the position has nothing to do (K3 reads chunks < P)
  }
  const uint32_t rw4 = (wg + G - a.b4 % G) % G;
  typedef const __attribute__((address_space(4))) PassLayer CLayer;

  for (uint32_t l = 0; l < a.nlayers; l++) {
    CLayer* Y = (CLayer*)a.layers + l;
    const bool last = l + 1 == a.nlayers;
    const uint32_t F = epoch * a.nlayers + l + 1, Fp = F - 1;  // this layer's flag, the previous layer's
    // the flag-word pointers, redefined in every iteration: addresses formed
    // from them stay inside the iteration (hoisted out of the layer loop they
    // would hold registers through every phase)
    uint64_t *llb = a.llb, *llq = a.llq, *llo = a.llo, *llact = a.llact;
    asm volatile("" : "+s"(llb), "+s"(llq), "+s"(llo), "+s"(llact));
    // K3's and K4's weights, issued at the layer's start: a workgroup that
    // has K1 or K2 work first would otherwise start them after it, and they
    // would arrive inside the phase's wait
    WUnit w3[1][1], w4[PASS_K4_TILES][1];
    {
      PHASE_IDS;
      if (has3) {
        const PassMat M = cmat(&Y->o);
        const uint32_t tt3[1] = {min(t3, M.tiles - 1)};
        const bool v3[1] = {true};
        units_load_any<Q8, 1, 1>(w3, M, tt3, v3, 0, M.ng + (M.tail ? 1u : 0u), wave, lane);
      }
      const PassMat M = cmat(&Y->gu);
      if (rw4 < M.tiles) {
        uint32_t tt4[PASS_K4_TILES];
        bool v4[PASS_K4_TILES];
#pragma unroll
        for (uint32_t j = 0; j < PASS_K4_TILES; j++) {
          const uint32_t t = rw4 + G * j;
          v4[j] = t < M.tiles;
          tt4[j] = v4[j] ? t : 0;
        }
        units_load_any<Q8, PASS_K4_TILES, 1>(w4, M, tt4, v4, 0, M.ng + (M.tail ? 1u : 0u), wave, lane);
      }
    }

    // ---- K1: h = RMSNorm(x) attn_norm; [q; k; v] = W h (+ b); RoPE; K, V appended at pos
    if (has1) {
      PHASE_IDS;
      const PassMat M = cmat(&Y->qkv);
      const float* bias_p = Y->bias;
      float* kvp = Y->kv;
      WUnit w1[1][1];
      const uint32_t tt1[1] = {min(t1, M.tiles - 1)};
      const bool v1[1] = {true};
      const uint32_t U = M.ng + (M.tail ? 1u : 0u);
      units_load_any<Q8, 1, 1>(w1, M, tt1, v1, 0, U, wave, lane);
      // the epilogue's inputs, ahead of the wait: the lane's bias and RoPE table entries
      const uint32_t lr = row_of_pos(t1 * 16 + r, M.map, M.map_hd, M.map_seg0, M.map_seg1, M.ff);
      const bool rv = wave == 0 && q == 0 && lr < M.rows;
      float bias = 0, c = 0, sn = 0;
      const uint32_t j = lr < nq ? lr : lr - nq, w = j & (HD - 1);
      if (rv) {
        if (bias_p) bias = bias_p[lr];
        if (lr < nq + nk) {
          const uint32_t i = a.neox ? w & (hp - 1) : w / 2;
          const uint64_t co = ((uint64_t)pos * hp + i) * 2;
          c = a.cs[co];
          sn = a.cs[co + 1];
        }
      }
      StageIn in{};
      in.ll = llb;
      in.plain = a.xn;
      in.flag = Fp;
      in.gate = true;  // (this workgroup has waited since its K4 work)
      in.kp = a.kp;
      in.E = E;
      UnitsB<1, 1> ub;
      units_deq_any<Q8, 1, 1>(w1, M, 0, wave, ub);
      float* ss = L.ss[0][l & 1];
      const int ex = l ? stage_rms_wave<SRC_XSUM, 1>(L, in, M.nb, 0, U, Y->attn_norm, ss, wt, wave, lane)
                       : stage_rms_wave<SRC_PLAIN, 1>(L, in, M.nb, 0, U, Y->attn_norm, ss, wt, wave, lane);
      float acc[1] = {0};
      units_mac_any<Q8, 1, 1>(ub, M, L.xs, L.bsum, 0, U, wave, lane, acc);
      acc[0] = ldexpf(acc[0], -ex);
      float v = split_sum<1>(L.part1[l & 1], acc, wave, lane);
      if (wave == 0) {
        v = __fmul_rn(v, rms_of(ss, M.nb * 32, a.eps));
        if (bias_p && rv) v += bias;
        const float o = __shfl_xor(v, a.neox ? 8 : 1);
        if (rv) {
          if (lr < nq + nk) {
            const bool first = a.neox ? w < hp : (w % 2) == 0;
            const float x = first ? v : o, zz = first ? o : v;
            const float res = first ? __fsub_rn(__fmul_rn(x, c), __fmul_rn(zz, sn))   // cpu.go:381
                                    : __fadd_rn(__fmul_rn(x, sn), __fmul_rn(zz, c));  // cpu.go:382
            if (lr < nq) {
              ll_store(llq + lr, res, F);
              if (last) a.q[lr] = res;
            } else {
              const uint64_t ci = (uint64_t)pos * a.kvd + j;
              float kvv = res;
              if (KVH) {
                const _Float16 hv = to_f16(res);
                ((_Float16*)kvp)[ci] = hv;
                kvv = (float)hv;
              } else {
                kvp[ci] = res;
              }
              ll_store(llq + nq + j, kvv, F);
            }
          } else {
            const uint32_t jv = lr - nq - nk;
            const uint64_t ci = (uint64_t)a.ctx * a.kvd + (uint64_t)pos * a.kvd + jv;
            float kvv = v;
            if (KVH) {
              const _Float16 hv = to_f16(v);
              ((_Float16*)kvp)[ci] = hv;
              kvv = (float)hv;
            } else {
              kvp[ci] = v;
            }
            ll_store(llq + nq + nk + jv, kvv, F);
          }
        }
      }
    }

    // ---- K2: query head hh over chunk hc's rows (cpu.go:300-334): the rows of
    // earlier positions from the cache, the position's row from K1's words;
    // out the chunk's max score M, sum of e L and sum of e v (unnormalised)
    if (hasA) {
      PHASE_IDS;
      const uint32_t cl = tid & 15, slot = tid >> 4, row0 = hc * RC;
      const float* kvp = Y->kv;
      AC rows;
      {
        // 32-bit element offsets (the cache holds 2 ctx kvd < 2^31 elements)
        const uint32_t lim = max(pos, 1u), Jr = min(a.rows - min(a.rows, row0), RC) / S;
        const uint32_t kb = hg * HD + 4 * cl, vb = a.ctx * a.kvd + hg * HD + 4 * cl;
#pragma unroll
        for (uint32_t j = 0; j < JC; j++) {
          if (j >= Jr) break;
          const uint32_t p = min(row0 + slot + S * j, lim - 1) * a.kvd;
#pragma unroll
          for (uint32_t v = 0; v < V4; v++) {
            rows.kr[j][v] = kv_load4<KVH>(kvp, kb + p + 64 * v);
            rows.vr[j][v] = kv_load4<KVH>(kvp, vb + p + 64 * v);
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
      if (pos >= row0 && pos < row0 + RC && slot == (pos - row0) % S) {
        // this thread's rows hold the position's row: K1's words
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
        const uint32_t jp = (pos - row0) / S;
#pragma unroll
        for (uint32_t j = 0; j < JC; j++)
          if (j == jp)
#pragma unroll
            for (uint32_t k = 0; k < V4; k++) {
              rows.kr[j][k] = f4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
              rows.vr[j][k] = f4{v[4 * V4 + 4 * k], v[4 * V4 + 4 * k + 1], v[4 * V4 + 4 * k + 2],
                                 v[4 * V4 + 4 * k + 3]};
            }
      }
      float M_, L_, o;
      rows.reduce(qv, row0, pos + 1, a.scale, L.am, &M_, &L_, &o);
      // llo: the partial sums of chunks c < P - 1 (o at c E, m and l in a
      // whole line of 16 words at np E + 16 (c heads + h), m at even words and
      // l at odd: a store of part of a line has been seen to reach other XCDs
      // later), then the output row
      uint64_t* fin = llo + a.np * (E + 16 * a.heads);
      if (P == 1) {
        // one chunk: its sums normalised (a one-chunk merge: M = m, weight 1)
        if (tid < HD) {
          const float r = o / L_;
          ll_store(fin + hh * HD + tid, r, F);
          if (last) a.att[hh * HD + tid] = r;
        }
      } else if (hc + 1 < P) {
        if (tid < HD) ll_store(llo + hc * E + hh * HD + tid, o, F);
        if (tid < 16) ll_store(llo + a.np * E + 16 * (hc * a.heads + hh) + tid, tid & 1 ? L_ : M_, F);
      } else if (!LONG) {
        // the second chunk merges the first's sums and its own as
        // attn_merge_kernel merges chunks (layer.hip): M, then the weights, L
        // and o, then o / L
        if (tid < HD) {
          float v[3];  // chunk 0's o, m, l
          ll_wait_f<3>([&](int i) { return i == 0 ? llo + hh * HD + tid : llo + a.np * E + 16 * hh + (i - 1); },
                       [](int) { return true; }, F, v, wt);
          const float Mx = fmaxf(fmaxf(-INFINITY, v[1]), M_);
          const float w0 = __expf(v[1] - Mx), w1 = __expf(M_ - Mx);
          float Ls = 0, oo = 0;
          Ls += w0 * v[2];
          Ls += w1 * L_;
          oo += w0 * v[0];
          oo += w1 * o;
          const float r = oo / Ls;
          ll_store(fin + hh * HD + tid, r, F);
          if (last) a.att[hh * HD + tid] = r;
        }
      } else {
        // the last chunk merges the others' sums and its own, as above in
        // chunk order; wave w polls chunks w and w + 8 into LDS
        const uint32_t lane = tid & 63;
        float v[6];  // chunk wave + 8 i: o, m, l at 3 i
        ll_wait_f<6>(
            [&](int i) {
              const uint32_t c = wave + PASS_WAVES * (i / 3), k = i % 3;
              return k == 0 ? llo + c * E + hh * HD + lane : llo + a.np * E + 16 * (c * a.heads + hh) + (k - 1);
            },
            [&](int i) { return wave + PASS_WAVES * (i / 3) + 1 < P; }, F, v, wt);
#pragma unroll
        for (uint32_t i = 0; i < 2; i++) {
          const uint32_t c = wave + PASS_WAVES * i;
          if (c + 1 < P) {
            L.mrg[c][lane] = v[3 * i];
            if (lane == 0) {
              L.mrg[c][HD] = v[3 * i + 1];
              L.mrg[c][HD + 1] = v[3 * i + 2];
            }
          }
        }
        __syncthreads();
        if (tid < HD) {
          float Mx = -INFINITY;
          for (uint32_t c = 0; c + 1 < P; c++) Mx = fmaxf(Mx, L.mrg[c][HD]);
          Mx = fmaxf(Mx, M_);
          float Ls = 0, oo = 0;
          for (uint32_t c = 0; c + 1 < P; c++) {
            const float w = __expf(L.mrg[c][HD] - Mx);
            Ls += w * L.mrg[c][HD + 1];
            oo += w * L.mrg[c][tid];
          }
          const float w = __expf(M_ - Mx);
          Ls += w * L_;
          oo += w * o;
          const float r = oo / Ls;
          ll_store(fin + hh * HD + tid, r, F);
          if (last) a.att[hh * HD + tid] = r;
        }
      }
    }

    // ---- K3: x + W_o att, att merged from the chunks
    if (has3) {
      PHASE_IDS;
      const PassMat M = cmat(&Y->o);
      const uint32_t U = M.ng + (M.tail ? 1u : 0u);
      // the residual row (x before this layer: layer 0's input, or the
      // previous layer's attention residual plus its down projection's parts),
      // ahead of the wait
      const uint32_t lr = t3 * 16 + r;
      const bool rv = wave == 0 && q == 0 && lr < M.rows;
      uint64_t r0[1 + PASS_MAX_KP] = {};
      float resf = 0;
      if (rv) {
        if (l == 0) {
          resf = a.xn[lr];
        } else {
#pragma unroll
          for (uint32_t p = 0; p <= PASS_MAX_KP; p++)
            if (p <= a.kp) r0[p] = ll_load(llb + p * E + lr);
        }
      }
      StageIn in{};
      in.ll = llo + a.np * (E + 16 * a.heads);
      in.flag = F;
      in.gate = true;
      UnitsB<1, 1> ub;
      units_deq_any<Q8, 1, 1>(w3, M, 0, wave, ub);
      const int ex = stage_wave<1, false>(L, in, 0, M.nb, 0, U, wt, wave, lane);
      float acc[1] = {0};
      units_mac_any<Q8, 1, 1>(ub, M, L.xs, L.bsum, 0, U, wave, lane, acc);
      acc[0] = ldexpf(acc[0], -ex);
      const float v = split_sum<1>(L.part2, acc, wave, lane);
      if (rv) {
        float res = resf;
        if (l != 0) {
          res = ll_settle(llb + lr, r0[0], Fp, wt);
#pragma unroll
          for (uint32_t p = 1; p <= PASS_MAX_KP; p++)
            if (p <= a.kp) res += ll_settle(llb + p * E + lr, r0[p], Fp, wt);
        }
        ll_store(llb + lr, res + v, F);
      }
    }

    // ---- K4: h = RMSNorm(x) ffn_norm; act = silu(W_gate h) * (W_up h).
    // K5's weights are issued here too (its workgroups take part in K4).
    WUnit w5[1][PASS_K5_UNITS];
    uint32_t u50 = 0, u51 = 0;  // K5: this part's units
    {
      const PassMat D = cmat(&Y->down);
      const uint32_t U5 = D.ng + (D.tail ? 1u : 0u);
      u50 = p5 * U5 / a.kp;
      u51 = (p5 + 1) * U5 / a.kp;
    }
    {
      const PassMat M = cmat(&Y->gu);
      if (rw4 < M.tiles) {
        PHASE_IDS;
        const uint32_t U = M.ng + (M.tail ? 1u : 0u);
        if (has5) {
          const PassMat D = cmat(&Y->down);
          const uint32_t tt5[1] = {min(t5, D.tiles - 1)};
          const bool v5[1] = {true};
          units_load_any<Q8, 1, PASS_K5_UNITS>(w5, D, tt5, v5, u50, u51, wave, lane);
        }
        StageIn in{};
        in.ll = llb;
        in.flag = F;
        in.gate = !has3;  // K3's workgroups come straight from producing this input
        UnitsB<PASS_K4_TILES, 1> ub;
        units_deq_any<Q8, PASS_K4_TILES, 1>(w4, M, 0, wave, ub);
        float* ss = L.ss[1][l & 1];
        const int ex = stage_rms_wave<SRC_LL, 1>(L, in, M.nb, 0, U, Y->ffn_norm, ss, wt, wave, lane);
        float acc[PASS_K4_TILES] = {};
        units_mac_any<Q8, PASS_K4_TILES, 1>(ub, M, L.xs, L.bsum, 0, U, wave, lane, acc);
#pragma unroll
        for (uint32_t t = 0; t < PASS_K4_TILES; t++) acc[t] = ldexpf(acc[t], -ex);
        float v = split_sum<PASS_K4_TILES>(L.part4[l & 1], acc, wave, lane);
        const uint32_t tile = rw4 + G * wave;
        if (wave < PASS_K4_TILES && tile < M.tiles) {
          v = __fmul_rn(v, rms_of(ss, M.nb * 32, a.eps));
          // gate row i at lane r < 8, up row i at r + 8 (MAP_GATEUP)
          const float u = __shfl_xor(v, 8);
          const uint32_t i = 8 * tile + (r & 7);
          if (q == 0) {
            // the tile's 8 activations and, as padding, its 8 up rows: one
            // whole line of 16 words (pass_act_words)
            const float act = r < 8 ? v / (1.f + __expf(-v)) * u : v;  // cpu.go:345
            ll_store(llact + 16 * tile + r, act, F);
            if (last && i < a.ff) {
              if (r < 8) a.act[i] = act;
              else a.up[i] = v;
            }
          }
        }
      } else if (has5) {
        PHASE_IDS;
        const PassMat D = cmat(&Y->down);
        const uint32_t tt5[1] = {min(t5, D.tiles - 1)};
        const bool v5[1] = {true};
        units_load_any<Q8, 1, PASS_K5_UNITS>(w5, D, tt5, v5, u50, u51, wave, lane);
      }
    }

    // ---- K5: part p5 of W_down act (its k-range of units [u50, u51)); the
    // next layer (or the last step) adds the parts to the residual
    if (has5) {
      PHASE_IDS;
      const PassMat M = cmat(&Y->down);
      StageIn in{};
      in.ll = llact;  // (8 of every 16 words: pass_act_words)
      in.flag = F;
      in.gate = false;  // every K5 workgroup comes straight from its K4 work
      const uint32_t nb0 = 4 * u50, nbp = min(4 * u51, M.nb) - nb0;
      UnitsB<1, PASS_K5_UNITS> ub;
      units_deq_any<Q8, 1, PASS_K5_UNITS>(w5, M, u50, wave, ub);
      const int ex = stage_wave<PASS_K5_UNITS, true>(L, in, nb0, nbp, u50, u51, wt, wave, lane);
      float acc[1] = {0};
      units_mac_any<Q8, 1, PASS_K5_UNITS>(ub, M, L.xs, L.bsum, u50, u51, wave, lane, acc);
      acc[0] = ldexpf(acc[0], -ex);
      const float v = split_sum<1>(L.part2, acc, wave, lane);
      const uint32_t lr = t5 * 16 + r;
      if (wave == 0 && q == 0 && lr < M.rows) ll_store(llb + (1 + p5) * E + lr, v, F);
    }
  }

  // ---- the pass's output row: x = the last layer's residual plus its down
  // projection's parts (the head's input, Peek("x"))
  if (wg < T3) {
    PHASE_IDS;
    const uint32_t lr = wg * 16 + r, F = epoch * a.nlayers + a.nlayers;
    if (wave == 0 && q == 0 && lr < E) {
      uint64_t r0[1 + PASS_MAX_KP] = {};
#pragma unroll
      for (uint32_t p = 0; p <= PASS_MAX_KP; p++)
        if (p <= a.kp) r0[p] = ll_load(a.llb + p * E + lr);
      float x = ll_settle(a.llb + lr, r0[0], F, wt);
#pragma unroll
      for (uint32_t p = 1; p <= PASS_MAX_KP; p++)
        if (p <= a.kp) x += ll_settle(a.llb + p * E + lr, r0[p], F, wt);
      a.x[lr] = x;
    }
  }
}

#undef PHASE_IDS

// ------------------------------------------------------------------ host

const char* pass_unfit(const llmhip_config& c, uint32_t kvd, const PassMat& qkv, const PassMat& o, const PassMat& gu,
                       const PassMat& down, uint32_t grid, uint32_t* kp) {
  if (grid == 0) return "no co-resident grid";
  if (c.head_dim != 64 && c.head_dim != 128) return "head size";
  if ((uint32_t)c.embd > PASS_MAX_EMBD) return "embedding above the staged row";
  if ((uint32_t)c.ff > PASS_MAX_FF) return "feed-forward above the staged row";
  const uint32_t E = (uint32_t)c.embd, GQ = (uint32_t)(c.heads / c.kv_heads);
  const uint32_t T5 = (E + 15) / 16;
  if ((E + 2 * kvd + 15) / 16 > grid || T5 > grid) return "more tiles than workgroups";
  if (pass_chunks((uint32_t)c.head_dim) * 8 * GQ * ((uint32_t)(c.kv_heads + 7) / 8) > grid)
    return "more heads than workgroups";
  auto units = [](const PassMat& m) { return m.ng + (m.tail ? 1u : 0u); };
  if (units(qkv) > PASS_WAVES || units(o) > PASS_WAVES || units(gu) > PASS_WAVES)
    return "more units per tile than waves";
  // k-parts: the fewest that leave each wave of a part one unit, else the
  // most the grid holds (more parts: fewer products per workgroup, more
  // vectors for the next layer to add)
  *kp = 0;
  for (uint32_t k = 1; k <= PASS_MAX_KP; k *= 2) {
    const uint32_t per = (units(down) + k - 1) / k;
    if (k * T5 > grid || per > PASS_WAVES * PASS_K5_UNITS || units(down) < k) continue;
    *kp = k;
    if (per <= PASS_WAVES) break;
  }
  if (*kp == 0) return "down projection too long";
  if (gu.tiles > PASS_K4_TILES * grid) return "gate/up too tall";
  if (gu.map != MAP_GATEUP || o.map != MAP_IDENT || down.map != MAP_IDENT) return "row maps";
  if (qkv.rows != E + 2 * kvd || o.rows != E || down.rows != E || gu.rows != 2 * (uint32_t)c.ff) return "shapes";
  return nullptr;
}

template <uint32_t HD, bool KVH, bool Q8, bool LONG>
static int occupancy() {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, pass_kernel<HD, KVH, Q8, LONG>, 64 * PASS_WAVES, 0) !=
      hipSuccess)
    return 0;
  return n;
}

template <uint32_t HD, bool KVH>
static uint32_t grid_of(int device) {
  // (the forms hold different registers: the least occupancy bounds them all)
  int n = std::min(occupancy<HD, KVH, false, false>(), occupancy<HD, KVH, true, false>());
  if (HD == 64) n = std::min({n, occupancy<64, KVH, false, true>(), occupancy<64, KVH, true, true>()});
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
  return n >= 1 && cus > 0 ? (uint32_t)cus : 0;
}

uint32_t pass_grid(int device, uint32_t hd, bool kv16) {
  if (hd == 64) return kv16 ? grid_of<64, true>(device) : grid_of<64, false>(device);
  if (hd == 128) return kv16 ? grid_of<128, true>(device) : grid_of<128, false>(device);
  return 0;
}

// K1's tiles from workgroup 0, the attention's (head, chunk)s after them
// (from a multiple of 8: a KV head's query heads on one XCD), K3's tiles
// after those where they fit, K5's (tile, part)s at the end, K4 round robin
// over the whole grid.  Where the grid is too small for disjoint ranges they
// overlap (the phases run in turn).
void pass_place(PassArgs* a, uint32_t grid, uint32_t t1, uint32_t t3, uint32_t t5) {
  const uint32_t natt = pass_chunks(a->hd) * 8 * (a->heads / a->kv_heads) * ((a->kv_heads + 7) / 8);
  a->b1 = 0;
  a->batt = (t1 + 7) / 8 * 8;
  if (a->batt + natt > grid) a->batt = 0;
  a->b5 = grid - a->kp * t5;
  const uint32_t e = std::max(t1, a->batt + natt);
  a->b3 = e + t3 <= a->b5 ? e : 0;
  a->b4 = 0;
}

template <uint32_t HD, bool KVH, bool LONG>
static void go(const PassArgs& a, uint32_t grid, bool q8, hipStream_t s) {
  if (q8) hipLaunchKernelGGL((pass_kernel<HD, KVH, true, LONG>), dim3(grid), dim3(64 * PASS_WAVES), 0, s, a);
  else hipLaunchKernelGGL((pass_kernel<HD, KVH, false, LONG>), dim3(grid), dim3(64 * PASS_WAVES), 0, s, a);
}

int pass_launch(const PassArgs& a, uint32_t grid, bool q8, bool lng, hipStream_t s) {
  if (lng && a.hd != 64) return set_error(LLMHIP_ERR_ARG, "llm: decode pass: long form at head size %u", a.hd);
  if (a.hd == 64) {
    if (lng) {
      if (a.kv16) go<64, true, true>(a, grid, q8, s);
      else go<64, false, true>(a, grid, q8, s);
    } else {
      if (a.kv16) go<64, true, false>(a, grid, q8, s);
      else go<64, false, false>(a, grid, q8, s);
    }
  } else if (a.hd == 128) {
    if (a.kv16) go<128, true, false>(a, grid, q8, s);
    else go<128, false, false>(a, grid, q8, s);
  } else {
    return set_error(LLMHIP_ERR_ARG, "llm: decode pass: head size %u", a.hd);
  }
  LLM_HIP(hipGetLastError());
  return 0;
}

}  // namespace llmhip
