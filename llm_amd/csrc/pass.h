// Host-side interface of the fused decode pass (pass.hip): every layer of a
// one-token pass in one persistent launch.
#pragma once

#include "common.h"
#include "gemv.h"

namespace llmhip {

// One layer matrix as the pass reads it (the fields of QMat it needs).
struct PassMat {
  const uint8_t* qs;
  uint32_t type, rows, nb, ng, tail, tiles;
  uint32_t map, map_hd, map_seg0, map_seg1, ff;
};

// One layer: the fused [q; k; v] and [gate; up] matrices, the output and
// down projections, the norm weights, the QKV biases (or null) and the cache.
struct PassLayer {
  PassMat qkv, o, gu, down;
  const float *attn_norm, *ffn_norm, *bias;
  float* kv;
};

// The vectors that cross from one phase to the next inside the launch are
// 64-bit words (f32 bits low, flag high), written and read with agent-scope
// relaxed atomics, so that a word's value and flag arrive together on any
// XCD.  A reader polls until every word it needs carries the flag of the
// current (pass, layer): epoch * layers + layer + 1, where the epoch (ctrl[0])
// is advanced by the sampling kernel after every head pass, so no flag of an
// earlier pass matches.  A wait gives up after ctrl[2] polls (0: the default),
// counts itself in ctrl[1] and stops waiting, so every wave of the launch
// still ends.
struct PassArgs {
  const PassLayer* layers;  // device memory, nlayers entries
  uint32_t nlayers;
  const float* xn;                // layer 0's input row (the sampling kernel wrote it)
  float *x, *q, *att, *act, *up;  // the last layer's values, stored plainly (the head's input, Peek)
  uint64_t* llq;    // [E + 2 kvd]: q, and the position's K and V rows (K1)
  uint64_t* llo;    // [np][E] the attention chunks' sums of e v (all but the last chunk), [np][heads][16]
                    // their max scores and sums of e (m, l, m, l, ...), then [E] the attention's output (K2)
  uint64_t* llb;    // [1 + kp][E]: x after the attention (K3), then the down projection's k-parts (K5);
                    // x after the layer is their sum
  uint64_t* llact;  // [pass_act_words(ff)]: the SwiGLU activations (K4), 8 in every 16 words
  uint32_t* ctrl;   // [0] epoch, [1] timed-out waits, [2] poll limit
  const uint32_t* state;
  const float* cs;  // RoPE table
  uint32_t embd, ff, heads, kv_heads, hd, kvd, ctx, neox, kv16;
  uint32_t rows;  // cache rows the attention reads: a multiple of 64 above the position, <= attn_full_max
  uint32_t kp;    // k-parts of the down projection (1 or 2)
  uint32_t np;    // chunks with partial sums in llo, at most (the chunks of the longest position, less one)
  float eps, scale;
  // the first workgroup of each phase's work: K1 tiles, attention (head, chunk)s, K3 tiles, K4 (round robin),
  // K5 (tile, part)s
  uint32_t b1, batt, b3, b4, b5;
};

constexpr uint32_t PASS_WAVES = 8;        // waves per workgroup
constexpr uint32_t PASS_MAX_EMBD = 1024;  // the embedding, at most
constexpr uint32_t PASS_MAX_FF = 6144;    // the feed-forward width, at most (its row is staged in LDS)
constexpr uint32_t PASS_K4_TILES = 3;     // gate/up tiles per workgroup, at most
constexpr uint32_t PASS_K5_UNITS = 3;     // down-projection units (groups of four blocks) per wave and part, at most
constexpr uint32_t PASS_MAX_KP = 2;       // k-parts of the down projection, at most
constexpr uint32_t PASS_CHUNK_ROWS = 128; // cache rows of an attention chunk (two chunks at head size 64)
constexpr uint32_t PASS_LONG_ROWS = 256;  // cache rows of a chunk past attn_full_max (head size 64)
constexpr uint32_t PASS_LONG_CHUNKS = 16; // chunks of a head past attn_full_max, at most
constexpr uint32_t PASS_SPIN_DEFAULT = 1u << 20;

// Attention chunks of a pass at head size hd (the one-chunk range: 256 rows at 64, 128 at 128).
__host__ __device__ inline uint32_t pass_chunks(uint32_t hd) { return hd == 64 ? 2 : 1; }
// Chunks with partial sums (PassArgs::np) for a cache of ctx rows.
inline uint32_t pass_partials(const llmhip_config& c, uint32_t ctx) {
  if (c.head_dim != 64 || ctx <= 256) return 1;
  return std::min((ctx + PASS_LONG_ROWS - 1) / PASS_LONG_ROWS, PASS_LONG_CHUNKS) - 1;
}
// Words of the activations (PassArgs::llact): each gate/up tile's 8 in a line
// of 16 words, whose other 8 carry the tile's up rows, so that every store of
// the phase covers a whole line.
inline uint64_t pass_act_words(uint64_t ff) { return 16 * ((ff + 7) / 8); }
// Flag-carrying words a model's pass needs (PassArgs: llq, llo with np
// chunks' partial sums, llb with the most k-parts, llact).
inline uint64_t pass_words(const llmhip_config& c, uint32_t kvd, uint32_t np) {
  const uint64_t E = (uint64_t)c.embd;
  return E + 2ull * kvd + np * (E + 16ull * (uint64_t)c.heads) + E + (1 + PASS_MAX_KP) * E + pass_act_words((uint64_t)c.ff);
}
// Whether a launch whose attention reads `rows` cache rows past
// attn_full_max fits the long form on `grid` workgroups (head size 64, a
// workgroup per query head and chunk; the query heads of a (chunk, KV head)
// pair on one XCD, the pairs dealt to the 8 XCDs in turn, each XCD's units on
// its workgroups from the grid's end down).
inline bool pass_long_fits(const llmhip_config& c, uint32_t rows, uint32_t grid) {
  const uint32_t pm = (rows + PASS_LONG_ROWS - 1) / PASS_LONG_ROWS;
  const uint64_t pairs = (uint64_t)pm * (uint32_t)c.kv_heads, gq = (uint32_t)(c.heads / c.kv_heads);
  return c.head_dim == 64 && pm <= PASS_LONG_CHUNKS && grid % 8 == 0 && 8 * ((pairs + 7) / 8) * gq <= grid;
}
// Why a model's decode passes cannot take the fused launch (nullptr: they can),
// for `grid` co-resident workgroups; *kp receives the down projection's k-parts.
const char* pass_unfit(const llmhip_config& c, uint32_t kvd, const PassMat& qkv, const PassMat& o, const PassMat& gu,
                       const PassMat& down, uint32_t grid, uint32_t* kp);
// Workgroups that are all resident at once for the pass kernel of head size
// hd (0: none; the launch needs every workgroup resident).
uint32_t pass_grid(int device, uint32_t hd, bool kv16);
// The work placement of a grid (PassArgs::b*); t1, t3, t5: tiles of [q; k; v], W_o and W_down.
void pass_place(PassArgs* a, uint32_t grid, uint32_t t1, uint32_t t3, uint32_t t5);
// q8: some layer matrix is Q8_0; lng: the long form (a.rows past attn_full_max, pass_long_fits).
int pass_launch(const PassArgs& a, uint32_t grid, bool q8, bool lng, hipStream_t s);

}  // namespace llmhip
