// Host-side interface of the non-matrix kernels (layer.hip).
#pragma once

#include "common.h"
#include "gemv.h"
#include "wave.h"

namespace llmhip {

struct AttnArgs {
  const float* q;   // [ntok][heads*hd], RoPE applied
  const float* kv;  // this layer's cache [2][ctx][kvd]
  float* pv;        // split: [ntok][heads][smax][hd] chunk sums of e*v
  float* ml;        // split: [ntok][heads][smax][2] chunk max and sum of e
  float* att;       // [ntok][heads*hd] attention output
  const uint32_t* state;
  uint32_t heads, kv_heads, hd, kvd, ctx;
  uint32_t smax;   // chunk slots of pv/ml per (token, head)
  uint32_t rows;   // cache rows read: > every position of the pass, <= ctx
  uint32_t split;  // 0: one chunk (rows <= attn_full_max(hd)); 1: chunks (ATTN_SPLIT_ROWS; one token ATTN_DECODE_ROWS) + merge
  uint32_t kv16;   // the cache holds binary16 values (F16KV)
  float scale;     // f32(1/sqrt(hd)), cpu.go:304
  // attn_kernel's divisors (heads / kv_heads, ntok * kv_heads, kv_heads), set by attn_launch
  FastDiv dgq, dni, dkv;
};

// Prefill: att also written as the output projection's prepared operands (per
// 32-element block of a token: exponent-scaled f16 hi/lo in the product's
// operand order, xdx = 2^-e, xbsum = the block sum, xexp = 0); xp null: not.
struct AttnOps {
  void* xp;
  float* xdx;
  float* xbsum;
  int32_t* xexp;
  uint32_t onb;  // blocks per token row (heads * hd / 32)
};

// Rows per chunk of the split attention: several tokens (the matrix-core
// prefill form stages a chunk in LDS), and one token (twice the rows: half the
// partials for the merge; measured 7.3 against 8.2 us at 2560 positions).
constexpr uint32_t ATTN_SPLIT_ROWS = 128;
constexpr uint32_t ATTN_DECODE_ROWS = 256;

// Head sizes with an attention kernel.
bool attn_ok(uint32_t hd);
// Positions the one-chunk kernel covers.
uint32_t attn_full_max(uint32_t hd);
// One launch (one chunk), or two (chunks, merge).  Every position of the pass
// (state[0] .. state[0] + ntok - 1) must be below a.rows.  merge false (one
// token, chunks): the merge is left to the output projection's prologue
// (PRO_MERGE).
int attn_launch(const AttnArgs& a, uint32_t ntok, hipStream_t s, const AttnOps* ops = nullptr, bool merge = true);
// Greedy sampling from the head's per-workgroup partials, the token written
// to tokens[step + adv] and out[0], the state advanced by adv; with embd and
// xn also the sampled token's embedding row into xn (the input of the next
// one-token pass, which then runs no embedding kernel); with epoch, epoch[0]
// advanced by one (the fused decode pass's flags, pass.h).
int argmax_launch(const float* pv, const uint32_t* pi, uint32_t n, const float* logits, int32_t* tokens,
                  int32_t* outb, uint32_t* state, uint32_t adv, hipStream_t s, const QMat* embd = nullptr,
                  float* xn = nullptr, uint32_t* epoch = nullptr);
int advance_launch(uint32_t* state, uint32_t n, hipStream_t s);
// state = (p, p) (a prefill chunk on a lane of its own).
int set_state_launch(uint32_t* state, uint32_t p, hipStream_t s);
// out[i] = x[i] * s * w[i], s = f32(1/sqrt(f64(sum x^2 / n + eps))) (rmsNorm, cpu.go:81-98), one
// workgroup; n <= 16384.  Not on the forward pass (the matrix kernels fuse it): Peek("h").
int rmsnorm_launch(const float* x, const float* w, uint32_t n, float eps, float* out, hipStream_t s);

}  // namespace llmhip
