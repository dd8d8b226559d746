// Host-side interface of the non-matrix kernels (layer.hip).
#pragma once

#include "common.h"

namespace llmhip {

struct AttnArgs {
  const float* q;   // [ntok][heads*hd], RoPE applied
  const float* kv;  // this layer's cache [2][ctx][kvd]
  float* pv;        // [ntok][heads][smax][hd]
  float* ml;        // [ntok][heads][smax][2]
  const uint32_t* state;
  uint32_t heads, kv_heads, hd, kvd, ctx, smax, chunk;
  float scale;  // f32(1/sqrt(hd)), cpu.go:304
  float* att;     // attn_full_kernel output [ntok][heads*hd]
  uint32_t rows;  // attn_full_kernel: cache rows read (> every position of the pass)
};

// Positions the short-context attention kernel covers.
constexpr uint32_t ATTN_FULL_MAX = 256;

uint32_t attn_lds_bytes(uint32_t heads, uint32_t kv_heads, uint32_t hd, uint32_t chunk);
int attn_launch(const AttnArgs& a, uint32_t ntok, hipStream_t s);
bool attn_full_ok(uint32_t heads, uint32_t kv_heads, uint32_t hd);
uint32_t attn_full_rows(uint32_t last_pos);
// Every position of the pass (state[0] .. state[0] + ntok - 1) must be below a.rows.
int attn_full_launch(const AttnArgs& a, uint32_t ntok, hipStream_t s);
int argmax_launch(const float* pv, const uint32_t* pi, uint32_t n, const float* logits, int32_t* tokens,
                  int32_t* outb, uint32_t* state, uint32_t adv, hipStream_t s);
int advance_launch(uint32_t* state, uint32_t n, hipStream_t s);

}  // namespace llmhip
