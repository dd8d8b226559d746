// Internal helpers shared by the HIP sources: error reporting, HIP checks and
// the geometry of the tiled weight layout.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "errors.h"

namespace llmhip {

#define LLM_HIP(call)                                                                            \
  do {                                                                                           \
    hipError_t e_ = (call);                                                                      \
    if (e_ != hipSuccess)                                                                        \
      return ::llmhip::set_error(LLMHIP_ERR_DEVICE, "llm: %s failed: %s (%s:%d)", #call,         \
                                 hipGetErrorString(e_), __FILE__, __LINE__);                     \
  } while (0)

// ggml block geometry (gguf/gguf.go:72-92) for the types with kernels.
struct QType {
  uint32_t type;
  uint32_t block_bytes;  // GGUF bytes per 32 weights
  uint32_t qs_bytes;     // quant bytes per block in the tiled layout
  uint32_t sc_bytes;     // scale bytes per block (f16 d, plus f16 m for Q4_1)
  uint32_t qs_off;       // offset of the quants inside a GGUF block
};

inline bool qtype_of(uint32_t t, QType* q) {
  switch (t) {
    case LLMHIP_Q4_0: *q = {t, 18, 16, 2, 2}; return true;
    case LLMHIP_Q4_1: *q = {t, 20, 16, 4, 4}; return true;
    case LLMHIP_Q8_0: *q = {t, 34, 32, 2, 2}; return true;
  }
  return false;
}

// Geometry of a [rows][k] quantised matrix on the device: rows in tiles of 16
// (padded with zero rows), a row's nb = k/32 blocks in ng groups of four and
// a tail of nb % 4; each tile's quants then its scales (the byte layout is
// Lay in gemv_impl.h).  Device bytes equal GGUF bytes for rows % 16 == 0.
struct Geom {
  QType q;
  uint64_t rows, k;
  uint32_t nb, ng, tail;  // blocks per row, full groups, blocks in the tail group
  uint64_t tiles;
  uint64_t dev_bytes() const { return tiles * 16ull * nb * (q.qs_bytes + q.sc_bytes); }
  uint64_t gguf_bytes() const { return rows * nb * (uint64_t)q.block_bytes; }
};

inline Geom make_geom(const QType& q, uint64_t rows, uint64_t k) {
  Geom g;
  g.q = q;
  g.rows = rows;
  g.k = k;
  g.nb = (uint32_t)(k / 32);
  g.ng = g.nb / 4;
  g.tail = g.nb % 4;
  g.tiles = (rows + 15) / 16;
  return g;
}

}  // namespace llmhip
