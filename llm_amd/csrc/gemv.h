// Host-side interface of the quantised matrix kernels (gemv.hip) used by the
// model orchestration (model.cpp).
#pragma once

#include "common.h"

namespace llmhip {

// How logical rows of a matrix sit in the 16-row tiles.  A fused epilogue
// needs both rows of a pair in one tile: RoPE pairs and [gate; up] pairs.
enum RowMap : uint32_t {
  MAP_IDENT = 0,  // position = row
  MAP_NEOX = 1,   // inside each head of hd rows, row i and i+hd/2 land 8 lanes apart
  MAP_GATEUP = 2  // rows [0,ff) gate and [ff,2ff) up: gate i and up i land 8 lanes apart
};

// A quantised matrix in the tiled layout.
struct QMat {
  int device = 0;
  Geom g;
  uint8_t* qs = nullptr;  // device: the unit records (quants and scales)
  uint64_t bytes = 0;
  bool owned = false;     // qs from qmat_alloc (freed by qmat_release), not placed in a caller's memory
  // row map (RowMap): NEOX pairs rows inside heads of map_hd rows for rows
  // [map_seg0, map_seg1); GATEUP pairs row i with row ff + i.
  uint32_t map = MAP_IDENT, map_hd = 0, map_seg0 = 0, map_seg1 = 0, ff = 0;
};

enum Prologue : int {
  PRO_PLAIN = 0,  // x[t*ldx + e]
  PRO_RMS = 1,    // RMSNorm(x[t]) * nw  (cpu.go:81-98), recomputed per workgroup
  PRO_Q8 = 2,     // flag: the input then quantised to Q8_0 / Q8_1 blocks and the products formed
                  // as ggml's CPU backend forms them (the ExactGGML mode, cpu.go:117-140, 166-214)
  PRO_MERGE = 4,  // one token, f32: x[e] is the attention output of head e / hd, merged from the
                  // split attention's chunk partials (mpv, mml) as attn_merge_kernel merges them;
                  // the bits from PRO_MERGE_SHIFT up hold how many chunks (merge_pro)
};
// Flag (one token, with PRO_RMS): the input row is x + xpart[0] + xpart[xpartstride]
// (the residual and the two k-halves of the previous down projection, added in
// that order; kparts), and workgroup 0 stores that sum to xout.
constexpr int PRO_XSUM = 64;
// Chunks of partials the merging prologue combines: all of them loaded at
// once, an even count from 2 to MERGE_MAX_CHUNKS chosen per pass (the chunks
// its attention rows can have), so that no load waits for the position.
constexpr uint32_t MERGE_MAX_CHUNKS = 16;
constexpr int PRO_MERGE_SHIFT = 3;
constexpr int merge_pro(uint32_t chunks) { return PRO_MERGE | (int)(((chunks + 1) / 2 - 1) << PRO_MERGE_SHIFT); }
constexpr uint32_t merge_chunks(int pro) {
  return (pro & PRO_MERGE) ? 2 * (((uint32_t)pro >> PRO_MERGE_SHIFT) & 7) + 2 : 0;
}

enum Epilogue : int {
  EPI_STORE = 0,   // y[t*ldy + row] = v
  EPI_ACC = 1,     // y[t*ldy + row] += v           (residual add, K3 / K5)
  EPI_QKV = 2,     // + bias, RoPE on pairs, q out, K/V appended to the cache (K1)
  EPI_GATEUP = 3,  // act[t*ff + i] = silu(gate_i) * up_i                   (K4)
  EPI_ARGMAX = 4,  // STORE, and each workgroup's (max, index) of its rows    (head)
  EPI_SWIGLU = 5   // y[t*ldy + row] = silu(aux[t*ldy + row]) * v  (up, gate stored apart)
};


struct GemvArgs {
  // matrix
  const uint8_t* qs;
  uint32_t rows, nb, ng, tail, tiles, k;
  uint32_t map, map_hd, map_seg0, map_seg1;  // RowMap; NEOX applies to rows [seg0, seg1)
  uint32_t row_base;                         // QKV: first row of this matrix in [q; k; v]
  uint32_t ntok;                             // tokens in the launch
  uint32_t split;                            // waves sharing one tile (split-K): 1..16
  uint32_t waves;                            // waves per workgroup: 4, 8 or 16 (a multiple of split)
  uint32_t stream, swaves;                   // one token: workgroups and waves per workgroup of the
                                             // streaming kernel (large matrices), 0: tile kernel
  // prologue
  const float* x;
  uint32_t ldx;
  uint32_t xrow0;  // token t reads row xrow0 + t of x (head: the last token of a chunk)
  const float* nw;
  float eps;
  uint32_t heads, hd;  // QKV epilogue: RoPE per head
  const uint32_t* state;            // (pos, step) on the device
  // epilogue
  float* y;
  uint32_t ldy;
  const float* yin;  // EPI_ACC: the residual read (nullptr: y itself)
  const float* bias;  // QKV biases, logical row order (nullptr: none)
  const float* cs;    // RoPE table [pos][hd/2][cos, sin]
  float* kv;          // this layer's cache [2][ctx][kvd], f32 or (kv16) binary16
  uint32_t kv16;
  uint32_t nq, nk, kvd, ctx;
  uint32_t neox;
  uint32_t ff;
  float* amax_v;  // EPI_ARGMAX: per-workgroup partials
  uint32_t* amax_i;
  const float* aux;  // EPI_SWIGLU: the gate values
  float* up;         // EPI_GATEUP / EPI_SWIGLU: the up product u = W_up h also stored here, [t*ff + i]
                     // (nullptr: not kept); Peek("up")
  // one token, EPI_STORE: kparts (1 or 2) workgroups per tile group, part p summing block groups
  // [p ng / kparts, (p + 1) ng / kparts) (the tail with the last) into y + p * pstride
  uint32_t kparts, pstride;
  // PRO_XSUM: the partial rows added to x, and where workgroup 0 stores the sum
  const float* xpart;
  uint32_t xpartstride;
  float* xout;
  // PRO_MERGE: the split attention's partials ([heads][msmax][hd] sums of e*v, [heads][msmax][2]
  // max and sum of e) over chunks of mrows positions; the merged row also goes to matt (tile 0)
  const float* mpv;
  const float* mml;
  uint32_t msmax, mrows;
  float* matt;
  // prefill (gemm_kernel): activations prepared once per launch by prep_kernel
  void* xp;        // [tg][nb][2][64 lanes] 16-byte MFMA operands: group g, block b, part h (0: the f16 hi
                   // parts, 1: lo), lane l: token 16 g + l % 16, k-group l / 16 of the block
  int32_t* xexp;   // [tg*16] power-of-two scale per token
  float* xbsum;    // [tg*16][nb] scaled block sums (Q4_1); PRO_Q8: the Q8_1 sums s
  float* xdx;      // [tg*16][nb] PRO_Q8: the activation block scales d (binary16 values)
  uint32_t tg;     // token groups of 16
  uint32_t q8;     // the prepared activations are Q8 blocks (PRO_Q8): gemm_kernel's block products
  // EPI_GATEUP (gemm_kernel): the activations also as the down projection's
  // block-scaled operands (op_xp in the layout of xp, op_nb blocks per token;
  // per token and block op_dx = 2^-e, op_bsum = the block's sum; op_exp = 0),
  // so that no staging launch runs between the two products (null: not)
  void* op_xp;
  float *op_dx, *op_bsum;
  int32_t* op_exp;
  uint32_t op_nb;
};

// Bytes of the prepared-activation buffers for ntok tokens of k inputs
// (room for xprep_bind's rounding of each part to 256 bytes included).
constexpr uint64_t xprep_bytes(uint32_t ntok, uint32_t k) {
  return ((uint64_t)ntok + 15) / 16 * (k / 32) * 2 * 64 * 16 + ((uint64_t)ntok + 15) / 16 * 16 * 4 +
         2 * (((uint64_t)ntok + 15) / 16) * 16 * (k / 32) * 4 + 4 * 256;
}
// Point a.xp / a.xexp / a.xbsum / a.xdx into one buffer of xprep_bytes.
inline void xprep_bind(GemvArgs* a, void* buf) {
  uint64_t tg = (a->ntok + 15) / 16, nb = a->nb;
  char* p = (char*)buf;
  a->xp = p;
  p += (tg * nb * 2 * 64 * 16 + 255) & ~255ull;
  a->xexp = (int32_t*)p;
  p += (tg * 16 * 4 + 255) & ~255ull;
  a->xbsum = (float*)p;
  p += (tg * 16 * nb * 4 + 255) & ~255ull;
  a->xdx = (float*)p;
  a->tg = (uint32_t)tg;
}
// Tokens at or above which the prefill kernel pair (prep + gemm) runs.
constexpr uint32_t GEMM_MIN_TOKENS = 5;
// The prefill kernel pair: prep_kernel stages the activations (prologue `pro`)
// once for the launch, gemm_kernel runs every weight tile over all tokens.
int prep_launch(const GemvArgs& a, int pro, hipStream_t s);
int gemm_launch(const GemvArgs& a, uint32_t qtype, int epi, hipStream_t s);

// Bytes of LDS a launch needs, and whether the shape is supported.
int gemv_launch(const GemvArgs& a, uint32_t qtype, int pro, int epi, hipStream_t s);
// Workgroups the launch uses along x (EPI_ARGMAX partial count).
uint32_t gemv_groups(const GemvArgs& a);
// Picks the split-K factor (waves per tile) and the waves per workgroup.
void gemv_pick(uint32_t tiles, uint32_t ng, uint32_t tail, uint32_t nb, uint32_t* split, uint32_t* waves);
// Picks the streaming form for a one-token launch: workgroups (0: none: fewer than
// GEMV_STREAM_MIN_TILES tiles, or tail blocks) and waves per workgroup.
void gemv_pick_stream(uint32_t tiles, uint32_t nb, uint32_t* wgs, uint32_t* waves);
// Tiles from which one-token launches stream.
constexpr uint32_t GEMV_STREAM_MIN_TILES = 4096;

// Fill a GemvArgs with the matrix fields of m.
void gemv_bind(GemvArgs* a, const QMat& m);

// Allocation and device repack of raw GGUF blocks.
int qmat_alloc(QMat* m, int device, uint32_t type, uint64_t rows, uint64_t k);
// The geometry of a matrix placed at mem (zeroed device memory of at least
// Geom::dev_bytes(), owned by the caller; nullptr only to size it).
int qmat_place(QMat* m, int device, uint32_t type, uint64_t rows, uint64_t k, uint8_t* mem);
void qmat_release(QMat* m);
// Host -> device staging for uploads of raw GGUF blocks (stage.cpp):
// STAGE_BUFS pinned host buffers and as many device buffers of cap bytes.
constexpr int STAGE_BUFS = 3;
struct Stager {
  int device = -1;
  uint8_t* host[STAGE_BUFS] = {};
  uint8_t* dev[STAGE_BUFS] = {};
  hipEvent_t done[STAGE_BUFS] = {};    // the model's stream finished with the buffer
  hipEvent_t copied[STAGE_BUFS] = {};  // the latest DMA out of the buffer finished
  hipStream_t copy = nullptr;          // the DMA stream (default priority)
  int cur = 0;        // the buffer being filled
  uint64_t used = 0;  // bytes of it handed out
  uint64_t cap = 0;   // 0: not allocated
  hipStream_t stream = nullptr;  // the repack and f32 copies run here
};
int stager_init(Stager* st, int device, uint64_t cap, hipStream_t s);
void stager_free(Stager* st);
// Where upload bytes come from: caller memory, or a file read with pread.
// Offsets passed with a Source count from mem / file_off.
struct Source {
  const uint8_t* mem = nullptr;
  int fd = -1;
  uint64_t file_off = 0;
};
// Fill dst with bytes [off, off+n) of src, split over the staging threads.
int stage_read(const Source& src, uint64_t off, void* dst, uint64_t n);
// Upload raw GGUF bytes [byte_off, byte_off+nbytes) of a tensor whose first
// row is logical row row_off of m (a fused matrix holds several tensors);
// src holds those nbytes.
int qmat_upload(Stager* st, const QMat& m, const Source& src, uint64_t nbytes, uint64_t byte_off, uint64_t row_off);
// Bytes [byte_off, byte_off+nbytes) of an f32 tensor at dst (device), staged
// like the quantised pieces (no synchronisation of the stream).
int f32_upload(Stager* st, float* dst, const Source& src, uint64_t nbytes, uint64_t byte_off);
// One piece of a batched file upload: bytes [off, off+bytes) of a tensor
// (whole blocks of q, or of the f32 array f) found at file offset `file`.
struct StagePiece {
  const QMat* q;
  float* f;
  uint64_t row_off, off, bytes, file;
};
// Upload pieces sorted by file offset, each at most the staging capacity:
// runs of consecutive pieces are read with one parallel pread and one DMA.
int stage_file_runs(Stager* st, int fd, const StagePiece* ps, size_t count);
inline int qmat_upload(Stager* st, const QMat& m, const void* raw, uint64_t nbytes, uint64_t byte_off,
                       uint64_t row_off) {
  Source src;
  src.mem = (const uint8_t*)raw;
  return qmat_upload(st, m, src, nbytes, byte_off, row_off);
}
// Dequantise rows [0, rows) (logical order) into out_dev[rows][k].
int qmat_dequant(const QMat& m, float* out_dev, hipStream_t s);
// Embedding gather: x[t][:] = row tokens[state[1] + t] of m (exact), t < ntok.
int embed_launch(const QMat& m, const int32_t* tokens, const uint32_t* state, float* x, uint32_t ntok,
                 hipStream_t s);

// Per-type launchers, instantiated in gemv_q40.hip / gemv_q41.hip / gemv_q80.hip.
template <uint32_t QT>
int gemv_launch_qt(const GemvArgs& a, int pro, int epi, hipStream_t s);
template <uint32_t QT>
int repack_launch_qt(const QMat& m, const uint8_t* raw_dev, uint64_t n, uint64_t blk0, uint64_t row_off,
                     uint32_t map, uint32_t hd, uint32_t seg0, uint32_t seg1, uint32_t ff, hipStream_t s);
template <uint32_t QT>
int dequant_launch_qt(const QMat& m, float* out, uint32_t map, uint32_t hd, uint32_t seg0, uint32_t seg1, uint32_t ff,
                      hipStream_t s);
template <uint32_t QT>
int gemm_launch_qt(const GemvArgs& a, int epi, hipStream_t s);
template <uint32_t QT>
int embed_launch_qt(const QMat& m, const int32_t* tokens, const uint32_t* state, float* x, uint32_t ntok,
                    hipStream_t s);

}  // namespace llmhip
