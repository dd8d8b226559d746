// The model: device buffers under a memory budget, the weights in fused
// groups, and the forward pass recorded once into hipGraphs (one decode step,
// one prefill chunk per chunk length).  Every kernel reads the position from
// the device-side state, so a graph replays at any position.
#include <algorithm>
#include <cmath>
#include <iterator>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "gemv.h"
#include "layer.h"
#include "pass.h"

namespace llmhip {

struct TensorInfo {
  uint32_t type = 0;
  std::vector<uint64_t> dims;
  uint64_t size = 0, received = 0;  // received: bytes covered by the uploads so far
  std::map<uint64_t, uint64_t> got;  // the uploaded byte ranges, start -> end, disjoint
  bool used = false;
};

// Refuses a range [off, off + n) of tensor `name` that overlaps one uploaded
// before (a second upload of the same bytes would let finalize accept a tensor
// part of which was never written).
static int check_range(const TensorInfo& t, const char* name, uint64_t off, uint64_t n) {
  if (n == 0) return 0;
  auto it = t.got.upper_bound(off);  // first range starting after off
  const bool before = it != t.got.begin() && std::prev(it)->second > off;
  const bool after = it != t.got.end() && it->first < off + n;
  if (before || after)
    return set_error(LLMHIP_ERR_ARG, "llm: upload of %s bytes [%llu, %llu) overlaps bytes already uploaded", name,
                     (unsigned long long)off, (unsigned long long)(off + n));
  return 0;
}

// Records an accepted range (check_range passed), merging it with its neighbours.
static void add_range(TensorInfo& t, uint64_t off, uint64_t n) {
  if (n == 0) return;
  uint64_t a = off, b = off + n;
  auto it = t.got.lower_bound(a);
  if (it != t.got.begin() && std::prev(it)->second == a) {
    --it;
    a = it->first;
    it = t.got.erase(it);
  }
  if (it != t.got.end() && it->first == b) {
    b = it->second;
    t.got.erase(it);
  }
  t.got[a] = b;
  t.received += n;
}

struct Layer {
  QMat qkv[3];
  uint32_t qkv_type[3] = {0, 0, 0}, qkv_base[3] = {0, 0, 0};
  int nqkv = 0;
  QMat o;
  QMat gu[2];
  int ngu = 0;
  QMat down;
  float* attn_norm = nullptr;
  float* ffn_norm = nullptr;
  float* bias = nullptr;  // [q; k; v] biases (qwen2)
  float* kv = nullptr;    // [2][ctx][kvd]
};

struct ProfRec {
  const char* cls;
  int layer;
  uint64_t bytes;
  hipEvent_t a, b;
};

// What one lane of a prefill wavefront owns: its stream, its activation and
// staging buffers, and its device-side position (the KV cache is shared:
// chunks write disjoint rows).  Lane 0 is the model's own fields.
constexpr int LANES = 3;
struct Lane {
  hipStream_t stream = nullptr;
  float *x = nullptr, *q = nullptr, *att = nullptr, *act = nullptr, *gbuf = nullptr, *pv = nullptr, *ml = nullptr;
  void* xprep = nullptr;
  uint32_t* state = nullptr;
  void* xprep2 = nullptr;
};

struct Model {
  int device = 0;
  llmhip_limits lim{};
  llmhip_config cfg{};
  uint32_t ctx = 0, pm = 64, smax = 0, kvd = 0;
  uint64_t used = 0;
  std::vector<void*> allocs;
  uint8_t* arena = nullptr;  // weights, norms, biases, KV caches (allocate)
  uint64_t arena_cap = 0, arena_used = 0;
  bool sizing = false;
  hipStream_t stream = nullptr;
  Stager st;
  // gbuf: the up product of the pass's last layer ([pm][ff], Peek "up"; the
  // gate values in between when gate and up have different types); h: the
  // head's normed row, formed on demand by Peek("h")
  // xn: the embedding row of the token the last head pass sampled, which the
  // sampling kernel writes: the input of the next one-token pass
  float *x = nullptr, *q = nullptr, *act = nullptr, *gbuf = nullptr, *logits = nullptr, *pv = nullptr,
        *ml = nullptr, *amax_v = nullptr, *cs = nullptr, *att = nullptr, *h = nullptr, *xn = nullptr;
  // kpart: rows 0 and 1 the two k-halves of a one-token pass's down
  // projection, which the next layer's K1 adds to the residual x and stores,
  // summed, to row 2, where that layer's K3 takes its residual from (x itself
  // is never written by a launch that reads it).  k5_split: the K5 just
  // recorded stored halves; xsum_ready: the K1 just recorded stored the sum.
  float* kpart = nullptr;
  bool k5_split = false, xsum_ready = false;
  void* xprep = nullptr;   // prepared activations of a prefill chunk
  void* xprep2 = nullptr;  // ... of its down projection, which the gate/up product writes (act_operands)
  uint32_t *amax_i = nullptr, *state = nullptr;
  int32_t *tokens = nullptr, *outb = nullptr;
  int32_t* host = nullptr;  // pinned: prompt ids in, sampled ids out
  uint32_t host_cap = 0;
  uint8_t* bounce = nullptr;  // pinned: every copy to or from caller memory passes through it
  QMat embd, out;
  bool tied = false;
  float* out_norm = nullptr;
  std::vector<Layer> layers;
  std::map<std::string, TensorInfo> tensors;
  bool allocated = false, finalized = false;
  bool kv16 = false;  // binary16 KV cache (the F16KV mode of cpu.go:22-24)
  bool q8 = false;    // ExactGGML (cpu.go:15-21): every matrix input quantised to Q8 blocks, binary16 cache
  hipGraphExec_t decode_exec = nullptr;
  std::map<uint64_t, hipGraphExec_t> chunk_exec;  // key: graph_key (pass or segment, lane, shape)
  std::map<uint64_t, uint32_t> graph_nodes;       // dispatches per graph key
  llmhip_stats stats{};
  int layers_limit = 0;
  std::set<std::string> skip;
  uint32_t pos = 0;  // host mirror of state[0] (== state[1])
  uint32_t last_row = 0;     // the row of x holding the last token of the latest pass
  uint32_t attn_rows = 0;    // pass being recorded: cache rows its attention reads
  bool attn_split = false;   // ... and whether it runs in chunks merged by a second kernel
  bool embed_in = true;      // ... and whether it embeds its tokens (else its one input row is xn)
  bool prompted = false;
  uint32_t dispatches = 0;  // counter while recording
  std::vector<ProfRec>* prof = nullptr;  // eager profiling: events around every launch
  int cur_layer = -1;
  // the prefill wavefront's lanes (lane 0: the fields above), whose buffers
  // use_lane puts into those fields while their work is recorded; an event per
  // segment of chunk c in set c % (LANES + 1), and per lane its start and end
  // (prefill_wavefront)
  Lane lanes[LANES];
  int lane = 0;
  std::vector<hipEvent_t> seg_done[LANES + 1];
  hipEvent_t lane_ev[LANES] = {};
  // the fused decode pass (pass.hip): its flag-carrying vectors (one
  // allocation), control words [epoch, timed-out waits, poll limit, pad], the
  // layer table on the device and the arguments; pass_ok: the model fits it
  // (else pass_why), pass_on: decode passes take it (llmhip_model_set_fused)
  uint64_t* ll = nullptr;
  uint32_t* pctrl = nullptr;
  PassLayer* ptab = nullptr;
  PassArgs pargs{};
  uint32_t pgrid = 0;
  bool pass_ok = false, pass_on = true, pass_q8 = false;
  std::string pass_why = "not finalized";
};

// Brackets one launch with HIP events on the model's stream when profiling.
template <class F>
static int launch_rec(Model& m, const char* cls, uint64_t bytes, F&& launch) {
  m.dispatches++;
  if (!m.prof) return launch();
  ProfRec r{cls, m.cur_layer, bytes, nullptr, nullptr};
  LLM_HIP(hipEventCreate(&r.a));
  LLM_HIP(hipEventCreate(&r.b));
  m.prof->push_back(r);
  LLM_HIP(hipEventRecord(r.a, m.stream));
  LLM_TRY(launch());
  LLM_HIP(hipEventRecord(r.b, m.stream));
  return 0;
}

// Transfers between the device and caller memory go through the model's
// pinned bounce buffer in pieces of BOUNCE_BYTES: the runtime only ever DMAs
// to or from memory the library allocated pinned, never to pageable caller
// memory (which it would have to lock or stage itself), and the library holds
// no caller pointer after a call returns.
constexpr uint64_t BOUNCE_BYTES = 1ull << 20;

// n bytes device -> caller memory, on the model's stream (synchronous).
static int copy_out(Model& m, void* dst, const void* src, uint64_t n) {
  for (uint64_t o = 0; o < n; o += BOUNCE_BYTES) {
    const uint64_t c = std::min(BOUNCE_BYTES, n - o);
    LLM_HIP(hipMemcpyAsync(m.bounce, (const char*)src + o, c, hipMemcpyDeviceToHost, m.stream));
    LLM_HIP(hipStreamSynchronize(m.stream));
    memcpy((char*)dst + o, m.bounce, c);
  }
  return 0;
}

// n bytes caller memory -> device, on the model's stream (synchronous).
static int copy_in(Model& m, void* dst, const void* src, uint64_t n) {
  for (uint64_t o = 0; o < n; o += BOUNCE_BYTES) {
    const uint64_t c = std::min(BOUNCE_BYTES, n - o);
    LLM_HIP(hipStreamSynchronize(m.stream));
    memcpy(m.bounce, (const char*)src + o, c);
    LLM_HIP(hipMemcpyAsync((char*)dst + o, m.bounce, c, hipMemcpyHostToDevice, m.stream));
  }
  LLM_HIP(hipStreamSynchronize(m.stream));
  return 0;
}

static int over_budget(const Model& m) {
  return set_error(LLMHIP_ERR_BUDGET,
                   "llm: the model needs more GPU memory than the %llu bytes granted (run with a larger budget)",
                   (unsigned long long)m.lim.memory_budget);
}

// Zeroed device memory of `bytes` (rounded up to 256), counted against the
// budget.  While the weights arena is being sized (m.sizing) only the size is
// counted; while it is being carved the memory comes from it.
static int dalloc(Model& m, void** p, uint64_t bytes) {
  bytes = (bytes + 255) & ~255ull;
  if (m.sizing) {
    *p = nullptr;
    m.arena_cap += bytes;
    return 0;
  }
  if (m.used + bytes > m.lim.memory_budget) return over_budget(m);
  if (m.arena && m.arena_used + bytes <= m.arena_cap) {
    *p = m.arena + m.arena_used;
    m.arena_used += bytes;
  } else {
    LLM_HIP(hipMalloc(p, bytes));
    LLM_HIP(hipMemset(*p, 0, bytes));
    m.allocs.push_back(*p);
  }
  m.used += bytes;
  return 0;
}

template <class T>
static int dalloc_n(Model& m, T** p, uint64_t n) {
  return dalloc(m, (void**)p, n * sizeof(T));
}

static int qalloc(Model& m, QMat* q, uint32_t type, uint64_t rows, uint64_t k) {
  QType qt;
  if (!qtype_of(type, &qt))
    return set_error(LLMHIP_ERR_TYPE, "llm: a tensor has ggml type %u, which has no GPU kernel yet (Q4_0, Q4_1, Q8_0)",
                     type);
  void* mem;
  LLM_TRY(dalloc(m, &mem, make_geom(qt, rows, k).dev_bytes()));
  return qmat_place(q, m.device, type, rows, k, (uint8_t*)mem);
}

static void destroy_graphs(Model& m) {
  if (m.decode_exec) (void)hipGraphExecDestroy(m.decode_exec);
  m.decode_exec = nullptr;
  for (auto& kv : m.chunk_exec) (void)hipGraphExecDestroy(kv.second);
  m.chunk_exec.clear();
  m.graph_nodes.clear();
}

static void model_destroy(Model* m) {
  if (!m) return;
  (void)hipSetDevice(m->device);
  if (m->stream) (void)hipStreamSynchronize(m->stream);
  for (int k = 1; k < LANES; k++)
    if (m->lanes[k].stream) (void)hipStreamSynchronize(m->lanes[k].stream);
  destroy_graphs(*m);
  for (auto& v : m->seg_done)
    for (hipEvent_t e : v) (void)hipEventDestroy(e);
  for (hipEvent_t e : m->lane_ev)
    if (e) (void)hipEventDestroy(e);
  for (int k = 1; k < LANES; k++)
    if (m->lanes[k].stream) (void)hipStreamDestroy(m->lanes[k].stream);
  stager_free(&m->st);
  qmat_release(&m->embd);
  qmat_release(&m->out);
  for (auto& l : m->layers) {
    for (auto& q : l.qkv) qmat_release(&q);
    qmat_release(&l.o);
    for (auto& q : l.gu) qmat_release(&q);
    qmat_release(&l.down);
  }
  for (void* p : m->allocs) (void)hipFree(p);
  if (m->host) (void)hipHostFree(m->host);
  if (m->bounce) (void)hipHostFree(m->bounce);
  if (m->stream) (void)hipStreamDestroy(m->stream);
  delete m;
}

// ------------------------------------------------------------ tensors

static std::string layer_name(int l, const char* suffix) { return "blk." + std::to_string(l) + "." + suffix; }

// Expected shape of every tensor the forward pass reads (cpu.go:225-366).
static bool expected(const Model& m, const std::string& name, bool* quant, std::vector<uint64_t>* dims) {
  const llmhip_config& c = m.cfg;
  uint64_t E = c.embd, F = c.ff, kvd = m.kvd, V = c.vocab;
  if (name == "token_embd.weight") { *quant = true; *dims = {E, V}; return true; }
  if (name == "output_norm.weight") { *quant = false; *dims = {E}; return true; }
  if (name == "output.weight") { *quant = true; *dims = {E, V}; return true; }
  if (name.rfind("blk.", 0) != 0) return false;
  size_t dot = name.find('.', 4);
  if (dot == std::string::npos) return false;
  int l = atoi(name.c_str() + 4);
  if (l < 0 || l >= c.layers || std::to_string(l) != name.substr(4, dot - 4)) return false;
  std::string s = name.substr(dot + 1);
  if (s == "attn_norm.weight" || s == "ffn_norm.weight") { *quant = false; *dims = {E}; return true; }
  if (s == "attn_q.weight" || s == "attn_output.weight") { *quant = true; *dims = {E, E}; return true; }
  if (s == "attn_k.weight" || s == "attn_v.weight") { *quant = true; *dims = {E, kvd}; return true; }
  if (s == "ffn_gate.weight" || s == "ffn_up.weight") { *quant = true; *dims = {E, F}; return true; }
  if (s == "ffn_down.weight") { *quant = true; *dims = {F, E}; return true; }
  if (c.bias) {
    if (s == "attn_q.bias") { *quant = false; *dims = {E}; return true; }
    if (s == "attn_k.bias" || s == "attn_v.bias") { *quant = false; *dims = {kvd}; return true; }
  }
  return false;
}

static const TensorInfo* need(Model& m, const std::string& n) {
  auto it = m.tensors.find(n);
  if (it == m.tensors.end()) {
    set_error(LLMHIP_ERR_FORMAT, "llm: missing tensor %s", n.c_str());
    return nullptr;
  }
  return &it->second;
}

// Allocate every weight once all tensors are declared: the fused groups need
// the types of all their members (fused.go:108-190 concatenates QKV and
// gate/up when they share a type; here mixed types get one matrix each).
static int allocate_pass(Model& m) {
  const llmhip_config& c = m.cfg;
  const uint32_t E = c.embd, F = c.ff, kvd = m.kvd, hd = c.head_dim;
  const TensorInfo* te = need(m, "token_embd.weight");
  if (!te) return LLMHIP_ERR_FORMAT;
  if (te->type != LLMHIP_Q8_0 && te->type != LLMHIP_Q4_0)
    return set_error(LLMHIP_ERR_TYPE, "llm: token_embd.weight must be Q8_0 or Q4_0");
  LLM_TRY(qalloc(m, &m.embd, te->type, c.vocab, E));
  if (!need(m, "output_norm.weight")) return LLMHIP_ERR_FORMAT;
  LLM_TRY(dalloc_n(m, &m.out_norm, E));
  m.tied = c.tied_output != 0;
  if (!m.tied) {
    const TensorInfo* to = need(m, "output.weight");
    if (!to) return LLMHIP_ERR_FORMAT;
    LLM_TRY(qalloc(m, &m.out, to->type, c.vocab, E));
  }
  m.layers.resize(c.layers);
  for (int l = 0; l < c.layers; l++) {
    Layer& L = m.layers[l];
    const TensorInfo* t[7];
    const char* names[7] = {"attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_output.weight",
                            "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"};
    for (int i = 0; i < 7; i++)
      if (!(t[i] = need(m, layer_name(l, names[i])))) return LLMHIP_ERR_FORMAT;
    if (!need(m, layer_name(l, "attn_norm.weight")) || !need(m, layer_name(l, "ffn_norm.weight")))
      return LLMHIP_ERR_FORMAT;
    LLM_TRY(dalloc_n(m, &L.attn_norm, E));
    LLM_TRY(dalloc_n(m, &L.ffn_norm, E));
    if (c.bias) {
      for (const char* b : {"attn_q.bias", "attn_k.bias", "attn_v.bias"})
        if (!need(m, layer_name(l, b))) return LLMHIP_ERR_FORMAT;
      LLM_TRY(dalloc_n(m, &L.bias, E + 2 * kvd));
    }
    // Q, K, V: one matrix [q; k; v] when they share a type
    if (t[0]->type == t[1]->type && t[1]->type == t[2]->type) {
      L.nqkv = 1;
      L.qkv_type[0] = t[0]->type;
      if (c.rope_neox) {
        L.qkv[0].map = MAP_NEOX;
        L.qkv[0].map_hd = hd;
        L.qkv[0].map_seg0 = 0;
        L.qkv[0].map_seg1 = E + kvd;
      }
      LLM_TRY(qalloc(m, &L.qkv[0], t[0]->type, E + 2 * kvd, E));
    } else {
      L.nqkv = 3;
      uint32_t rows[3] = {E, kvd, kvd}, base[3] = {0, E, E + kvd};
      for (int i = 0; i < 3; i++) {
        L.qkv_type[i] = t[i]->type;
        L.qkv_base[i] = base[i];
        if (c.rope_neox && i < 2) {
          L.qkv[i].map = MAP_NEOX;
          L.qkv[i].map_hd = hd;
          L.qkv[i].map_seg0 = 0;
          L.qkv[i].map_seg1 = rows[i];
        }
        LLM_TRY(qalloc(m, &L.qkv[i], t[i]->type, rows[i], E));
      }
    }
    LLM_TRY(qalloc(m, &L.o, t[3]->type, E, E));
    if (t[4]->type == t[5]->type && F % 8 == 0) {
      L.ngu = 1;
      L.gu[0].map = MAP_GATEUP;
      L.gu[0].ff = F;
      LLM_TRY(qalloc(m, &L.gu[0], t[4]->type, 2 * F, E));
    } else {
      L.ngu = 2;
      LLM_TRY(qalloc(m, &L.gu[0], t[4]->type, F, E));
      LLM_TRY(qalloc(m, &L.gu[1], t[5]->type, F, E));
    }
    LLM_TRY(qalloc(m, &L.down, t[6]->type, E, F));
    LLM_TRY(dalloc(m, (void**)&L.kv, 2ull * m.ctx * kvd * (m.kv16 ? 2 : 4)));
  }
  return 0;
}

// The weights, norms, biases and KV caches in one zeroed device arena: one
// pass sizes it, one hipMalloc and one fill, a second pass carves it (about a
// hundred separate allocations cost milliseconds at load and at free).
static int allocate(Model& m) {
  m.sizing = true;
  m.arena_cap = 0;
  int rc = allocate_pass(m);
  m.sizing = false;
  if (rc) return rc;
  if (m.used + m.arena_cap > m.lim.memory_budget) return over_budget(m);
  LLM_HIP(hipSetDevice(m.device));
  LLM_HIP(hipMalloc((void**)&m.arena, m.arena_cap));
  m.allocs.push_back(m.arena);
  LLM_HIP(hipMemsetAsync(m.arena, 0, m.arena_cap, m.stream));
  m.arena_used = 0;
  LLM_TRY(allocate_pass(m));
  m.allocated = true;
  return 0;
}

// Where the bytes of a tensor go: a matrix (and its first row there) or a
// float array (and its float offset).
static int route(Model& m, const std::string& name, QMat** q, uint64_t* row_off, float** f) {
  *q = nullptr;
  *f = nullptr;
  *row_off = 0;
  const uint32_t E = m.cfg.embd, kvd = m.kvd, F = m.cfg.ff;
  if (name == "token_embd.weight") { *q = &m.embd; return 0; }
  if (name == "output.weight") { *q = &m.out; return 0; }
  if (name == "output_norm.weight") { *f = m.out_norm; return 0; }
  int l = atoi(name.c_str() + 4);
  Layer& L = m.layers[l];
  std::string s = name.substr(name.find('.', 4) + 1);
  if (s == "attn_norm.weight") { *f = L.attn_norm; return 0; }
  if (s == "ffn_norm.weight") { *f = L.ffn_norm; return 0; }
  if (s == "attn_q.bias") { *f = L.bias; return 0; }
  if (s == "attn_k.bias") { *f = L.bias + E; return 0; }
  if (s == "attn_v.bias") { *f = L.bias + E + kvd; return 0; }
  int i = s == "attn_q.weight" ? 0 : s == "attn_k.weight" ? 1 : s == "attn_v.weight" ? 2 : -1;
  if (i >= 0) {
    if (L.nqkv == 1) {
      *q = &L.qkv[0];
      *row_off = i == 0 ? 0 : i == 1 ? E : E + kvd;
    } else {
      *q = &L.qkv[i];
    }
    return 0;
  }
  if (s == "attn_output.weight") { *q = &L.o; return 0; }
  if (s == "ffn_gate.weight" || s == "ffn_up.weight") {
    bool up = s == "ffn_up.weight";
    if (L.ngu == 1) {
      *q = &L.gu[0];
      *row_off = up ? F : 0;
    } else {
      *q = &L.gu[up ? 1 : 0];
    }
    return 0;
  }
  if (s == "ffn_down.weight") { *q = &L.down; return 0; }
  return set_error(LLMHIP_ERR_ARG, "llm: no place for tensor %s", name.c_str());
}

// ------------------------------------------------------------ recording

static bool skipped(const Model& m, const char* cls) { return m.skip.count("all") || m.skip.count(cls); }

static int gemv_rec(Model& m, const char* cls, const GemvArgs& a, uint32_t qtype, int pro, int epi, uint64_t bytes) {
  if (skipped(m, cls)) return 0;
  if (m.q8) pro |= PRO_Q8;
  return launch_rec(m, cls, bytes, [&]() { return gemv_launch(a, qtype, pro, epi, m.stream); });
}

// A prefill chunk (ntok >= GEMM_MIN_TOKENS) stages its activations once
// (prep_kernel) and runs gemm_kernel; decode runs gemv_kernel with the
// prologue fused.  `prep` false reuses the staging of the previous call (the
// matrices of one mixed-type group share an input).
static int mat_rec(Model& m, const char* cls, const char* pcls, GemvArgs a, uint32_t qtype, int pro, int epi,
                   uint64_t bytes, bool prep = true, bool block_scaled = false, void* xbuf = nullptr) {
  if (a.ntok < GEMM_MIN_TOKENS) return gemv_rec(m, cls, a, qtype, pro, epi, bytes);
  xprep_bind(&a, xbuf ? xbuf : m.xprep);
  if (m.q8) {
    pro |= PRO_Q8;
    a.q8 = 1;
  }
  if (block_scaled) a.q8 = 1;  // operands already staged per block (scale 2^-e in xdx)
  if (prep && !skipped(m, cls) && !skipped(m, pcls))
    LLM_TRY(launch_rec(m, pcls, 0, [&]() { return prep_launch(a, pro, m.stream); }));
  if (skipped(m, cls)) return 0;
  return launch_rec(m, cls, bytes, [&]() { return gemm_launch(a, qtype, epi, m.stream); });
}

static GemvArgs base_args(const Model& m, const QMat& q, uint32_t ntok) {
  GemvArgs a;
  memset(&a, 0, sizeof a);
  gemv_bind(&a, q);
  a.ntok = ntok;
  a.eps = m.cfg.eps;
  a.state = m.state;
  a.heads = m.cfg.heads;
  a.hd = m.cfg.head_dim;
  a.kv16 = m.kv16 ? 1 : 0;
  return a;
}

// Whether a one-token K5 (bound in a) runs in two k-parts whose halves the
// next layer's K1 adds: `want` when that K1 follows in the same pass.
// (The summing prologue holds the whole row in two float4s per lane: k <= 512 * 4 waves.)
// Decode passes only (!embed_in): the halves buffer and the flags that pass
// them from K5 to K1 to K3 belong to the model, not to a prefill lane, and a
// prefill's segments of different chunks (a one-token last chunk beside a
// 64-token one, or every chunk at PrefillBatch 1) are recorded interleaved.
static bool k5_splits(const Model& m, const GemvArgs& a, uint32_t ntok, bool want) {
  return want && ntok == 1 && !m.embed_in && !m.q8 && !a.stream && a.ng >= 2 && m.cfg.embd <= 2048 &&
         !skipped(m, "k5") && !skipped(m, "k1");
}

static int pass_layers(const Model& m, bool* head);

// Whether the layer after the current one runs in this pass.
static bool next_layer_runs(const Model& m) {
  bool h = true;
  return m.cur_layer + 1 < pass_layers(m, &h);
}

static int rec_k1(Model& m, const Layer& L, uint32_t ntok) {
  const llmhip_config& c = m.cfg;
  for (int i = 0; i < L.nqkv; i++) {
    GemvArgs a = base_args(m, L.qkv[i], ntok);
    a.x = m.cur_layer == 0 && !m.embed_in ? m.xn : m.x;
    int pro = PRO_RMS;
    if (m.k5_split) {  // the residual is x + the previous down projection's two halves
      a.xpart = m.kpart;
      a.xpartstride = c.embd;
      a.xout = m.kpart + 2 * c.embd;  // each launch's workgroup 0 stores the (same) sum there
      pro |= PRO_XSUM;
    }
    a.ldx = c.embd;
    a.nw = L.attn_norm;
    a.y = m.q;
    a.bias = L.bias;
    a.cs = m.cs;
    a.kv = L.kv;
    a.nq = c.embd;
    a.nk = m.kvd;
    a.kvd = m.kvd;
    a.ctx = m.ctx;
    a.neox = c.rope_neox;
    a.row_base = L.qkv_base[i];
    LLM_TRY(mat_rec(m, "k1", "p1", a, L.qkv_type[i], pro, EPI_QKV, L.qkv[i].g.gguf_bytes(), i == 0));
  }
  m.xsum_ready = m.k5_split;
  m.k5_split = false;
  return 0;
}

static AttnArgs attn_args(const Model& m, const Layer& L) {
  AttnArgs a;
  memset(&a, 0, sizeof a);
  a.q = m.q;
  a.kv = L.kv;
  a.pv = m.pv;
  a.ml = m.ml;
  a.att = m.att;
  a.state = m.state;
  a.heads = m.cfg.heads;
  a.kv_heads = m.cfg.kv_heads;
  a.hd = m.cfg.head_dim;
  a.kvd = m.kvd;
  a.ctx = m.ctx;
  a.smax = m.smax;
  a.rows = m.attn_rows;
  a.split = m.attn_split ? 1 : 0;
  a.kv16 = m.kv16 ? 1 : 0;
  a.scale = (float)(1 / std::sqrt((double)m.cfg.head_dim));  // cpu.go:304
  return a;
}

// A prefill chunk in f32 mode has the attention write the output
// projection's operands itself (per-block exponents), so K3 runs without its
// activation prep.
static bool att_operands(const Model& m, uint32_t ntok) {
  return ntok >= GEMM_MIN_TOKENS && !m.q8 && !skipped(m, "k2") && !skipped(m, "k3");
}

// Whether a prefill chunk's gate/up product (one matrix) also writes the down
// projection's block-scaled operands (GemvArgs::op_xp, into xprep2), so that
// no staging launch runs between the two (measured on MI355X, config 3
// prefill: 86.1k -> 87.2k tok/s; the staging launches took 6.7 us a layer,
// the four tiles per workgroup this form needs give most of it back).
static bool act_operands(const Model& m, const Layer& L, uint32_t ntok) {
  return ntok >= GEMM_MIN_TOKENS && !m.q8 && L.ngu == 1 && m.cfg.ff % 32 == 0 && !skipped(m, "k4") &&
         !skipped(m, "k5");
}

// A one-token pass with the split attention leaves the merge of the chunk
// partials to the output projection's prologue (PRO_MERGE: no merge kernel)
// where the partials fit its loads and registers; f32 activations only.
static bool merge_in_k3(const Model& m, const Layer& L, uint32_t ntok) {
  if (ntok != 1 || !m.attn_split || m.q8) return false;
  GemvArgs a;
  gemv_bind(&a, L.o);
  return (m.attn_rows + ATTN_DECODE_ROWS - 1) / ATTN_DECODE_ROWS <= MERGE_MAX_CHUNKS && a.waves <= 8 && !a.stream &&
         (a.ng + a.split - 1) / a.split <= 2;
}

static int rec_k2(Model& m, const Layer& L, uint32_t ntok) {
  if (skipped(m, "k2")) return 0;
  // KV bytes read for the last token of the pass (the decode step's one token)
  uint64_t bytes = 2ull * (m.pos + 1) * m.kvd * 4;
  AttnArgs a = attn_args(m, L);
  if (merge_in_k3(m, L, ntok)) return launch_rec(m, "k2", bytes, [&]() { return attn_launch(a, ntok, m.stream, nullptr, false); });
  if (m.attn_split) m.dispatches++;  // the merge kernel
  if (att_operands(m, ntok)) {
    GemvArgs g = base_args(m, L.o, ntok);
    xprep_bind(&g, m.xprep);
    const AttnOps ops = {g.xp, g.xdx, g.xbsum, g.xexp, g.nb};
    return launch_rec(m, "k2", bytes, [&]() { return attn_launch(a, ntok, m.stream, &ops); });
  }
  return launch_rec(m, "k2", bytes, [&]() { return attn_launch(a, ntok, m.stream); });
}

// the heads' merged outputs times W_o, added to the residual
static int rec_k3(Model& m, const Layer& L, uint32_t ntok) {
  GemvArgs a = base_args(m, L.o, ntok);
  a.x = m.att;
  a.ldx = m.cfg.embd;
  a.y = m.x;
  a.ldy = m.cfg.embd;
  if (m.cur_layer == 0 && !m.embed_in) a.yin = m.xn;  // the residual stream starts at the embedding row
  if (m.xsum_ready) a.yin = m.kpart + 2 * m.cfg.embd;  // x + the previous layer's down halves (K1 summed them)
  m.xsum_ready = false;
  if (merge_in_k3(m, L, ntok)) {
    a.mpv = m.pv;
    a.mml = m.ml;
    a.msmax = m.smax;
    a.mrows = ATTN_DECODE_ROWS;
    a.matt = m.att;  // Peek("att")
    const uint32_t chunks = (m.attn_rows + ATTN_DECODE_ROWS - 1) / ATTN_DECODE_ROWS;
    return gemv_rec(m, "k3", a, L.o.g.q.type, merge_pro(chunks), EPI_ACC, L.o.g.gguf_bytes());
  }
  const bool staged = att_operands(m, ntok);
  return mat_rec(m, "k3", "p3", a, L.o.g.q.type, PRO_PLAIN, EPI_ACC, L.o.g.gguf_bytes(), !staged, staged);
}

static int rec_k4(Model& m, const Layer& L, uint32_t ntok) {
  const llmhip_config& c = m.cfg;
  if (L.ngu == 1) {
    GemvArgs a = base_args(m, L.gu[0], ntok);
    a.x = m.x;
    a.ldx = c.embd;
    a.nw = L.ffn_norm;
    a.y = m.act;
    a.up = m.gbuf;
    a.ff = c.ff;
    if (act_operands(m, L, ntok)) {
      GemvArgs d = base_args(m, L.down, ntok);
      xprep_bind(&d, m.xprep2);
      a.op_xp = d.xp;
      a.op_dx = d.xdx;
      a.op_bsum = d.xbsum;
      a.op_exp = d.xexp;
      a.op_nb = d.nb;
    }
    return mat_rec(m, "k4", "p4", a, L.gu[0].g.q.type, PRO_RMS, EPI_GATEUP, L.gu[0].g.gguf_bytes());
  }
  GemvArgs g = base_args(m, L.gu[0], ntok);
  g.x = m.x;
  g.ldx = c.embd;
  g.nw = L.ffn_norm;
  g.y = m.gbuf;
  g.ldy = c.ff;
  LLM_TRY(mat_rec(m, "k4", "p4", g, L.gu[0].g.q.type, PRO_RMS, EPI_STORE, L.gu[0].g.gguf_bytes()));
  GemvArgs u = base_args(m, L.gu[1], ntok);
  u.x = m.x;
  u.ldx = c.embd;
  u.nw = L.ffn_norm;
  u.y = m.act;
  u.ldy = c.ff;
  u.aux = m.gbuf;
  u.up = m.gbuf;
  return mat_rec(m, "k4", "p4", u, L.gu[1].g.q.type, PRO_RMS, EPI_SWIGLU, L.gu[1].g.gguf_bytes(), false);
}

// split: a one-token pass whose next layer's K1 follows in the same pass
// stores the product's two k-halves to kpart instead of adding it to x (twice
// the workgroups for the long down rows; that K1 adds them, in order, to x).
static int rec_k5(Model& m, const Layer& L, uint32_t ntok, bool split = false) {
  GemvArgs a = base_args(m, L.down, ntok);
  a.x = m.act;
  a.ldx = m.cfg.ff;
  a.y = m.x;
  split = k5_splits(m, a, ntok, split);
  if (split) {
    a.kparts = 2;
    a.y = m.kpart;
    a.pstride = m.cfg.embd;
    m.k5_split = true;
    // a part's groups over eight waves, not sixteen, where the pick took
    // sixteen (Qwen shape: 3.71 against 3.99 us; 4 waves of 8: 5.36 us)
    if (a.split == 16 && a.waves == 16 && (uint64_t)a.nb * 4 <= 2ull * 64 * 8) {
      a.split = 8;
      a.waves = 8;
    }
    return gemv_rec(m, "k5", a, L.down.g.q.type, PRO_PLAIN, EPI_STORE, L.down.g.gguf_bytes());
  }
  a.ldy = m.cfg.embd;
  const bool staged = act_operands(m, L, ntok);
  return mat_rec(m, "k5", "p5", a, L.down.g.q.type, PRO_PLAIN, EPI_ACC, L.down.g.gguf_bytes(), !staged, staged,
                 staged ? m.xprep2 : nullptr);
}

static int rec_adv(Model& m, uint32_t n) {
  if (skipped(m, "adv")) return 0;
  m.cur_layer = -1;
  return launch_rec(m, "adv", 0, [&]() { return advance_launch(m.state, n, m.stream); });
}

static GemvArgs head_args(const Model& m, uint32_t xrow, uint32_t adv) {
  const QMat& w = m.tied ? m.embd : m.out;
  GemvArgs a = base_args(m, w, 1);
  a.x = m.x;
  a.ldx = m.cfg.embd;
  a.xrow0 = xrow;
  a.nw = m.out_norm;
  a.y = m.logits;
  a.ldy = m.cfg.vocab;
  a.amax_v = m.amax_v;
  a.amax_i = m.amax_i;
  (void)adv;
  return a;
}

// The final RMSNorm, the logits and per-workgroup argmax partials of the last
// token of the pass (recordHead, fused.go:269-289), then the sampling kernel,
// which writes tokens[step + adv] and advances the state.  With "argmax"
// skipped the state still advances.
static int rec_head(Model& m, uint32_t xrow, uint32_t adv) {
  const QMat& w = m.tied ? m.embd : m.out;
  GemvArgs a = head_args(m, xrow, adv);
  m.cur_layer = -1;
  LLM_TRY(gemv_rec(m, "head", a, w.g.q.type, PRO_RMS, EPI_ARGMAX, w.g.gguf_bytes()));
  if (skipped(m, "argmax")) return rec_adv(m, adv);
  uint32_t groups = gemv_groups(a);
  const bool emb = !skipped(m, "embed");  // the next one-token pass's input row
  return launch_rec(m, "argmax", 8ull * groups, [&]() {
    return argmax_launch(m.amax_v, m.amax_i, groups, m.logits, m.tokens, m.outb, m.state, adv, m.stream,
                         emb ? &m.embd : nullptr, emb ? m.xn : nullptr, m.pctrl);
  });
}


// LLMHIP_EAGER=1: passes go to the stream as direct launches instead of graph
// replays (same kernels, arguments and order), for tools that trace kernel
// launches but not graph replays.
static bool eager_passes() {
  static const bool e = [] {
    const char* v = getenv("LLMHIP_EAGER");
    return v && *v && strcmp(v, "0") != 0;
  }();
  return e;
}

// Layers a pass runs (Layers, gpu.go:143-146); fewer than all: no head.
static int pass_layers(const Model& m, bool* head) {
  int nl = m.cfg.layers;
  if (m.layers_limit != 0 && m.layers_limit < nl) {
    nl = std::max(m.layers_limit, 0);
    *head = false;
  }
  return nl;
}

// Slot s (0 .. layers) of a pass: s = 0 the embedding and layer 0's K1;
// then layer s-1's K2..K5 and layer s's K1; the last, the last layer's K2..K5
// and the head (or the advance).  A slot ends with the K1 that appends its
// layer's cache rows, which is what a later chunk's attention waits for.
static int record_slot(Model& m, uint32_t ntok, bool head, int s) {
  const int nl = pass_layers(m, &head);
  if (s == 0 && m.embed_in && !skipped(m, "embed")) {
    m.cur_layer = -1;
    uint64_t row = (uint64_t)m.embd.g.nb * m.embd.g.q.block_bytes;
    LLM_TRY(launch_rec(m, "embed", row * ntok,
                       [&]() { return embed_launch(m.embd, m.tokens, m.state, m.x, ntok, m.stream); }));
  }
  if (s >= 1 && s <= nl) {
    const Layer& L = m.layers[s - 1];
    m.cur_layer = s - 1;
    LLM_TRY(rec_k2(m, L, ntok));
    LLM_TRY(rec_k3(m, L, ntok));
    LLM_TRY(rec_k4(m, L, ntok));
    LLM_TRY(rec_k5(m, L, ntok, s < nl));  // split when this slot's K1 adds the halves
  }
  if (s < nl) {
    m.cur_layer = s;
    LLM_TRY(rec_k1(m, m.layers[s], ntok));
  }
  if (s == nl) return head ? rec_head(m, ntok - 1, ntok) : rec_adv(m, ntok);
  return 0;
}

// A segment of a pass of nl layers: slots [s0, s0 + n) (the pass's slots
// 0 .. nl).
static int record_segment(Model& m, uint32_t ntok, bool head, bool embed_in, int s0, int n) {
  m.embed_in = embed_in || ntok != 1;
  m.k5_split = m.xsum_ready = false;  // an embedding pass never splits its K5 (k5_splits)
  bool h = head;
  const int nl = pass_layers(m, &h);
  for (int s = s0; s < std::min(s0 + n, nl + 1); s++) LLM_TRY(record_slot(m, ntok, head, s));
  return 0;
}
// A prefill chunk's segments: G slots each from slot `shift` on, the slots
// before it one segment of their own.  seg_start: the first slot of segment
// i; seg_of: the segment that holds slot s.
static int seg_start(int i, int shift, int G) { return shift == 0 ? i * G : i == 0 ? 0 : shift + (i - 1) * G; }
static int seg_of(int s, int shift, int G) { return shift == 0 ? s / G : s < shift ? 0 : 1 + (s - shift) / G; }

// One pass of ntok tokens at positions state[0] .. state[0]+ntok-1: the
// embedding (embed_in; else the one token's row is xn, which the previous
// head pass's sampling kernel wrote), the layers, and (head) the logits and
// the sampled token of the last one, which goes to tokens[step + ntok], its
// embedding row to xn; state advances by ntok.
// Whether the one-token pass being recorded runs as the fused decode launch:
// a decode step (its input row is xn) of a model that fits it, with every
// layer and kernel class running, f32 activations, and positions past
// attn_full_max only where the long form holds them.
static bool use_pass(const Model& m, uint32_t ntok, bool head) {
  bool h = head;
  return m.pass_ok && m.pass_on && ntok == 1 && !m.embed_in && head && !m.q8 && m.skip.empty() &&
         (!m.attn_split || pass_long_fits(m.cfg, m.attn_rows, m.pgrid)) && pass_layers(m, &h) == m.cfg.layers && h;
}

static int record_pass(Model& m, uint32_t ntok, bool head, bool embed_in) {
  m.embed_in = embed_in || ntok != 1;
  m.k5_split = m.xsum_ready = false;  // a pass's last K5 never splits: nothing carries over
  if (use_pass(m, ntok, head)) {
    m.cur_layer = -1;
    PassArgs a = m.pargs;
    a.rows = m.attn_rows;
    // algorithmic bytes: every layer's matrices and the KV rows of the
    // positions attended
    uint64_t bytes = 0;
    for (const Layer& L : m.layers)
      bytes += L.qkv[0].g.gguf_bytes() + L.o.g.gguf_bytes() + L.gu[0].g.gguf_bytes() + L.down.g.gguf_bytes() +
               2ull * (m.pos + 1) * m.kvd * (m.kv16 ? 2 : 4);
    LLM_TRY(launch_rec(m, "pass", bytes, [&]() { return pass_launch(a, m.pgrid, m.pass_q8, m.attn_split, m.stream); }));
    return rec_head(m, ntok - 1, ntok);
  }
  bool h = head;
  const int nl = pass_layers(m, &h);
  for (int s = 0; s <= nl; s++) LLM_TRY(record_slot(m, ntok, head, s));
  return 0;
}

// Put lane k's buffers and stream into the model's fields.
static void use_lane(Model& m, int k) {
  if (m.lane == k) return;
  const Lane& a = m.lanes[k];
  m.stream = a.stream;
  m.x = a.x;
  m.q = a.q;
  m.att = a.att;
  m.act = a.act;
  m.gbuf = a.gbuf;
  m.pv = a.pv;
  m.ml = a.ml;
  m.xprep = a.xprep;
  m.state = a.state;
  m.xprep2 = a.xprep2;
  m.lane = k;
}

// The attention of a pass of ntok tokens from position pos: one chunk while
// every position is below attn_full_max (rows read: the next multiple of 64),
// else chunks merged by a second kernel (rows read: the next multiple of a
// granule of >= 512 rows, at most 16 per context).  Each (rows, split) pair is
// a graph variant.
static void attn_plan(Model& m, uint32_t pos, uint32_t ntok) {
  const uint32_t last = pos + ntok - 1;
  if (last < attn_full_max(m.cfg.head_dim)) {
    m.attn_rows = std::min((last / 64 + 1) * 64, m.ctx);
    m.attn_split = false;
    return;
  }
  const uint32_t gran = std::max(512u, (m.ctx / 16 + 127) / 128 * 128);
  m.attn_rows = std::min((last / gran + 1) * gran, m.ctx);
  m.attn_split = true;
}

// seg: -1 the whole pass (G > 1: G passes of one token, a decode submit),
// else segment seg of G layers (of the lane whose buffers the model holds)
static uint64_t graph_key(const Model& m, uint32_t ntok, bool head, bool embed_in, int seg, int G = 0) {
  return ((uint64_t)(seg + 1) << 50) | ((uint64_t)G << 46) | ((uint64_t)m.lane << 44) | ((uint64_t)ntok << 32) |
         ((uint64_t)m.attn_rows << 3) | (embed_in ? 4 : 0) | (m.attn_split ? 2 : 0) | (head ? 1 : 0);
}

// Capture record_pass (seg -1) or the segment of slots [seg, seg + G) into a
// graph (once per key).
static int graph_for(Model& m, uint32_t ntok, bool head, bool embed_in, int seg, int G, hipGraphExec_t* out) {
  uint64_t key = graph_key(m, ntok, head, embed_in, seg, G);
  auto it = m.chunk_exec.find(key);
  if (it != m.chunk_exec.end()) {
    *out = it->second;
    return 0;
  }
  hipGraph_t g = nullptr;
  m.dispatches = 0;
  LLM_HIP(hipStreamBeginCapture(m.stream, hipStreamCaptureModeThreadLocal));
  int rc = 0;
  if (seg >= 0) rc = record_segment(m, ntok, head, embed_in, seg, G);
  for (int i = 0; seg < 0 && i < std::max(G, 1) && rc == 0; i++) rc = record_pass(m, ntok, head, embed_in);
  hipError_t e = hipStreamEndCapture(m.stream, &g);
  if (rc != 0) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return set_error(LLMHIP_ERR_DEVICE, "llm: graph capture failed: %s", hipGetErrorString(e));
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return set_error(LLMHIP_ERR_DEVICE, "llm: graph instantiate failed: %s", hipGetErrorString(e));
  m.chunk_exec[key] = ex;
  m.graph_nodes[key] = m.dispatches;
  *out = ex;
  return 0;
}

// One pass of ntok tokens whose first position is pos (known on the host).

// embed_in false: a decode step, whose input row the previous pass's sampling
// kernel wrote to xn.
static int launch_graph(Model& m, uint32_t pos, uint32_t ntok, bool head, bool embed_in) {
  hipGraphExec_t ex;
  attn_plan(m, pos, ntok);
  m.last_row = ntok - 1;
  embed_in = embed_in || ntok != 1;
  if (eager_passes()) {
    m.dispatches = 0;
    LLM_TRY(record_pass(m, ntok, head, embed_in));
    m.stats.dispatches += m.dispatches;
    return 0;
  }
  LLM_TRY(graph_for(m, ntok, head, embed_in, -1, 0, &ex));
  LLM_HIP(hipGraphLaunch(ex, m.stream));
  m.stats.dispatches += m.graph_nodes[graph_key(m, ntok, head, embed_in, -1, 0)];
  return 0;
}

// cnt one-token decode passes from position pos as one graph (part of a
// submit, at most 15 passes): its attention variant is the last position's, and the
// earlier tokens stop at their own causal bound (the kernels read the
// position from the device).
static int launch_decode(Model& m, uint32_t pos, uint32_t cnt) {
  attn_plan(m, pos + cnt - 1, 1);
  m.last_row = 0;
  if (eager_passes()) {
    m.dispatches = 0;
    for (uint32_t i = 0; i < cnt; i++) LLM_TRY(record_pass(m, 1, true, false));
    m.stats.dispatches += m.dispatches;
    return 0;
  }
  hipGraphExec_t ex;
  LLM_TRY(graph_for(m, 1, true, false, -1, (int)cnt, &ex));
  LLM_HIP(hipGraphLaunch(ex, m.stream));
  m.stats.dispatches += m.graph_nodes[graph_key(m, 1, true, false, -1, (int)cnt)];
  return 0;
}

// Lanes of the prefill wavefront, at most (LLMHIP_PREFILL_LANES=1 or 2: that
// many, for comparison).
static int prefill_lanes() {
  static const int n = [] {
    const char* v = getenv("LLMHIP_PREFILL_LANES");
    return v && (*v == '1' || *v == '2') ? *v - '0' : LANES;
  }();
  return n;
}

// A prompt of several chunks as a wavefront over L lanes (two for two
// chunks, three for more: measured, two and three whole prefills run at once
// reach 1.55x and 1.84x the throughput of one, four 1.58x): chunk c runs on
// lane (C-1-c) % L (the last on lane 0, whose buffers Peek and decode use),
// from its own position (set_state), as graph segments of G layers
// (record_segment); a segment of chunk c waits for the segment of chunk c-1
// that appended the cache rows of the latest layer whose attention it runs
// (the chunks before c-1 ran earlier on its lane or were waited for by c-1).
// The chunks of a group of L are enqueued segment by segment in turn, so that
// each starts one segment behind the one before rather than after the host
// has enqueued all of it; chunk c's events are set c % (LANES + 1), so that
// every wait names the record of the chunk right before.  On two lanes chunk
// c's segments start c % G slots later than chunk c-1's (seg_start): a
// segment then waits for the one of c-1 that ends one slot before its own
// end, so c trails c-1 by G - 1 slots, not G.  Several chunks' layers then
// run at once where one chunk's kernels leave the GPU idle.
static int prefill_wavefront(Model& m, uint32_t n) {
  const uint32_t C = (n + m.pm - 1) / m.pm;
  const uint32_t L = std::min<uint32_t>(std::min<uint32_t>(C, 3), (uint32_t)prefill_lanes());
  constexpr uint32_t S = LANES + 1;
  LLM_HIP(hipEventRecord(m.lane_ev[0], m.lanes[0].stream));  // the prompt upload
  for (uint32_t k = 1; k < L; k++) LLM_HIP(hipStreamWaitEvent(m.lanes[k].stream, m.lane_ev[0], 0));
  int rc = 0;
  auto chunk = [&](uint32_t c, uint32_t* a, uint32_t* ntok, bool* head) {
    *a = c * m.pm;
    const uint32_t b = std::min(*a + m.pm, n);
    *ntok = b - *a;
    *head = b == n;
    use_lane(m, (int)((C - 1 - c) % L));
    attn_plan(m, *a, *ntok);
    m.last_row = *ntok - 1;
  };
  // segments of three layers for a two-chunk prompt, where the second chunk's
  // lag weighs most; six for longer ones, where fewer graph launches weigh
  // more (measured: configs 3 and 4 at one to eight layers).  With three
  // lanes chunk c-2 runs on another stream: its rows are ready for chunk c
  // because c-1 waited for the same segment of it, which holds them only when
  // a segment has two or more layers and the chunks' segments line up.
  const int G = C <= 2 ? 3 : 6;
  static_assert(LANES <= 3, "the event sets and the G >= 2 argument are for at most three lanes");
  bool h0 = true;
  const int nl = pass_layers(m, &h0);
  auto shift = [&](uint32_t c) { return L == 2 ? (int)(c % (uint32_t)G) : 0; };
  for (uint32_t c0 = 0; c0 < C && rc == 0; c0 += L) {
    const uint32_t cn = std::min(C - c0, L);
    for (int i = 0; rc == 0; i++) {
      bool any = false;
      for (uint32_t c = c0; c < c0 + cn && rc == 0; c++) {
        const int s0 = seg_start(i, shift(c), G), s1 = std::min(seg_start(i + 1, shift(c), G), nl + 1);
        if (s0 > nl) continue;
        any = true;
        uint32_t a, ntok;
        bool head;
        chunk(c, &a, &ntok, &head);
        if (i == 0) {
          rc = set_state_launch(m.state, a, m.stream);
          m.stats.submits++;
        }
        // the latest attention here is layer s1 - 2's, which reads the rows chunk c-1's slot s1 - 2 appends
        if (rc == 0 && c > 0 && s1 >= 2 &&
            hipStreamWaitEvent(m.stream, m.seg_done[(c - 1) % S][seg_of(s1 - 2, shift(c - 1), G)], 0) != hipSuccess)
          rc = set_error(LLMHIP_ERR_DEVICE, "llm: prefill: stream wait failed");
        if (rc == 0 && eager_passes()) {
          m.dispatches = 0;
          rc = record_segment(m, ntok, head, true, s0, s1 - s0);
          m.stats.dispatches += m.dispatches;
        } else if (rc == 0) {
          hipGraphExec_t ex;
          rc = graph_for(m, ntok, head, true, s0, s1 - s0, &ex);
          if (rc == 0 && hipGraphLaunch(ex, m.stream) != hipSuccess)
            rc = set_error(LLMHIP_ERR_DEVICE, "llm: prefill: graph launch failed");
          if (rc == 0) m.stats.dispatches += m.graph_nodes[graph_key(m, ntok, head, true, s0, s1 - s0)];
        }
        if (rc == 0 && hipEventRecord(m.seg_done[c % S][i], m.stream) != hipSuccess)
          rc = set_error(LLMHIP_ERR_DEVICE, "llm: prefill: event record failed");
      }
      if (!any) break;
    }
  }
  use_lane(m, 0);
  // lane 0 goes on after the other lanes' last work
  for (uint32_t k = 1; k < L; k++)
    if (hipEventRecord(m.lane_ev[k], m.lanes[k].stream) != hipSuccess ||
        hipStreamWaitEvent(m.stream, m.lane_ev[k], 0) != hipSuccess)
      rc = rc ? rc : set_error(LLMHIP_ERR_DEVICE, "llm: prefill: lane join failed");
  m.last_row = (n - 1) % m.pm;
  return rc;
}

static PassMat pass_mat(const QMat& q) {
  PassMat p;
  p.qs = q.qs;
  p.type = q.g.q.type;
  p.rows = (uint32_t)q.g.rows;
  p.nb = q.g.nb;
  p.ng = q.g.ng;
  p.tail = q.g.tail;
  p.tiles = (uint32_t)q.g.tiles;
  p.map = q.map;
  p.map_hd = q.map_hd;
  p.map_seg0 = q.map_seg0;
  p.map_seg1 = q.map_seg1;
  p.ff = q.ff;
  return p;
}

// Whether the model fits the fused decode pass, and its layer table and
// arguments (at finalize, when every matrix is in place).
static int pass_setup(Model& m) {
  const llmhip_config& c = m.cfg;
  m.pass_ok = false;
  m.pgrid = pass_grid(m.device, (uint32_t)c.head_dim, m.kv16);
  std::vector<PassLayer> tab((size_t)c.layers);
  uint32_t kp = 1;
  m.pass_q8 = false;
  m.pass_why.clear();
  for (int l = 0; l < c.layers && m.pass_why.empty(); l++) {
    const Layer& L = m.layers[(size_t)l];
    if (L.nqkv != 1 || L.ngu != 1) {
      m.pass_why = "q, k, v or gate, up of different types";
      break;
    }
    PassLayer& p = tab[(size_t)l];
    p.qkv = pass_mat(L.qkv[0]);
    p.o = pass_mat(L.o);
    p.gu = pass_mat(L.gu[0]);
    p.down = pass_mat(L.down);
    p.attn_norm = L.attn_norm;
    p.ffn_norm = L.ffn_norm;
    p.bias = L.bias;
    p.kv = L.kv;
    for (const PassMat* q : {&p.qkv, &p.o, &p.gu, &p.down}) m.pass_q8 = m.pass_q8 || q->type == LLMHIP_Q8_0;
    if (const char* why = pass_unfit(c, m.kvd, p.qkv, p.o, p.gu, p.down, m.pgrid, &kp)) m.pass_why = why;
  }
  if (!m.pass_why.empty()) return 0;
  LLM_HIP(hipMemcpyAsync(m.ptab, tab.data(), tab.size() * sizeof(PassLayer), hipMemcpyHostToDevice, m.stream));
  LLM_HIP(hipStreamSynchronize(m.stream));
  PassArgs& a = m.pargs;
  memset(&a, 0, sizeof a);
  const uint64_t E = c.embd, F = c.ff;
  a.layers = m.ptab;
  a.nlayers = (uint32_t)c.layers;
  a.xn = m.xn;
  a.x = m.x;
  a.q = m.q;
  a.att = m.att;
  a.act = m.act;
  a.up = m.gbuf;
  a.np = pass_partials(c, m.ctx);
  a.llq = m.ll;                                        // [E + 2 kvd]
  a.llo = a.llq + E + 2ull * m.kvd;                    // [np][E], [np][heads][16], then [E]
  a.llb = a.llo + a.np * (E + 16ull * c.heads) + E;    // [1 + kp][E]
  a.llact = a.llb + (1 + kp) * E;                      // [pass_act_words(ff)]
  (void)F;
  a.kp = kp;
  a.ctrl = m.pctrl;
  a.state = m.state;
  a.cs = m.cs;
  a.embd = (uint32_t)c.embd;
  a.ff = (uint32_t)c.ff;
  a.heads = (uint32_t)c.heads;
  a.kv_heads = (uint32_t)c.kv_heads;
  a.hd = (uint32_t)c.head_dim;
  a.kvd = m.kvd;
  a.ctx = m.ctx;
  a.neox = (uint32_t)c.rope_neox;
  a.kv16 = m.kv16 ? 1 : 0;
  a.eps = c.eps;
  a.scale = (float)(1 / std::sqrt((double)c.head_dim));  // cpu.go:304
  const uint32_t t1 = (uint32_t)(E + 2 * m.kvd + 15) / 16, t3 = (uint32_t)(E + 15) / 16;
  pass_place(&a, m.pgrid, t1, t3, t3);
  m.pass_ok = true;
  return 0;
}

}  // namespace llmhip

using namespace llmhip;

struct llmhip_model {
  Model* m;
};

extern "C" {

int llmhip_model_create(int ordinal, const llmhip_limits* lim, const llmhip_config* cfg, int ctx, int prefill_batch,
                        llmhip_model** out) {
  clear_error();
  *out = nullptr;
  const llmhip_config& c = *cfg;
  if (c.layers <= 0 || c.embd <= 0 || c.ff <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.vocab <= 0 ||
      c.embd % c.heads != 0 || c.heads % c.kv_heads != 0 || c.head_dim != c.embd / c.heads)
    return set_error(LLMHIP_ERR_FORMAT, "llm: implausible hyperparameters");
  if (c.embd % 32 != 0 || c.ff % 32 != 0)
    return set_error(LLMHIP_ERR_FORMAT, "llm: embedding %d and feed-forward %d must be multiples of 32", c.embd, c.ff);
  if (!attn_ok((uint32_t)c.head_dim))
    return set_error(LLMHIP_ERR_FORMAT, "llm: head size %d is not supported (64 or 128)", c.head_dim);
  Model* m = new Model();
  m->device = ordinal;
  m->cfg = c;
  if (lim) m->lim = *lim;
  else if (llmhip_device_limits(ordinal, &m->lim) != 0) {
    delete m;
    return LLMHIP_ERR_DEVICE;
  }
  int cx = ctx;
  if (cx <= 0 || cx > c.ctx) cx = c.ctx;  // gpu.go:470-472
  if (cx <= 0) {
    delete m;
    return set_error(LLMHIP_ERR_FORMAT, "llm: context length %d", cx);
  }
  m->ctx = (uint32_t)cx;
  m->pm = prefill_batch > 0 ? (uint32_t)std::min(prefill_batch, 64) : 64;
  m->kvd = (uint32_t)(c.kv_heads * c.head_dim);
  m->smax = (m->ctx + ATTN_SPLIT_ROWS - 1) / ATTN_SPLIT_ROWS;
  auto fail = [&](int rc) {
    model_destroy(m);
    return rc;
  };
  if (hipSetDevice(ordinal) != hipSuccess) return fail(set_error(LLMHIP_ERR_DEVICE, "llm: no GPU %d", ordinal));
  if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess)
    return fail(set_error(LLMHIP_ERR_DEVICE, "llm: hipStreamCreate failed"));
  int rc;
  const uint64_t E = c.embd, F = c.ff, V = c.vocab, pm = m->pm, H = c.heads;
  if ((rc = dalloc_n(*m, &m->x, pm * E)) || (rc = dalloc_n(*m, &m->q, pm * E)) || (rc = dalloc_n(*m, &m->att, pm * E)) ||
      (rc = dalloc_n(*m, &m->act, pm * F)) || (rc = dalloc_n(*m, &m->gbuf, pm * F)) ||
      (rc = dalloc_n(*m, &m->logits, V)) || (rc = dalloc_n(*m, &m->amax_v, V / 16 + 64)) ||
      (rc = dalloc_n(*m, &m->amax_i, V / 16 + 64)) || (rc = dalloc_n(*m, &m->pv, pm * H * m->smax * c.head_dim)) ||
      (rc = dalloc_n(*m, &m->ml, pm * H * m->smax * 2)) || (rc = dalloc_n(*m, &m->state, 2)) ||
      (rc = dalloc_n(*m, &m->tokens, (uint64_t)m->ctx + 1)) || (rc = dalloc_n(*m, &m->outb, 1)) ||
      (rc = dalloc(*m, &m->xprep, xprep_bytes(m->pm, (uint32_t)std::max(c.embd, c.ff)))) ||
      (rc = dalloc(*m, &m->xprep2, xprep_bytes(m->pm, (uint32_t)c.ff))) ||
      (rc = dalloc_n(*m, &m->cs, (uint64_t)m->ctx * c.head_dim)) || (rc = dalloc_n(*m, &m->h, E)) ||
      (rc = dalloc_n(*m, &m->xn, E)) || (rc = dalloc_n(*m, &m->kpart, 3 * E)) ||
      (rc = dalloc_n(*m, &m->ll, pass_words(c, m->kvd, pass_partials(c, m->ctx)))) || (rc = dalloc_n(*m, &m->pctrl, 4)) ||
      (rc = dalloc_n(*m, &m->ptab, (uint64_t)c.layers)))
    return fail(rc);
  {  // the prefill lanes: lane 0 is the model's own buffers
    m->lanes[0] = Lane{m->stream, m->x, m->q, m->att, m->act, m->gbuf, m->pv, m->ml, m->xprep, m->state, m->xprep2};
    for (int k = 1; k < LANES; k++) {
      Lane& a = m->lanes[k];
      if (hipStreamCreateWithFlags(&a.stream, hipStreamNonBlocking) != hipSuccess)
        return fail(set_error(LLMHIP_ERR_DEVICE, "llm: hipStreamCreate failed"));
      if ((rc = dalloc_n(*m, &a.x, pm * E)) || (rc = dalloc_n(*m, &a.q, pm * E)) ||
          (rc = dalloc_n(*m, &a.att, pm * E)) || (rc = dalloc_n(*m, &a.act, pm * F)) ||
          (rc = dalloc_n(*m, &a.gbuf, pm * F)) || (rc = dalloc_n(*m, &a.pv, pm * H * m->smax * c.head_dim)) ||
          (rc = dalloc_n(*m, &a.ml, pm * H * m->smax * 2)) ||
          (rc = dalloc(*m, &a.xprep, xprep_bytes(m->pm, (uint32_t)std::max(c.embd, c.ff)))) ||
          (rc = dalloc_n(*m, &a.state, 2)) ||
          (rc = dalloc(*m, &a.xprep2, xprep_bytes(m->pm, (uint32_t)c.ff))))
        return fail(rc);
    }
    for (hipEvent_t& e : m->lane_ev)
      if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess)
        return fail(set_error(LLMHIP_ERR_DEVICE, "llm: hipEventCreate failed"));
    for (auto& v : m->seg_done) {
      v.resize((size_t)c.layers + 1);
      for (hipEvent_t& e : v)
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess)
          return fail(set_error(LLMHIP_ERR_DEVICE, "llm: hipEventCreate failed"));
    }
  }
  // RoPE table in double precision, gpu.go:524-534 (and cpu.go:374-375)
  std::vector<float> cs((size_t)m->ctx * c.head_dim);
  const int hp = c.head_dim / 2;
  for (uint32_t p = 0; p < m->ctx; p++)
    for (int i = 0; i < hp; i++) {
      double theta = (double)p * std::pow((double)c.rope_base, -(double)(2 * i) / (double)c.head_dim);
      double sn, co;
      sincos(theta, &sn, &co);
      cs[((size_t)p * hp + i) * 2] = (float)co;
      cs[((size_t)p * hp + i) * 2 + 1] = (float)sn;
    }
  m->host_cap = std::max<uint32_t>(m->ctx + 1, 64);
  if (hipHostMalloc((void**)&m->host, (size_t)m->host_cap * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc((void**)&m->bounce, BOUNCE_BYTES, hipHostMallocDefault) != hipSuccess)
    return fail(set_error(LLMHIP_ERR_DEVICE, "llm: hipHostMalloc failed"));
  if ((rc = copy_in(*m, m->cs, cs.data(), cs.size() * 4)) != 0) return fail(rc);
  const uint32_t ctrl0[4] = {1, 0, 0, 0};  // epoch 1: no word of the zeroed vectors carries a flag of a pass
  if ((rc = copy_in(*m, m->pctrl, ctrl0, sizeof ctrl0)) != 0) return fail(rc);
  *out = new llmhip_model{m};
  return 0;
}

int llmhip_model_tensor(llmhip_model* h, const char* name, uint32_t type, const uint64_t* dims, uint32_t ndims) {
  clear_error();
  Model& m = *h->m;
  if (m.allocated) return set_error(LLMHIP_ERR_STATE, "llm: tensor %s declared after the first upload", name);
  bool quant;
  std::vector<uint64_t> want;
  TensorInfo t;
  t.type = type;
  t.dims.assign(dims, dims + ndims);
  if (!expected(m, name, &quant, &want)) {
    t.used = false;
    m.tensors[name] = t;
    return 0;
  }
  t.used = true;
  if (t.dims != want) {
    std::string got, exp;
    for (auto d : t.dims) got += std::to_string(d) + " ";
    for (auto d : want) exp += std::to_string(d) + " ";
    return set_error(LLMHIP_ERR_FORMAT, "llm: tensor %s has dims [%s], want [%s]", name, got.c_str(), exp.c_str());
  }
  uint64_t elems = 1;
  for (auto d : t.dims) elems *= d;
  if (quant) {
    QType q;
    if (!qtype_of(type, &q))
      return set_error(LLMHIP_ERR_TYPE, "llm: tensor %s has ggml type %u, which has no GPU kernel yet (Q4_0, Q4_1, Q8_0)",
                       name, type);
    t.size = elems / 32 * q.block_bytes;
  } else {
    if (type != LLMHIP_F32) return set_error(LLMHIP_ERR_FORMAT, "llm: tensor %s missing or not F32", name);
    t.size = elems * 4;
  }
  m.tensors[name] = t;
  return 0;
}

}  // extern "C"

// Staging of one load (a model's uploads, then freed at finalize).
constexpr uint64_t MODEL_STAGE_BYTES = 8ull << 20;

static int upload_from(Model& m, const char* name, const Source& src, uint64_t nbytes, uint64_t off) {
  auto it = m.tensors.find(name);
  if (it == m.tensors.end()) return set_error(LLMHIP_ERR_ARG, "llm: tensor %s was not declared", name);
  TensorInfo& t = it->second;
  if (!t.used) return 0;
  if (!m.allocated) LLM_TRY(allocate(m));
  if (off + nbytes > t.size)
    return set_error(LLMHIP_ERR_ARG, "llm: upload of %s runs past its %llu bytes", name, (unsigned long long)t.size);
  LLM_TRY(check_range(t, name, off, nbytes));
  QMat* q;
  uint64_t row_off;
  float* f;
  LLM_TRY(route(m, name, &q, &row_off, &f));
  LLM_HIP(hipSetDevice(m.device));
  if (!q && (off % 4 || nbytes % 4))
    return set_error(LLMHIP_ERR_ARG, "llm: F32 upload of %s not whole floats", name);
  if (!m.st.cap) LLM_TRY(stager_init(&m.st, m.device, MODEL_STAGE_BYTES, m.stream));
  if (q)
    LLM_TRY(qmat_upload(&m.st, *q, src, nbytes, off, row_off));
  else
    LLM_TRY(f32_upload(&m.st, f, src, nbytes, off));
  add_range(t, off, nbytes);
  return 0;
}

extern "C" {

int llmhip_model_upload(llmhip_model* h, const char* name, const void* raw, uint64_t nbytes, uint64_t off) {
  clear_error();
  Source src;
  src.mem = (const uint8_t*)raw;
  return upload_from(*h->m, name, src, nbytes, off);
}

int llmhip_model_upload_file_tensors(llmhip_model* h, int fd, uint32_t n, const char* const* names,
                                     const uint64_t* file_offsets) {
  clear_error();
  Model& m = *h->m;
  if (fd < 0) return set_error(LLMHIP_ERR_ARG, "llm: upload from a bad file descriptor");
  std::vector<StagePiece> ps;
  std::vector<TensorInfo*> owner;
  for (uint32_t i = 0; i < n; i++) {
    auto it = m.tensors.find(names[i]);
    if (it == m.tensors.end()) return set_error(LLMHIP_ERR_ARG, "llm: tensor %s was not declared", names[i]);
    TensorInfo& t = it->second;
    if (!t.used) continue;
    LLM_TRY(check_range(t, names[i], 0, t.size));
    for (uint32_t j = 0; j < i; j++)
      if (strcmp(names[j], names[i]) == 0)
        return set_error(LLMHIP_ERR_ARG, "llm: tensor %s listed twice in one upload", names[i]);
    if (!m.allocated) LLM_TRY(allocate(m));
    StagePiece p{};
    QMat* q;
    LLM_TRY(route(m, names[i], &q, &p.row_off, &p.f));
    p.q = q;
    uint64_t per = p.q ? MODEL_STAGE_BYTES / p.q->g.q.block_bytes * p.q->g.q.block_bytes : MODEL_STAGE_BYTES;
    for (uint64_t a = 0; a < t.size; a += per) {
      p.off = a;
      p.bytes = std::min(per, t.size - a);
      p.file = file_offsets[i] + a;
      ps.push_back(p);
      owner.push_back(&t);
    }
  }
  std::vector<size_t> order(ps.size());
  for (size_t i = 0; i < order.size(); i++) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return ps[a].file < ps[b].file; });
  std::vector<StagePiece> sorted;
  for (size_t i : order) sorted.push_back(ps[i]);
  if (!m.allocated) LLM_TRY(allocate(m));
  LLM_HIP(hipSetDevice(m.device));
  if (!m.st.cap) LLM_TRY(stager_init(&m.st, m.device, MODEL_STAGE_BYTES, m.stream));
  LLM_TRY(stage_file_runs(&m.st, fd, sorted.data(), sorted.size()));
  for (size_t i = 0; i < ps.size(); i++) add_range(*owner[i], ps[i].off, ps[i].bytes);
  return 0;
}

int llmhip_model_upload_file(llmhip_model* h, const char* name, int fd, uint64_t file_offset, uint64_t nbytes,
                             uint64_t off) {
  clear_error();
  if (fd < 0) return set_error(LLMHIP_ERR_ARG, "llm: upload of %s from a bad file descriptor", name);
  Source src;
  src.fd = fd;
  src.file_off = file_offset;
  return upload_from(*h->m, name, src, nbytes, off);
}

int llmhip_model_finalize(llmhip_model* h) {
  clear_error();
  Model& m = *h->m;
  if (!m.allocated) LLM_TRY(allocate(m));
  // every used tensor covered in full: its uploads are disjoint, so the bytes
  // received count each byte once
  for (auto& kv : m.tensors)
    if (kv.second.used && kv.second.received < kv.second.size)
      return set_error(LLMHIP_ERR_FORMAT, "llm: tensor %s: %llu of %llu bytes uploaded", kv.first.c_str(),
                       (unsigned long long)kv.second.received, (unsigned long long)kv.second.size);
  LLM_HIP(hipStreamSynchronize(m.stream));
  stager_free(&m.st);  // the load is over: release its pinned and device staging
  LLM_TRY(pass_setup(m));
  m.stats.submits++;
  m.finalized = true;
  return 0;
}

int llmhip_model_prefill(llmhip_model* h, const int32_t* ids, int n, float* logits, int32_t* first) {
  clear_error();
  Model& m = *h->m;
  if (!m.finalized) return set_error(LLMHIP_ERR_STATE, "llm: model not finalized");
  if (n <= 0) return set_error(LLMHIP_ERR_ARG, "llm: empty prompt");
  if ((uint32_t)n > m.ctx) return set_error(LLMHIP_ERR_CONTEXT, "llm: prompt longer than the context");
  for (int i = 0; i < n; i++)
    if (ids[i] < 0 || ids[i] >= m.cfg.vocab)
      return set_error(LLMHIP_ERR_ARG, "llm: token id %d outside the vocabulary of %d", ids[i], m.cfg.vocab);
  LLM_HIP(hipSetDevice(m.device));
  // begin (gpu.go:839-847): the prompt into tokens[0:], state = (0, 0) (a
  // kernel on the stream rather than a second copy, so nothing waits on the
  // host in between; the wavefront sets every chunk's state itself)
  LLM_HIP(hipStreamSynchronize(m.stream));
  memcpy(m.host, ids, (size_t)n * 4);
  LLM_HIP(hipMemcpyAsync(m.tokens, m.host, (size_t)n * 4, hipMemcpyHostToDevice, m.stream));
  bool full = m.layers_limit == 0 || m.layers_limit >= m.cfg.layers;
  if ((uint32_t)n > m.pm && prefill_lanes() > 1) {
    LLM_TRY(prefill_wavefront(m, (uint32_t)n));
  } else {
    LLM_TRY(set_state_launch(m.state, 0, m.stream));
    for (int a = 0; a < n; a += (int)m.pm) {
      int b = std::min(a + (int)m.pm, n);
      LLM_TRY(launch_graph(m, (uint32_t)a, (uint32_t)(b - a), b == n, true));
      m.stats.submits++;
    }
  }
  m.pos = (uint32_t)n;
  m.prompted = full;
  LLM_HIP(hipMemcpyAsync(m.host, m.tokens + n, 4, hipMemcpyDeviceToHost, m.stream));
  LLM_HIP(hipStreamSynchronize(m.stream));
  if (first) *first = m.host[0];
  if (logits) LLM_TRY(copy_out(m, logits, m.logits, (uint64_t)m.cfg.vocab * 4));
  m.stats.tokens += n;
  return 0;
}

int llmhip_model_decode(llmhip_model* h, int cnt, int32_t* out) {
  clear_error();
  Model& m = *h->m;
  if (!m.prompted) return set_error(LLMHIP_ERR_STATE, "llm: decode before a prompt");
  if (cnt <= 0) return 0;
  if (m.pos + (uint32_t)cnt > m.ctx)
    return set_error(LLMHIP_ERR_CONTEXT, "llm: %d more tokens exceed the context of %u at position %u", cnt, m.ctx,
                     m.pos);
  LLM_HIP(hipSetDevice(m.device));
  uint32_t first = m.pos;
  // four passes per graph (measured, decode tok/s at configs 4 / 3: one 1514 / 1751, two 1510 / 1759,
  // four 1508 / 1762, eight 1476 / 1765)
  for (int j = 0; j < cnt; j += 4) LLM_TRY(launch_decode(m, first + (uint32_t)j, (uint32_t)std::min(cnt - j, 4)));
  LLM_HIP(hipMemcpyAsync(m.host, m.tokens + first + 1, (size_t)cnt * 4, hipMemcpyDeviceToHost, m.stream));
  LLM_HIP(hipMemcpyAsync(m.host + cnt, m.pctrl + 1, 4, hipMemcpyDeviceToHost, m.stream));
  LLM_HIP(hipStreamSynchronize(m.stream));
  if (m.host[cnt] != 0) {
    // a fused pass gave up waiting: its results are not to be trusted; later
    // decode steps take one launch per kernel
    const uint32_t zero = 0;
    LLM_TRY(copy_in(m, m.pctrl + 1, &zero, 4));
    m.pass_ok = false;
    m.pass_why = "a hand-off wait timed out";
    destroy_graphs(m);
    return set_error(LLMHIP_ERR_DEVICE,
                     "llm: decode: %d waits of the fused pass timed out (later decode steps take one launch per kernel)",
                     m.host[cnt]);
  }
  memcpy(out, m.host, (size_t)cnt * 4);
  m.pos += (uint32_t)cnt;
  m.stats.submits++;
  m.stats.tokens += cnt;
  return 0;
}

int llmhip_model_peek(llmhip_model* h, const char* name, float* out, uint64_t n) {
  clear_error();
  Model& m = *h->m;
  const void* src = nullptr;
  uint64_t cap = 0;
  std::string s = name;
  const uint64_t E = m.cfg.embd, F = m.cfg.ff;
  bool kv_row = false;  // src is an element offset into a cache of binary16 or f32 values
  if (s == "x") { src = m.x; cap = m.pm * E; }
  else if (s == "q") { src = m.q; cap = m.pm * E; }
  else if (s == "att") { src = m.att; cap = m.pm * E; }
  else if (s == "gate" || s == "act") { src = m.act; cap = m.pm * F; }
  else if (s == "up") { src = m.gbuf; cap = m.pm * F; }
  else if (s == "h") {
    // the head's input (recordHead's rms, fused.go:269-275): RMSNorm of the
    // last token's residual row with output_norm, formed here from x
    if (!m.allocated) return set_error(LLMHIP_ERR_STATE, "llm: no buffer \"h\" before the weights are loaded");
    LLM_HIP(hipSetDevice(m.device));
    LLM_TRY(rmsnorm_launch(m.x + (uint64_t)m.last_row * E, m.out_norm, (uint32_t)E, m.cfg.eps, m.h, m.stream));
    src = m.h;
    cap = E;
  } else if (s == "k" || s == "v") {
    // the K or V row the latest pass appended last: the last layer run, the
    // last position (as stored in the cache: K after bias and RoPE)
    const int nl = m.layers_limit > 0 && m.layers_limit < m.cfg.layers ? m.layers_limit : m.cfg.layers;
    if (m.allocated && m.pos > 0 && nl > 0) {
      src = (const void*)(uintptr_t)(((uint64_t)(s == "v") * m.ctx + (m.pos - 1)) * m.kvd);
      kv_row = true;
      cap = m.kvd;
    }
  }
  else if (s == "logits") { src = m.logits; cap = m.cfg.vocab; }
  else if (s == "state") { src = m.state; cap = 2; }
  else if (s == "tokens") { src = m.tokens; cap = m.ctx + 1; }
  else if (s == "outb") { src = m.outb; cap = 1; }
  else if (s.rfind("kvblk.", 0) == 0) {
    int l = atoi(s.c_str() + 6);
    if (l >= 0 && l < m.cfg.layers && m.allocated) {
      src = m.layers[l].kv;
      cap = 2ull * m.ctx * m.kvd;
    }
  }
  if (!src && !kv_row) return set_error(LLMHIP_ERR_ARG, "llm: no buffer \"%s\"", name);
  if (n > cap) return set_error(LLMHIP_ERR_ARG, "llm: buffer \"%s\" holds %llu words", name, (unsigned long long)cap);
  LLM_HIP(hipSetDevice(m.device));
  LLM_HIP(hipStreamSynchronize(m.stream));
  if (kv_row) {  // src: the row's element offset in the last layer's cache
    const int nl = m.layers_limit > 0 && m.layers_limit < m.cfg.layers ? m.layers_limit : m.cfg.layers;
    const uint64_t e = (uint64_t)(uintptr_t)src;
    const char* kv = (const char*)m.layers[nl - 1].kv;
    if (m.kv16) {
      std::vector<_Float16> hv(n);
      LLM_TRY(copy_out(m, hv.data(), kv + e * 2, n * 2));
      for (uint64_t i = 0; i < n; i++) out[i] = (float)hv[i];
    } else {
      LLM_TRY(copy_out(m, out, kv + e * 4, n * 4));
    }
  } else if (m.kv16 && s.rfind("kvblk.", 0) == 0) {  // binary16 cache: widened on the host
    std::vector<_Float16> h(n);
    LLM_TRY(copy_out(m, h.data(), src, n * 2));
    for (uint64_t i = 0; i < n; i++) out[i] = (float)h[i];
  } else {
    LLM_TRY(copy_out(m, out, src, n * 4));
  }
  m.stats.submits++;
  return 0;
}

uint64_t llmhip_model_memory_used(const llmhip_model* h) { return h->m->used; }

int llmhip_model_stats(const llmhip_model* h, llmhip_stats* out) {
  *out = h->m->stats;
  return 0;
}

int llmhip_model_config(const llmhip_model* h, llmhip_config* out, int* ctx) {
  *out = h->m->cfg;
  if (ctx) *ctx = (int)h->m->ctx;
  return 0;
}

int llmhip_model_set_kv_f16(llmhip_model* h, int on) {
  clear_error();
  Model& m = *h->m;
  if (m.allocated) return set_error(LLMHIP_ERR_STATE, "llm: the KV cache format is fixed once tensors are uploaded");
  if (m.q8 && !on) return set_error(LLMHIP_ERR_STATE, "llm: the ExactGGML mode keeps a binary16 KV cache");
  m.kv16 = on != 0;
  return 0;
}

int llmhip_model_set_exact_ggml(llmhip_model* h, int on) {
  clear_error();
  Model& m = *h->m;
  if (m.allocated) return set_error(LLMHIP_ERR_STATE, "llm: the ExactGGML mode is fixed once tensors are uploaded");
  m.q8 = on != 0;
  if (m.q8) m.kv16 = true;  // cpu.go:298: ExactGGML stores K and V in binary16
  destroy_graphs(m);
  return 0;
}

int llmhip_model_set_fused(llmhip_model* h, int on, uint32_t poll_limit, char* why, uint64_t cap) {
  clear_error();
  Model& m = *h->m;
  LLM_HIP(hipSetDevice(m.device));
  LLM_HIP(hipStreamSynchronize(m.stream));
  if (m.pass_on != (on != 0)) destroy_graphs(m);
  m.pass_on = on != 0;
  LLM_TRY(copy_in(m, m.pctrl + 2, &poll_limit, 4));
  const bool taken = m.pass_ok && m.pass_on;
  if (why && cap) {
    const std::string w = taken ? "" : !m.pass_on ? "turned off" : m.pass_why;
    const size_t n = std::min<size_t>(w.size(), cap - 1);
    memcpy(why, w.data(), n);
    why[n] = 0;
  }
  return taken ? 1 : 0;
}

int llmhip_model_set_layers(llmhip_model* h, int layers) {
  clear_error();
  Model& m = *h->m;
  (void)hipStreamSynchronize(m.stream);
  if (m.layers_limit != layers) destroy_graphs(m);
  m.layers_limit = layers;
  return 0;
}

int llmhip_model_set_skip(llmhip_model* h, const char* classes) {
  clear_error();
  Model& m = *h->m;
  (void)hipStreamSynchronize(m.stream);
  std::set<std::string> s;
  std::string c = classes ? classes : "";
  size_t a = 0;
  while (a <= c.size()) {
    size_t b = c.find(',', a);
    if (b == std::string::npos) b = c.size();
    if (b > a) s.insert(c.substr(a, b - a));
    a = b + 1;
  }
  if (s != m.skip) destroy_graphs(m);
  m.skip = s;
  return 0;
}

int llmhip_model_bench_kernel(llmhip_model* h, const char* kernel, int iters, float* avg_us, uint64_t* bytes) {
  clear_error();
  Model& m = *h->m;
  if (!m.finalized) return set_error(LLMHIP_ERR_STATE, "llm: model not finalized");
  if (iters < 1) return set_error(LLMHIP_ERR_ARG, "llm: iters %d", iters);
  LLM_HIP(hipSetDevice(m.device));
  const std::string k = kernel;
  if (k != "head" && k != "k1" && k != "k2" && k != "k3" && k != "k4" && k != "k5")
    return set_error(LLMHIP_ERR_ARG, "llm: no kernel \"%s\" (head, k1..k5)", kernel);
  std::set<std::string> saved = m.skip;
  m.skip.clear();
  attn_plan(m, m.pos, 1);  // the variant the next decode step runs
  const int L = m.cfg.layers;
  auto wb = [](const QMat& q) { return q.g.gguf_bytes(); };
  // launch i runs layer i % L: consecutive launches read different weights,
  // as in the decode pass
  auto one = [&](int i) -> int {
    const Layer& ly = m.layers[i % L];
    m.cur_layer = i % L;
    if (k == "head") {  // the decode head kernel without the sampling kernel, which advances the state
      const QMat& w = m.tied ? m.embd : m.out;
      return gemv_launch(head_args(m, 0, 0), w.g.q.type, PRO_RMS | (m.q8 ? PRO_Q8 : 0), EPI_ARGMAX, m.stream);
    }
    if (k == "k1") {  // as in the pass: after layer 0 the previous down projection's halves are added
      m.k5_split = i % L > 0 && m.cfg.embd <= 2048 && !m.q8;
      const int rc1 = rec_k1(m, ly, 1);
      m.xsum_ready = false;
      return rc1;
    }
    if (k == "k2") return rec_k2(m, ly, 1);
    if (k == "k3") return rec_k3(m, ly, 1);
    if (k == "k4") return rec_k4(m, ly, 1);
    const int rc5 = rec_k5(m, ly, 1, i % L < L - 1);  // as in the pass: halves but for the last layer
    m.k5_split = false;
    return rc5;
  };
  uint64_t b = 0;
  const Layer& L0 = m.layers[0];
  if (k == "head") b = wb(m.tied ? m.embd : m.out);
  else if (k == "k1") b = wb(L0.qkv[0]) + (L0.nqkv == 3 ? wb(L0.qkv[1]) + wb(L0.qkv[2]) : 0);
  else if (k == "k2") b = 2ull * (m.pos + 1) * m.kvd * (m.kv16 ? 2 : 4);
  else if (k == "k3") b = wb(L0.o);
  else if (k == "k4") b = wb(L0.gu[0]) + (L0.ngu == 2 ? wb(L0.gu[1]) : 0);
  else b = wb(L0.down);
  int rc = 0;
  for (int i = 0; i < L && rc == 0; i++) rc = one(i);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (rc == 0 && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
    rc = set_error(LLMHIP_ERR_DEVICE, "llm: hipEventCreate failed");
  if (rc == 0 && hipEventRecord(e0, m.stream) != hipSuccess) rc = set_error(LLMHIP_ERR_DEVICE, "llm: event record");
  for (int i = 0; i < iters && rc == 0; i++) rc = one(i);
  if (rc == 0 && hipEventRecord(e1, m.stream) != hipSuccess) rc = set_error(LLMHIP_ERR_DEVICE, "llm: event record");
  float ms = 0;
  if (rc == 0 && hipEventSynchronize(e1) == hipSuccess) (void)hipEventElapsedTime(&ms, e0, e1);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  m.skip = saved;
  m.cur_layer = -1;
  if (rc) return rc;
  *avg_us = ms * 1000.f / (float)iters;
  if (bytes) *bytes = b;
  return 0;
}

int llmhip_model_profile(llmhip_model* h, int tokens, llmhip_kernel_time* out, int cap, int* n) {
  clear_error();
  Model& m = *h->m;
  *n = 0;
  if (!m.prompted) return set_error(LLMHIP_ERR_STATE, "llm: profile before a prompt");
  if (tokens < 1 || m.pos + (uint32_t)tokens > m.ctx)
    return set_error(LLMHIP_ERR_CONTEXT, "llm: %d profiled tokens exceed the context", tokens);
  LLM_HIP(hipSetDevice(m.device));
  LLM_HIP(hipStreamSynchronize(m.stream));
  int rc = 0;
  for (int t = 0; t < tokens && rc == 0; t++) {
    std::vector<ProfRec> recs;
    m.prof = &recs;
    attn_plan(m, m.pos, 1);
    rc = record_pass(m, 1, true, false);
    m.prof = nullptr;
    if (hipStreamSynchronize(m.stream) != hipSuccess && rc == 0)
      rc = set_error(LLMHIP_ERR_DEVICE, "llm: profile step failed");
    if (rc == 0) {
      m.pos++;
      m.stats.tokens++;
      m.stats.dispatches += (int64_t)recs.size();
      m.stats.submits++;
    }
    if (rc == 0 && t == tokens - 1) {
      int k = 0;
      for (auto& r : recs) {
        if (k >= cap) break;
        llmhip_kernel_time& o = out[k++];
        memset(o.cls, 0, sizeof o.cls);
        strncpy(o.cls, r.cls, sizeof o.cls - 1);
        o.layer = r.layer;
        o.bytes = r.bytes;
        float ms = 0;
        (void)hipEventElapsedTime(&ms, r.a, r.b);
        o.us = ms * 1000.f;
      }
      *n = k;
    }
    for (auto& r : recs) {
      if (r.a) (void)hipEventDestroy(r.a);
      if (r.b) (void)hipEventDestroy(r.b);
    }
  }
  return rc;
}

void llmhip_model_free(llmhip_model* h) {
  if (!h) return;
  model_destroy(h->m);
  delete h;
}

}  // extern "C"
