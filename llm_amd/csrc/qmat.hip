// Host side of the quantised matrices: allocation, staged upload with
// the repack on the device, dispatch of the typed kernels, and the
// llmhip_qmat_* / llmhip_device_* entry points.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "gemv.h"

namespace llmhip {

int qmat_place(QMat* m, int device, uint32_t type, uint64_t rows, uint64_t k, uint8_t* mem) {
  QType q;
  if (!qtype_of(type, &q))
    return set_error(LLMHIP_ERR_TYPE, "llm: ggml type %u has no GPU kernel (Q4_0, Q4_1, Q8_0)", type);
  if (rows == 0 || k == 0 || k % 32 != 0 || rows > (1u << 31) || k > (1u << 20))
    return set_error(LLMHIP_ERR_ARG, "llm: a [%llu][%llu] quantised matrix is not supported (k a multiple of 32)",
                     (unsigned long long)rows, (unsigned long long)k);
  m->device = device;
  m->g = make_geom(q, rows, k);
  m->qs = mem;
  m->owned = false;
  m->bytes = m->g.dev_bytes();
  return 0;
}

int qmat_alloc(QMat* m, int device, uint32_t type, uint64_t rows, uint64_t k) {
  LLM_TRY(qmat_place(m, device, type, rows, k, nullptr));
  LLM_HIP(hipSetDevice(device));
  LLM_HIP(hipMalloc(&m->qs, m->bytes));
  m->owned = true;
  // padding rows of the last tile must read as zero weights
  LLM_HIP(hipMemset(m->qs, 0, m->bytes));
  return 0;
}

void qmat_release(QMat* m) {
  if (m->qs && m->owned) (void)hipFree(m->qs);
  m->qs = nullptr;
  m->owned = false;
}

void gemv_bind(GemvArgs* a, const QMat& m) {
  a->qs = m.qs;
  a->rows = (uint32_t)m.g.rows;
  a->nb = m.g.nb;
  a->ng = m.g.ng;
  a->tail = m.g.tail;
  a->tiles = (uint32_t)m.g.tiles;
  a->k = (uint32_t)m.g.k;
  a->map = m.map;
  a->map_hd = m.map_hd;
  a->map_seg0 = m.map_seg0;
  a->map_seg1 = m.map_seg1;
  a->ff = m.ff;
  gemv_pick(a->tiles, a->ng, a->tail, a->nb, &a->split, &a->waves);
  gemv_pick_stream(a->tiles, a->nb, &a->stream, &a->swaves);
}

void gemv_pick_stream(uint32_t tiles, uint32_t nb, uint32_t* wgs, uint32_t* waves) {
  *wgs = 0;
  *waves = 4;
  if (tiles < GEMV_STREAM_MIN_TILES || nb % 4) return;  // tail blocks: the tile kernel
  uint32_t w = 4;  // the prologue stages at most two 8-element items per thread
  while (w < 8 && nb * 4 > 2 * 64 * w) w *= 2;
  if (nb * 4 > 2 * 64 * w) return;  // k > 8192: the tile kernel
  // about 16 waves per CU (4 per SIMD), each streaming several tiles; at
  // nb == 28 (k = 896) each wave keeps a whole tile in flight and the
  // activations in registers, which leaves room for 8 waves per CU
  const uint32_t total = nb == 28 ? 2048u : 4096u;
  *wgs = std::min((tiles + w - 1) / w, total / w);
  *waves = w;
}

void gemv_pick(uint32_t tiles, uint32_t ng, uint32_t tail, uint32_t nb, uint32_t* split, uint32_t* waves) {
  // Aim for >= 2048 waves (8 per CU) so the loads of small matrices are all
  // in flight at once: split a tile's block groups over up to 16 waves, each
  // keeping at least one group.
  uint32_t groups = ng + (tail ? 1 : 0), s = 1;
  while (s < 16 && tiles * s < 2048 && 2 * s <= groups) s *= 2;
  // the prologue stages at most two 8-element items per thread
  uint32_t w = 4;
  while (w < 16 && (w < s || nb * 4 > 2 * 64 * w)) w *= 2;
  *split = s;
  *waves = w;
}

uint32_t gemv_groups(const GemvArgs& a) {
  if (a.stream && a.ntok == 1) return a.stream;
  uint32_t tpw = a.waves / a.split;
  return (a.tiles + tpw - 1) / tpw * (a.kparts > 1 ? a.kparts : 1);
}

int gemv_launch(const GemvArgs& a, uint32_t qtype, int pro, int epi, hipStream_t s) {
  if (a.ntok == 0) return 0;
  if (a.split == 0 || a.split > 16 || (a.split & (a.split - 1)) || a.waves % a.split || a.waves > 16)
    return set_error(LLMHIP_ERR_ARG, "llm: gemv: split %u over %u waves", a.split, a.waves);
  if ((uint64_t)a.nb * 4 > 2ull * 64 * a.waves)
    return set_error(LLMHIP_ERR_ARG, "llm: gemv: k=%u is too long for %u waves", a.k, a.waves);
  if (a.kparts > 1 && (a.ntok != 1 || a.stream || a.kparts > 2 || a.ng < a.kparts || epi != EPI_STORE))
    return set_error(LLMHIP_ERR_ARG, "llm: gemv: k in %u parts is for one token's tile-kernel store", a.kparts);
  if ((pro & PRO_XSUM) && (a.ntok != 1 || a.k > 512u * a.waves))
    return set_error(LLMHIP_ERR_ARG, "llm: gemv: the summing prologue is for one token, k <= 512 * waves");
  switch (qtype) {
    case LLMHIP_Q4_0: return gemv_launch_qt<LLMHIP_Q4_0>(a, pro, epi, s);
    case LLMHIP_Q4_1: return gemv_launch_qt<LLMHIP_Q4_1>(a, pro, epi, s);
    case LLMHIP_Q8_0: return gemv_launch_qt<LLMHIP_Q8_0>(a, pro, epi, s);
  }
  return set_error(LLMHIP_ERR_TYPE, "llm: ggml type %u has no GPU kernel", qtype);
}

int gemm_launch(const GemvArgs& a, uint32_t qtype, int epi, hipStream_t s) {
  if (a.ntok == 0) return 0;
  if (a.ntok > a.tg * 16 || a.tg > 4) return set_error(LLMHIP_ERR_ARG, "llm: gemm: %u tokens in %u groups", a.ntok, a.tg);
  if (a.op_xp && (epi != EPI_GATEUP || a.q8 || a.tiles % 4 || a.op_nb != a.tiles / 4 || !a.op_dx || !a.op_bsum ||
                  !a.op_exp))
    return set_error(LLMHIP_ERR_ARG, "llm: gemm: the down operands come from a gate/up product of 32-row blocks");
  switch (qtype) {
    case LLMHIP_Q4_0: return gemm_launch_qt<LLMHIP_Q4_0>(a, epi, s);
    case LLMHIP_Q4_1: return gemm_launch_qt<LLMHIP_Q4_1>(a, epi, s);
    case LLMHIP_Q8_0: return gemm_launch_qt<LLMHIP_Q8_0>(a, epi, s);
  }
  return set_error(LLMHIP_ERR_TYPE, "llm: ggml type %u has no GPU kernel", qtype);
}

int qmat_dequant(const QMat& m, float* out, hipStream_t s) {
  switch (m.g.q.type) {
    case LLMHIP_Q4_0:
      return dequant_launch_qt<LLMHIP_Q4_0>(m, out, m.map, m.map_hd, m.map_seg0, m.map_seg1, m.ff, s);
    case LLMHIP_Q4_1:
      return dequant_launch_qt<LLMHIP_Q4_1>(m, out, m.map, m.map_hd, m.map_seg0, m.map_seg1, m.ff, s);
    case LLMHIP_Q8_0:
      return dequant_launch_qt<LLMHIP_Q8_0>(m, out, m.map, m.map_hd, m.map_seg0, m.map_seg1, m.ff, s);
  }
  return set_error(LLMHIP_ERR_TYPE, "llm: ggml type %u has no GPU kernel", m.g.q.type);
}

int embed_launch(const QMat& m, const int32_t* tokens, const uint32_t* state, float* x, uint32_t ntok,
                 hipStream_t s) {
  if (ntok == 0) return 0;
  switch (m.g.q.type) {
    case LLMHIP_Q4_0: return embed_launch_qt<LLMHIP_Q4_0>(m, tokens, state, x, ntok, s);
    case LLMHIP_Q8_0: return embed_launch_qt<LLMHIP_Q8_0>(m, tokens, state, x, ntok, s);
    case LLMHIP_Q4_1: return embed_launch_qt<LLMHIP_Q4_1>(m, tokens, state, x, ntok, s);
  }
  return set_error(LLMHIP_ERR_TYPE, "llm: token_embd.weight must be Q8_0 or Q4_0");
}

}  // namespace llmhip

using namespace llmhip;

// ------------------------------------------------------------------ C-ABI

// The scratch of llmhip_qmat_gemv_noalloc: the prepared activations of up to
// 64 tokens of k <= LLMHIP_NOALLOC_MAX_K, one copy per device for the life of
// the process.  Host code uses the address noalloc_scratch() returns for a
// device, never the array's name (a host-side stand-in).
static __device__ __align__(256) uint8_t scratch[xprep_bytes(64, LLMHIP_NOALLOC_MAX_K)];

static std::mutex g_scratch_mu;
static std::vector<void*> g_scratch_at;  // per device ordinal, from hipGetSymbolAddress

// The array's address on `device`, looked up once per device with that
// device current (the caller's current device is what it was, afterwards).
static int noalloc_scratch(int device, void** out) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (device < 0) return set_error(LLMHIP_ERR_ARG, "llm: device %d", device);
  if ((size_t)device >= g_scratch_at.size()) g_scratch_at.resize((size_t)device + 1, nullptr);
  if (!g_scratch_at[(size_t)device]) {
    int cur = 0;
    LLM_HIP(hipGetDevice(&cur));
    LLM_HIP(hipSetDevice(device));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    LLM_HIP(hipSetDevice(cur));
    if (e != hipSuccess || !p)
      return set_error(LLMHIP_ERR_DEVICE, "llm: no device address for the scratch array: %s", hipGetErrorString(e));
    g_scratch_at[(size_t)device] = p;
  }
  *out = g_scratch_at[(size_t)device];
  return 0;
}

struct llmhip_qmat {
  QMat m;
  Stager st;
  hipStream_t stream = nullptr;
  void* xprep = nullptr;  // prepared activations of up to 64 tokens (allocated on first use)
  void* scratch = nullptr;  // this device's noalloc scratch array (resolved at create)
};

extern "C" {


int llmhip_device_count(int* n) {
  clear_error();
  *n = 0;
  hipError_t e = hipGetDeviceCount(n);
  if (e == hipErrorNoDevice) {
    *n = 0;
    return 0;
  }
  if (e != hipSuccess) return set_error(LLMHIP_ERR_DEVICE, "llm: no GPU: %s", hipGetErrorString(e));
  return 0;
}

int llmhip_device_limits(int ordinal, llmhip_limits* out) {
  clear_error();
  hipDeviceProp_t p;
  LLM_HIP(hipGetDeviceProperties(&p, ordinal));
  out->max_invocations_per_workgroup = (uint32_t)p.maxThreadsPerBlock;
  out->max_workgroup_storage = (uint32_t)p.sharedMemPerBlock;
  out->max_workgroups_per_dimension = (uint32_t)p.maxGridSize[0];
  out->max_storage_buffers = 0xffffffffu;  // no binding slots: kernels take raw pointers
  out->max_binding_size = p.totalGlobalMem;
  out->max_buffer_size = p.totalGlobalMem;
  out->memory_budget = p.totalGlobalMem;
  return 0;
}

int llmhip_buffer_alloc(int ordinal, uint64_t bytes, void** out) {
  clear_error();
  *out = nullptr;
  LLM_HIP(hipSetDevice(ordinal));
  LLM_HIP(hipMalloc(out, bytes ? bytes : 1));
  if (hipMemset(*out, 0, bytes ? bytes : 1) != hipSuccess) {
    (void)hipFree(*out);
    *out = nullptr;
    return set_error(LLMHIP_ERR_DEVICE, "llm: hipMemset failed");
  }
  return 0;
}

void llmhip_buffer_free(void* dev) {
  if (dev) (void)hipFree(dev);
}

// Synchronous copies between caller memory and the device in pieces through
// a pinned staging buffer of this call.
constexpr uint64_t BUFFER_STAGE = 4ull << 20;

static int buffer_copy(void* dst, const void* src, uint64_t bytes, bool to_dev) {
  clear_error();
  if (!bytes) return 0;
  uint8_t* stage = nullptr;
  LLM_HIP(hipHostMalloc((void**)&stage, std::min(bytes, BUFFER_STAGE), hipHostMallocDefault));
  int rc = 0;
  for (uint64_t o = 0; o < bytes && rc == 0; o += BUFFER_STAGE) {
    const uint64_t c = std::min(BUFFER_STAGE, bytes - o);
    if (to_dev) {
      memcpy(stage, (const uint8_t*)src + o, c);
      if (hipMemcpy((uint8_t*)dst + o, stage, c, hipMemcpyHostToDevice) != hipSuccess)
        rc = set_error(LLMHIP_ERR_DEVICE, "llm: copy to the device failed");
    } else {
      if (hipMemcpy(stage, (const uint8_t*)src + o, c, hipMemcpyDeviceToHost) != hipSuccess)
        rc = set_error(LLMHIP_ERR_DEVICE, "llm: copy from the device failed");
      else
        memcpy((uint8_t*)dst + o, stage, c);
    }
  }
  (void)hipHostFree(stage);
  return rc;
}

int llmhip_buffer_write(void* dev, const void* host, uint64_t bytes) { return buffer_copy(dev, host, bytes, true); }

int llmhip_buffer_read(void* host, const void* dev, uint64_t bytes) { return buffer_copy(host, dev, bytes, false); }

int llmhip_device_synchronize(int ordinal) {
  clear_error();
  LLM_HIP(hipSetDevice(ordinal));
  LLM_HIP(hipDeviceSynchronize());
  return 0;
}

int llmhip_bench_h2d(int ordinal, uint64_t bytes, int iters, float* gbps) {
  clear_error();
  if (iters < 1 || bytes == 0) return set_error(LLMHIP_ERR_ARG, "llm: h2d bench of %d copies", iters);
  LLM_HIP(hipSetDevice(ordinal));
  uint8_t *h = nullptr, *d = nullptr;
  hipStream_t s = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = 0;
  float ms = 0;
  if (hipHostMalloc((void**)&h, bytes, hipHostMallocDefault) != hipSuccess || hipMalloc((void**)&d, bytes) != hipSuccess ||
      hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess || hipEventCreate(&e0) != hipSuccess ||
      hipEventCreate(&e1) != hipSuccess)
    rc = set_error(LLMHIP_ERR_DEVICE, "llm: h2d bench setup failed");
  for (int i = 0; i < 3 && rc == 0; i++)
    if (hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, s) != hipSuccess) rc = LLMHIP_ERR_DEVICE;
  if (rc == 0 && hipEventRecord(e0, s) != hipSuccess) rc = LLMHIP_ERR_DEVICE;
  for (int i = 0; i < iters && rc == 0; i++)
    if (hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, s) != hipSuccess) rc = LLMHIP_ERR_DEVICE;
  if (rc == 0 && (hipEventRecord(e1, s) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                  hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
    rc = LLMHIP_ERR_DEVICE;
  if (rc == LLMHIP_ERR_DEVICE) set_error(LLMHIP_ERR_DEVICE, "llm: h2d bench failed");
  if (s) (void)hipStreamSynchronize(s);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (s) (void)hipStreamDestroy(s);
  if (d) (void)hipFree(d);
  if (h) (void)hipHostFree(h);
  if (rc == 0) *gbps = (float)((double)bytes * iters / (ms * 1e-3) * 1e-9);
  return rc;
}

int llmhip_copy_calibration(int ordinal, uint64_t bytes) {
  clear_error();
  LLM_HIP(hipSetDevice(ordinal));
  void *a = nullptr, *b = nullptr;
  int rc = 0;
  if (hipMalloc(&a, bytes) != hipSuccess || hipMalloc(&b, bytes) != hipSuccess || hipMemset(a, 1, bytes) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess || hipMemcpy(b, a, bytes, hipMemcpyDeviceToDevice) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess)
    rc = set_error(LLMHIP_ERR_DEVICE, "llm: calibration copy failed");
  if (a) (void)hipFree(a);
  if (b) (void)hipFree(b);
  return rc;
}

// A matrix holds only its device memory; an upload creates the matrix's
// stream on first use and pinned staging for the duration of the call (a
// benchmark rotates thousands of clones, which never upload).
int llmhip_qmat_create(int ordinal, uint32_t ggml_type, uint64_t rows, uint64_t k, llmhip_qmat** out) {
  clear_error();
  *out = nullptr;
  llmhip_qmat* q = new llmhip_qmat();
  int rc = qmat_alloc(&q->m, ordinal, ggml_type, rows, k);
  if (rc == 0) rc = noalloc_scratch(ordinal, &q->scratch);
  if (rc != 0) {
    qmat_release(&q->m);
    delete q;
    return rc;
  }
  *out = q;
  return 0;
}

int llmhip_qmat_upload(llmhip_qmat* q, const void* raw, uint64_t nbytes, uint64_t byte_offset) {
  clear_error();
  LLM_HIP(hipSetDevice(q->m.device));
  if (!q->stream) LLM_HIP(hipStreamCreateWithFlags(&q->stream, hipStreamNonBlocking));
  int rc = stager_init(&q->st, q->m.device, 4ull << 20, q->stream);
  if (rc == 0) rc = qmat_upload(&q->st, q->m, raw, nbytes, byte_offset, 0);
  if (hipStreamSynchronize(q->stream) != hipSuccess && rc == 0)
    rc = set_error(LLMHIP_ERR_DEVICE, "llm: upload failed");
  stager_free(&q->st);
  return rc;
}

// Work queued by an upload is complete before a product reads the matrix.
static int qmat_ready(llmhip_qmat* q) {
  LLM_HIP(hipSetDevice(q->m.device));
  if (q->stream) LLM_HIP(hipStreamSynchronize(q->stream));
  return 0;
}

int llmhip_qmat_dequant(llmhip_qmat* q, float* out_dev, void* hip_stream) {
  clear_error();
  LLM_TRY(qmat_ready(q));
  return qmat_dequant(q->m, out_dev, (hipStream_t)hip_stream);
}

static int qmat_gemv_args(llmhip_qmat* q, const float* x, float* y, int n, GemvArgs* a) {
  if (n < 1 || n > 64) return set_error(LLMHIP_ERR_ARG, "llm: gemv of %d tokens (1..64)", n);
  memset(a, 0, sizeof *a);
  gemv_bind(a, q->m);
  a->ntok = (uint32_t)n;
  a->x = x;
  a->ldx = a->k;
  a->y = y;
  a->ldy = a->rows;
  return 0;
}

// One product: the decode kernel below GEMM_MIN_TOKENS tokens, else the
// prefill pair, whose prepared activations go to `xprep` (xprep_bytes(64, k)
// bytes; nullptr: the matrix's own buffer, allocated on first use).
static int qmat_launch(llmhip_qmat* q, GemvArgs& a, int epi, hipStream_t s, int pro = PRO_PLAIN,
                       void* xprep = nullptr) {
  if (a.ntok < GEMM_MIN_TOKENS) return gemv_launch(a, q->m.g.q.type, pro, epi, s);
  if (!xprep) {
    if (!q->xprep) LLM_HIP(hipMalloc(&q->xprep, xprep_bytes(64, (uint32_t)q->m.g.k)));
    xprep = q->xprep;
  }
  xprep_bind(&a, xprep);
  a.q8 = (pro & PRO_Q8) ? 1 : 0;
  LLM_TRY(prep_launch(a, pro, s));
  return gemm_launch(a, q->m.g.q.type, epi, s);
}

int llmhip_qmat_gemv(llmhip_qmat* q, const float* x_dev, float* y_dev, int n, int accumulate, void* hip_stream) {
  clear_error();
  GemvArgs a;
  LLM_TRY(qmat_gemv_args(q, x_dev, y_dev, n, &a));
  LLM_TRY(qmat_ready(q));
  return qmat_launch(q, a, accumulate ? EPI_ACC : EPI_STORE, (hipStream_t)hip_stream);
}

// Makes no runtime call but its launches (capturable into a HIP graph): the
// scratch address was resolved at create, and an upload is complete when
// llmhip_qmat_upload returns, so no wait for the matrix's own stream either.
int llmhip_qmat_gemv_noalloc(llmhip_qmat* q, const float* x_dev, float* y_dev, int n, int accumulate,
                             void* hip_stream) {
  clear_error();
  if (q->m.g.k > LLMHIP_NOALLOC_MAX_K)
    return set_error(LLMHIP_ERR_ARG, "llm: gemv_noalloc: k=%llu is above its scratch's maximum of %u",
                     (unsigned long long)q->m.g.k, (unsigned)LLMHIP_NOALLOC_MAX_K);
  GemvArgs a;
  LLM_TRY(qmat_gemv_args(q, x_dev, y_dev, n, &a));
  return qmat_launch(q, a, accumulate ? EPI_ACC : EPI_STORE, (hipStream_t)hip_stream, PRO_PLAIN, q->scratch);
}

int llmhip_qmat_gemv_q8(llmhip_qmat* q, const float* x_dev, float* y_dev, int n, void* hip_stream) {
  clear_error();
  GemvArgs a;
  LLM_TRY(qmat_gemv_args(q, x_dev, y_dev, n, &a));
  LLM_TRY(qmat_ready(q));
  return qmat_launch(q, a, EPI_STORE, (hipStream_t)hip_stream, PRO_PLAIN | PRO_Q8);
}

uint64_t llmhip_qmat_bytes(const llmhip_qmat* q) { return q->m.bytes; }
uint64_t llmhip_qmat_gguf_bytes(const llmhip_qmat* q) { return q->m.g.gguf_bytes(); }

int llmhip_qmat_bench(llmhip_qmat* const* mats, int count, const float* x_dev, float* y_dev, int n, int iters,
                      int warmup, void* hip_stream, float* avg_us) {
  clear_error();
  if (count < 1 || iters < 1) return set_error(LLMHIP_ERR_ARG, "llm: bench of %d matrices, %d iterations", count, iters);
  hipStream_t s = (hipStream_t)hip_stream;
  std::vector<GemvArgs> args((size_t)count);
  for (int i = 0; i < count; i++) {
    LLM_TRY(qmat_gemv_args(mats[i], x_dev, y_dev, n, &args[i]));
    if (mats[i]->m.g.q.type != mats[0]->m.g.q.type || mats[i]->m.g.rows != mats[0]->m.g.rows ||
        mats[i]->m.g.k != mats[0]->m.g.k)
      return set_error(LLMHIP_ERR_ARG, "llm: bench matrices differ in shape or type");
    LLM_TRY(qmat_ready(mats[i]));
  }
  LLM_HIP(hipSetDevice(mats[0]->m.device));
  const uint32_t t = mats[0]->m.g.q.type;
  (void)t;
  for (int i = 0; i < warmup; i++) LLM_TRY(qmat_launch(mats[i % count], args[i % count], EPI_STORE, s));
  hipEvent_t e0, e1;
  LLM_HIP(hipEventCreate(&e0));
  LLM_HIP(hipEventCreate(&e1));
  LLM_HIP(hipEventRecord(e0, s));
  for (int i = 0; i < iters; i++) LLM_TRY(qmat_launch(mats[i % count], args[i % count], EPI_STORE, s));
  LLM_HIP(hipEventRecord(e1, s));
  LLM_HIP(hipEventSynchronize(e1));
  float ms = 0;
  LLM_HIP(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *avg_us = ms * 1000.f / (float)iters;
  return 0;
}

int llmhip_qmat_bench_graph(llmhip_qmat* const* mats, int count, const float* x_dev, float* y_dev, int n,
                            int iters, int warmup, void* hip_stream, float* avg_us) {
  clear_error();
  if (count < 1 || iters < 1) return set_error(LLMHIP_ERR_ARG, "llm: bench of %d matrices, %d iterations", count, iters);
  std::vector<GemvArgs> args((size_t)count);
  for (int i = 0; i < count; i++) {
    LLM_TRY(qmat_gemv_args(mats[i], x_dev, y_dev, n, &args[i]));
    if (mats[i]->m.g.q.type != mats[0]->m.g.q.type || mats[i]->m.g.rows != mats[0]->m.g.rows ||
        mats[i]->m.g.k != mats[0]->m.g.k)
      return set_error(LLMHIP_ERR_ARG, "llm: bench matrices differ in shape or type");
    LLM_TRY(qmat_ready(mats[i]));
  }
  LLM_HIP(hipSetDevice(mats[0]->m.device));
  hipStream_t s = (hipStream_t)hip_stream;
  bool own = false;
  if (!s) {  // the legacy stream cannot be captured
    LLM_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    own = true;
  }
  hipGraph_t g = nullptr;
  hipGraphExec_t ex = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = 0;
  // direct launches first: they make what a first launch allocates (the
  // prefill pair's activation buffer), which a capture must not
  for (int i = 0; i < std::max(warmup, count) && rc == 0; i++) rc = qmat_launch(mats[i % count], args[i % count], EPI_STORE, s);
  if (rc == 0 && hipStreamSynchronize(s) != hipSuccess) rc = set_error(LLMHIP_ERR_DEVICE, "llm: warmup failed");
  const int per = std::max(count, 16);  // launches per graph, cycling through the matrices
  if (rc == 0) {
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) {
      rc = set_error(LLMHIP_ERR_DEVICE, "llm: stream capture failed");
    } else {
      for (int i = 0; i < per && rc == 0; i++) rc = qmat_launch(mats[i % count], args[i % count], EPI_STORE, s);
      const hipError_t e = hipStreamEndCapture(s, &g);
      if (rc == 0 && e != hipSuccess) rc = set_error(LLMHIP_ERR_DEVICE, "llm: capture failed: %s", hipGetErrorString(e));
    }
  }
  if (rc == 0 && hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) != hipSuccess)
    rc = set_error(LLMHIP_ERR_DEVICE, "llm: graph instantiate failed");
  if (rc == 0 && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
    rc = set_error(LLMHIP_ERR_DEVICE, "llm: hipEventCreate failed");
  const int reps = (iters + per - 1) / per;
  float ms = 0;
  if (rc == 0) {
    bool ok = hipGraphLaunch(ex, s) == hipSuccess && hipStreamSynchronize(s) == hipSuccess;  // one untimed replay
    ok = ok && hipEventRecord(e0, s) == hipSuccess;
    for (int r = 0; r < reps && ok; r++) ok = hipGraphLaunch(ex, s) == hipSuccess;
    ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess &&
         hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
    if (!ok) rc = set_error(LLMHIP_ERR_DEVICE, "llm: graph replay failed");
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (ex) (void)hipGraphExecDestroy(ex);
  if (g) (void)hipGraphDestroy(g);
  if (own) (void)hipStreamDestroy(s);
  if (rc == 0) *avg_us = ms * 1000.f / (float)(reps * per);
  return rc;
}

int llmhip_qmat_clone(const llmhip_qmat* q, llmhip_qmat** out) {
  clear_error();
  *out = nullptr;
  llmhip_qmat* c = nullptr;
  LLM_TRY(llmhip_qmat_create(q->m.device, q->m.g.q.type, q->m.g.rows, q->m.g.k, &c));
  c->m.map = q->m.map;
  c->m.map_hd = q->m.map_hd;
  c->m.map_seg0 = q->m.map_seg0;
  c->m.map_seg1 = q->m.map_seg1;
  c->m.ff = q->m.ff;
  if (hipMemcpy(c->m.qs, q->m.qs, q->m.g.dev_bytes(), hipMemcpyDeviceToDevice) != hipSuccess) {
    llmhip_qmat_free(c);
    return set_error(LLMHIP_ERR_DEVICE, "llm: clone copy failed");
  }
  *out = c;
  return 0;
}

void llmhip_qmat_free(llmhip_qmat* q) {
  if (!q) return;
  (void)hipSetDevice(q->m.device);
  stager_free(&q->st);
  if (q->stream) (void)hipStreamDestroy(q->stream);
  if (q->xprep) (void)hipFree(q->xprep);
  qmat_release(&q->m);
  delete q;
}

}  // extern "C"
