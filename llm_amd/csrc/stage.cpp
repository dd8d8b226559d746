// Host -> device staging of raw GGUF blocks (the loader's fast path).
//
// The reference reads each tensor in PieceSize pieces through an io.ReaderAt,
// repacks every block on the host and writes the result with
// Queue.WriteBuffer (gpu.go:231-269, 347-391).  Here the raw blocks go from
// the page cache (pread) or from caller memory (memcpy) straight into pinned
// staging, filled by a pool of host threads, then one DMA per piece and the
// repack on the device (repack_kernel).  STAGE_BUFS buffers keep the host
// fill of piece i+2 and the DMA of piece i+1 running under the repack of
// piece i; small tensors share a buffer.
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "gemv.h"

namespace llmhip {

// A fixed set of worker threads that run the tasks of one job at a time; the
// calling thread takes tasks too.  One job at a time process-wide (run() holds
// a mutex), which serialises concurrent loads rather than oversubscribing.
class HostPool {
 public:
  explicit HostPool(int n) {
    for (int i = 0; i < n; i++) th_.emplace_back([this] { work(); });
  }
  ~HostPool() {
    {
      std::lock_guard<std::mutex> l(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : th_) t.join();
  }
  int threads() const { return (int)th_.size() + 1; }
  void run(int tasks, const std::function<void(int)>& fn) {
    std::lock_guard<std::mutex> job(job_mu_);
    {
      std::lock_guard<std::mutex> l(mu_);
      fn_ = &fn;
      tasks_ = tasks;
      next_ = 0;
      pending_ = tasks;
      gen_++;
    }
    cv_.notify_all();
    take();
    std::unique_lock<std::mutex> l(mu_);
    done_cv_.wait(l, [this] { return pending_ == 0; });
    fn_ = nullptr;
  }

 private:
  // run tasks of the current job until none is left
  void take() {
    for (;;) {
      int i;
      const std::function<void(int)>* fn;
      {
        std::lock_guard<std::mutex> l(mu_);
        if (!fn_ || next_ >= tasks_) return;
        i = next_++;
        fn = fn_;
      }
      (*fn)(i);
      std::lock_guard<std::mutex> l(mu_);
      if (--pending_ == 0) done_cv_.notify_all();
    }
  }
  void work() {
    uint64_t seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> l(mu_);
        cv_.wait(l, [&] { return stop_ || gen_ != seen; });
        if (stop_) return;
        seen = gen_;
      }
      take();
    }
  }
  std::vector<std::thread> th_;
  std::mutex mu_, job_mu_;
  std::condition_variable cv_, done_cv_;
  const std::function<void(int)>* fn_ = nullptr;
  int tasks_ = 0, next_ = 0, pending_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

// Threads for staging, the caller included: up to 12 (measured: parallel
// page-cache reads pass the PCIe link's ~50 GB/s at 8-12 threads).
static HostPool& host_pool() {
  static HostPool pool(std::max(1, std::min(12, (int)std::thread::hardware_concurrency()) - 1));
  return pool;
}

int stager_init(Stager* st, int device, uint64_t cap, hipStream_t s) {
  st->device = device;
  st->cap = cap;
  st->stream = s;
  st->cur = 0;
  st->used = 0;
  LLM_HIP(hipSetDevice(device));
  LLM_HIP(hipStreamCreateWithFlags(&st->copy, hipStreamNonBlocking));
  for (int i = 0; i < STAGE_BUFS; i++) {
    LLM_HIP(hipHostMalloc((void**)&st->host[i], cap, hipHostMallocDefault));
    LLM_HIP(hipMalloc((void**)&st->dev[i], cap));
    LLM_HIP(hipEventCreateWithFlags(&st->done[i], hipEventDisableTiming));
    LLM_HIP(hipEventCreateWithFlags(&st->copied[i], hipEventDisableTiming));
    LLM_HIP(hipEventRecord(st->done[i], s));
  }
  return 0;
}

void stager_free(Stager* st) {
  for (int i = 0; i < STAGE_BUFS; i++) {
    if (st->done[i]) (void)hipEventSynchronize(st->done[i]);
    if (st->host[i]) (void)hipHostFree(st->host[i]);
    if (st->dev[i]) (void)hipFree(st->dev[i]);
    if (st->done[i]) (void)hipEventDestroy(st->done[i]);
    if (st->copied[i]) (void)hipEventDestroy(st->copied[i]);
    st->host[i] = st->dev[i] = nullptr;
    st->done[i] = st->copied[i] = nullptr;
  }
  if (st->copy) {
    (void)hipStreamSynchronize(st->copy);
    (void)hipStreamDestroy(st->copy);
    st->copy = nullptr;
  }
  st->cap = 0;
}

// DMA n staged bytes h -> d on the copy stream; work queued on the model's
// stream after this waits for it.  The copy stream runs the next piece's DMA
// while the model's stream repacks this one.
static int stage_dma(Stager* st, void* d, const void* h, uint64_t n) {
  LLM_HIP(hipMemcpyAsync(d, h, n, hipMemcpyHostToDevice, st->copy));
  LLM_HIP(hipEventRecord(st->copied[st->cur], st->copy));
  LLM_HIP(hipStreamWaitEvent(st->stream, st->copied[st->cur], 0));
  return 0;
}

// Whole pread of n bytes at off, retrying short reads; false at end of file or error.
static bool pread_all(int fd, void* dst, uint64_t n, uint64_t off) {
  uint64_t got = 0;
  while (got < n) {
    ssize_t r = pread(fd, (char*)dst + got, n - got, (off_t)(off + got));
    if (r <= 0) return false;
    got += (uint64_t)r;
  }
  return true;
}

// Slices of at least 1 MiB, one per pool thread at most.
constexpr uint64_t STAGE_SLICE_MIN = 1ull << 20;

int stage_read(const Source& src, uint64_t off, void* dst, uint64_t n) {
  if (n == 0) return 0;
  HostPool& pool = host_pool();
  uint64_t slices = std::min<uint64_t>((uint64_t)pool.threads(), (n + STAGE_SLICE_MIN - 1) / STAGE_SLICE_MIN);
  uint64_t per = ((n + slices - 1) / slices + 4095) & ~4095ull;
  std::atomic<bool> ok{true};
  auto one = [&](int i) {
    uint64_t a = (uint64_t)i * per;
    if (a >= n) return;
    uint64_t b = std::min(n, a + per);
    if (src.mem)
      memcpy((char*)dst + a, src.mem + off + a, b - a);
    else if (!pread_all(src.fd, (char*)dst + a, b - a, src.file_off + off + a))
      ok = false;
  };
  if (slices <= 1)
    one(0);
  else
    pool.run((int)slices, one);
  if (!ok) return set_error(LLMHIP_ERR_IO, "llm: short read at file offset %llu", (unsigned long long)(src.file_off + off));
  return 0;
}

static int repack_dev(const QMat& m, const uint8_t* raw_dev, uint64_t n, uint64_t blk0, uint64_t row_off,
                      hipStream_t s) {
  switch (m.g.q.type) {
    case LLMHIP_Q4_0:
      return repack_launch_qt<LLMHIP_Q4_0>(m, raw_dev, n, blk0, row_off, m.map, m.map_hd, m.map_seg0, m.map_seg1,
                                           m.ff, s);
    case LLMHIP_Q4_1:
      return repack_launch_qt<LLMHIP_Q4_1>(m, raw_dev, n, blk0, row_off, m.map, m.map_hd, m.map_seg0, m.map_seg1,
                                           m.ff, s);
    case LLMHIP_Q8_0:
      return repack_launch_qt<LLMHIP_Q8_0>(m, raw_dev, n, blk0, row_off, m.map, m.map_hd, m.map_seg0, m.map_seg1,
                                           m.ff, s);
  }
  return set_error(LLMHIP_ERR_TYPE, "llm: ggml type %u has no GPU kernel", m.g.q.type);
}

// Room for a piece of n <= cap bytes: the rest of the current buffer, or the
// next buffer once the work queued on it has finished.  Small tensors share a
// buffer, so the host waits once per buffer, not once per tensor.
static int stage_slot(Stager* st, uint64_t n, uint8_t** host, uint8_t** dev) {
  if (st->used + n > st->cap) {
    st->cur = (st->cur + 1) % STAGE_BUFS;
    st->used = 0;
    LLM_HIP(hipEventSynchronize(st->done[st->cur]));
  }
  *host = st->host[st->cur] + st->used;
  *dev = st->dev[st->cur] + st->used;
  st->used += (n + 255) & ~255ull;
  return 0;
}

// The raw blocks cross PCIe once and the repack runs on the device.
int qmat_upload(Stager* st, const QMat& m, const Source& src, uint64_t nbytes, uint64_t byte_off, uint64_t row_off) {
  const uint32_t bb = m.g.q.block_bytes;
  if (nbytes % bb != 0 || byte_off % bb != 0)
    return set_error(LLMHIP_ERR_ARG, "llm: upload of %llu bytes at %llu is not whole %u-byte blocks",
                     (unsigned long long)nbytes, (unsigned long long)byte_off, bb);
  uint64_t blk0 = byte_off / bb, nblk = nbytes / bb;
  if (row_off * m.g.nb + blk0 + nblk > m.g.rows * m.g.nb)
    return set_error(LLMHIP_ERR_ARG, "llm: upload past the end of a [%llu][%llu] matrix",
                     (unsigned long long)m.g.rows, (unsigned long long)m.g.k);
  uint64_t per = st->cap / bb;
  LLM_HIP(hipSetDevice(st->device));
  for (uint64_t i = 0; i < nblk; i += per) {
    uint64_t n = nblk - i < per ? nblk - i : per;
    uint8_t *h, *d;
    LLM_TRY(stage_slot(st, n * bb, &h, &d));
    LLM_TRY(stage_read(src, i * bb, h, n * bb));
    LLM_TRY(stage_dma(st, d, h, n * bb));
    LLM_TRY(repack_dev(m, d, n, blk0 + i, row_off, st->stream));
    LLM_HIP(hipEventRecord(st->done[st->cur], st->stream));
  }
  return 0;
}

// Gaps between consecutive pieces (alignment padding, tensors the model does
// not use) up to this size are read along; a larger gap starts a new run.
constexpr uint64_t STAGE_RUN_GAP = 64ull << 10;

int stage_file_runs(Stager* st, int fd, const StagePiece* ps, size_t count) {
  LLM_HIP(hipSetDevice(st->device));
  Source src;
  src.fd = fd;
  for (size_t i = 0; i < count;) {
    uint64_t start = ps[i].file, end = start + ps[i].bytes;
    size_t j = i + 1;
    while (j < count && ps[j].file >= end && ps[j].file - end <= STAGE_RUN_GAP && ps[j].file + ps[j].bytes - start <= st->cap)
      end = ps[j].file + ps[j].bytes, j++;
    uint8_t *h, *d;
    LLM_TRY(stage_slot(st, end - start, &h, &d));
    LLM_TRY(stage_read(src, start, h, end - start));
    LLM_TRY(stage_dma(st, d, h, end - start));
    for (size_t k = i; k < j; k++) {
      const StagePiece& p = ps[k];
      const uint8_t* pd = d + (p.file - start);
      if (p.q) {
        const uint32_t bb = p.q->g.q.block_bytes;
        LLM_TRY(repack_dev(*p.q, pd, p.bytes / bb, p.off / bb, p.row_off, st->stream));
      } else {
        LLM_HIP(hipMemcpyAsync((char*)p.f + p.off, pd, p.bytes, hipMemcpyDeviceToDevice, st->stream));
      }
    }
    LLM_HIP(hipEventRecord(st->done[st->cur], st->stream));
    i = j;
  }
  return 0;
}

int f32_upload(Stager* st, float* dst, const Source& src, uint64_t nbytes, uint64_t byte_off) {
  LLM_HIP(hipSetDevice(st->device));
  for (uint64_t i = 0; i < nbytes; i += st->cap) {
    uint64_t n = nbytes - i < st->cap ? nbytes - i : st->cap;
    uint8_t *h, *d;
    LLM_TRY(stage_slot(st, n, &h, &d));
    LLM_TRY(stage_read(src, i, h, n));
    LLM_TRY(stage_dma(st, d, h, n));
    LLM_HIP(hipMemcpyAsync((char*)dst + byte_off + i, d, n, hipMemcpyDeviceToDevice, st->stream));
    LLM_HIP(hipEventRecord(st->done[st->cur], st->stream));
  }
  return 0;
}

}  // namespace llmhip
