// The host half of the reference's Go package, in C++, above the llmhip_*
// device layer: NewGPU's streaming loader (gpu.go:465-764 with the repack now
// on the device), Generate, PrefillLogits and Peek (gpu.go:904-1043).  The
// GGUF header parser and ConfigFrom it uses are in gguf.cpp.
#include <execinfo.h>
#include <fcntl.h>
#include <signal.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "common.h"
#include "gguf.h"
#include "host.h"

using namespace llm;
using llmhip::set_error;

// Tunables of the Go package (gpu.go:20-23,165,1046-1054).
static int g_decode_batch = 8, g_prefill_batch = 64, g_f16kv = 0, g_exact = 0;

// With LLMHIP_CRASH_TRACE set when the library loads, a SIGSEGV, SIGBUS or
// SIGABRT first writes the native stack to stderr (frames as path(+offset),
// for addr2line on the library), then goes to the handler that was installed
// before (Python's faulthandler, say), or to the default action.
namespace {
struct sigaction g_prev_act[3];
const int g_trace_sigs[3] = {SIGSEGV, SIGBUS, SIGABRT};

void crash_trace(int sig, siginfo_t* info, void* uctx) {
  static const char head[] = "llmhip: fatal signal, native stack:\n";
  (void)!write(2, head, sizeof head - 1);
  void* frames[64];
  int n = backtrace(frames, 64);
  backtrace_symbols_fd(frames, n, 2);
  for (int i = 0; i < 3; i++) {
    if (g_trace_sigs[i] != sig) continue;
    sigaction(sig, &g_prev_act[i], nullptr);
    if ((g_prev_act[i].sa_flags & SA_SIGINFO) && g_prev_act[i].sa_sigaction) {
      g_prev_act[i].sa_sigaction(sig, info, uctx);
    } else if (g_prev_act[i].sa_handler != SIG_DFL && g_prev_act[i].sa_handler != SIG_IGN) {
      g_prev_act[i].sa_handler(sig);
    }
    break;
  }
  raise(sig);  // the default action, if the previous handler returned
}

__attribute__((constructor)) void install_crash_trace() {
  const char* e = getenv("LLMHIP_CRASH_TRACE");
  if (!e || !*e || *e == '0') return;
  void* warm[2];
  (void)backtrace(warm, 2);  // loads the unwinder now, not inside the handler
  for (int i = 0; i < 3; i++) {
    struct sigaction a;
    memset(&a, 0, sizeof a);
    a.sa_sigaction = crash_trace;
    a.sa_flags = SA_SIGINFO | SA_ONSTACK;
    sigemptyset(&a.sa_mask);
    sigaction(g_trace_sigs[i], &a, &g_prev_act[i]);
  }
}
}  // namespace
static const int kMaxBatch = 16;

struct llm_gpu {
  llmhip_model* m = nullptr;
  llmhip_config cfg{};
  int ctx = 0;
};

extern "C" {


int llm_set_decode_batch(int n) {
  g_decode_batch = n;
  return 0;
}
int llm_set_f16kv(int on) {
  g_f16kv = on != 0;
  return 0;
}

int llm_set_exact_ggml(int on) {
  g_exact = on != 0;
  return 0;
}

int llm_set_prefill_batch(int n) {
  g_prefill_batch = n;
  return 0;
}

// NewGPU, gpu.go:465-764: the header, ConfigFrom, every needed tensor declared,
// then streamed from the file in PieceSize reads of whole blocks.
int llm_new_gpu(int ordinal, const llmhip_limits* lim, const char* path, int ctx, llm_gpu** out) {
  llmhip::clear_error();
  *out = nullptr;
  int fd = open(path, O_RDONLY);
  if (fd < 0) return set_error(LLMHIP_ERR_IO, "llm: cannot open %s", path);
  llm_gguf* gf = nullptr;
  int rc = parse_fd(fd, &gf, nullptr);
  llm_gpu* g = nullptr;
  if (rc == 0) {
    g = new llm_gpu();
    rc = config_from(gf->f, &g->cfg);
  }
  if (rc == 0) rc = llmhip_model_create(ordinal, lim, &g->cfg, ctx, g_prefill_batch, &g->m);
  if (rc == 0) rc = llmhip_model_set_exact_ggml(g->m, g_exact);
  if (rc == 0 && !g_exact) rc = llmhip_model_set_kv_f16(g->m, g_f16kv);
  if (rc == 0) llmhip_model_config(g->m, &g->cfg, &g->ctx);
  for (size_t i = 0; rc == 0 && i < gf->f.tensors.size(); i++) {
    const gguf::Tensor& t = gf->f.tensors[i];
    rc = llmhip_model_tensor(g->m, t.name.c_str(), t.type, t.dims.data(), (uint32_t)t.dims.size());
  }
  // whole tensors straight from the file into pinned staging (the parser
  // checked that every tensor lies inside the file)
  if (rc == 0) (void)posix_fadvise(fd, 0, 0, POSIX_FADV_SEQUENTIAL);
  if (rc == 0) {
    std::vector<const char*> names;
    std::vector<uint64_t> offs;
    for (const gguf::Tensor& t : gf->f.tensors) {
      names.push_back(t.name.c_str());
      offs.push_back(gf->f.data_offset + t.offset);
    }
    rc = llmhip_model_upload_file_tensors(g->m, fd, (uint32_t)names.size(), names.data(), offs.data());
  }
  if (rc == 0) rc = llmhip_model_finalize(g->m);
  close(fd);
  llm_gguf_free(gf);
  if (rc) {
    if (g) {
      llmhip_model_free(g->m);
      delete g;
    }
    return rc;
  }
  *out = g;
  return 0;
}

static int64_t ns_since(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t).count();
}

// Generate, gpu.go:946-1014: the prompt, then submits of up to DecodeBatch
// tokens each sampled on the GPU; emit runs on the caller's thread; stops after
// n tokens, at eos (not emitted) or when emit returns 0.
int llm_gpu_generate(llm_gpu* g, const int32_t* prompt, int n_prompt, int n, int32_t eos, llm_emit_fn emit,
                     void* user, llm_timing* tm) {
  llmhip::clear_error();
  llm_timing t{};
  if (n < 0) return set_error(LLMHIP_ERR_ARG, "llm: %d new tokens", n);
  if ((int64_t)n_prompt + n > g->ctx)
    return set_error(LLMHIP_ERR_CONTEXT, "llm: prompt of %d tokens and %d new tokens exceed the context of %d",
                     n_prompt, n, g->ctx);
  llmhip_stats s0;
  llmhip_model_stats(g->m, &s0);
  auto t0 = std::chrono::steady_clock::now();
  int32_t buf[kMaxBatch];
  LLM_TRY(llmhip_model_prefill(g->m, prompt, n_prompt, nullptr, &buf[0]));
  t.prefill_ns = ns_since(t0);
  t.prompt_tokens = n_prompt;
  auto t1 = std::chrono::steady_clock::now();
  int cnt = 1, produced = 0;
  const int batch = std::max(1, std::min(g_decode_batch, kMaxBatch));
  while (produced < n) {
    for (int j = 0; j < cnt && produced < n; j++) {
      int32_t tok = buf[j];
      if (tok == eos) {
        n = produced;
        break;
      }
      t.generated++;
      produced++;
      if (emit && !emit(tok, user)) {
        n = produced;
        break;
      }
    }
    if (produced >= n) break;
    cnt = std::min(batch, n - produced);
    auto ta = std::chrono::steady_clock::now();
    LLM_TRY(llmhip_model_decode(g->m, cnt, buf));
    t.submit_ns += ns_since(ta);
  }
  t.decode_ns = ns_since(t1);
  llmhip_stats s1;
  llmhip_model_stats(g->m, &s1);
  t.submits = s1.submits - s0.submits;
  t.dispatches = s1.dispatches - s0.dispatches;
  if (tm) *tm = t;
  return 0;
}

// PrefillLogits, gpu.go:904-927.
int llm_gpu_prefill_logits(llm_gpu* g, const int32_t* prompt, int n_prompt, float* logits) {
  llmhip::clear_error();
  if (n_prompt >= g->ctx) return set_error(LLMHIP_ERR_CONTEXT, "llm: prompt longer than the context");
  return llmhip_model_prefill(g->m, prompt, n_prompt, logits, nullptr);
}

int llm_gpu_peek(llm_gpu* g, const char* name, float* out, uint64_t n) {
  return llmhip_model_peek(g->m, name, out, n);
}

llmhip_model* llm_gpu_model(llm_gpu* g) { return g->m; }

int llm_gpu_config(const llm_gpu* g, llmhip_config* out, int* ctx) {
  *out = g->cfg;
  if (ctx) *ctx = g->ctx;
  return 0;
}

void llm_gpu_free(llm_gpu* g) {
  if (!g) return;
  llmhip_model_free(g->m);
  delete g;
}

}  // extern "C"
