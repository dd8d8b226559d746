// llm-generate: the caller harness of examples/generate/main.go as a native
// tool over the C-ABI (include/llmhip.h), for hosts without Go.
//
//   llm-generate run   [-n N] [-ctx C] [-model FILE] [-ids 1,2,3 | -p P]     greedy generation on the GPU
//   llm-generate check [-n N] [-ctx C] [-model FILE] -ref FILE [-tol T]      step-1 logits and the first N
//                                                                           tokens against a reference file
//   llm-generate bench [-rounds R] [-p P] [-n N] [-ctx C] [-model FILE]      R rounds of P-token prefill and
//                                                                           N-token decode (round 0 dropped)
//   llm-generate trace [-ctx C] [-model FILE] -ref FILE                      the residual stream after k layers
//                                                                           against the reference's x.<k>
//   llm-generate dump  [-n N] [-ctx C] [-model FILE] [-ids ... | -p P] [-layers 1,2,5] -out FILE
//                                                                           the GPU's own results as a reference file
//
// Modes and printed lines follow main.go:46-240 (run :109-117, check
// :141-181, bench :183-207, trace :212-240), with two differences that come
// from the boundary: prompts are token ids (the tokenizer is not part of this
// library; -ids, or -p P for a fixed synthetic prompt of P ids), and the CPU
// side of check / trace comes from a reference file (the CPU path is a
// separate program: any implementation of cpu.go writes the same records)
// instead of an in-process LoadCPU.  Exit 2 (printing "no GPU") without a
// GPU; check exits 3 when the logits or tokens fall outside -tol.  -f16kv and
// -exactggml select the CPU path's F16KV and ExactGGML numerics (cpu.go:15-24).
//
// Reference file: the 8 bytes "LLMREF01", then records until the end of the
// file: u32 name length, the name, u32 kind (0 f32, 1 i32), u64 count, count
// little-endian 4-byte values.  Names: "prompt" (i32 ids), "logits" (f32
// logits after the prompt), "tokens" (i32 greedy tokens), "x.<k>" (f32
// residual stream after k layers for the prompt's first token; k = -1 is the
// embedding).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "llmhip.h"

namespace {

[[noreturn]] void die(const std::string& msg) {
  fprintf(stderr, "error: %s\n", msg.c_str());
  exit(1);
}

void check_rc(int rc) {
  if (rc != 0) die(llmhip_last_error());
}

double ms_since(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t).count();
}

// ------------------------------------------------------------ flags

struct Flags {
  int n = 32, ctx = 512, rounds = 5, p = 128, batch = 8, prefillbatch = 64, device = 0;
  bool f16kv = false, exact = false;
  double tol = 1e-4;
  std::string model = "/models/smollm2-135m-instruct-q4_0.gguf", skip, ids, ref, out, layers = "-1,1,2,5,15,30";
  std::vector<std::string> args;  // positional: token ids
};

Flags parse_flags(int argc, char** argv) {
  Flags f;
  std::map<std::string, std::string*> str = {{"model", &f.model}, {"skip", &f.skip}, {"ids", &f.ids},
                                             {"ref", &f.ref},     {"out", &f.out},   {"layers", &f.layers}};
  std::map<std::string, int*> num = {{"n", &f.n},           {"ctx", &f.ctx},     {"rounds", &f.rounds},
                                     {"p", &f.p},           {"batch", &f.batch}, {"prefillbatch", &f.prefillbatch},
                                     {"device", &f.device}};
  for (int i = 0; i < argc; i++) {
    std::string a = argv[i];
    if (a.size() < 2 || a[0] != '-') {
      f.args.push_back(a);
      continue;
    }
    a = a.substr(a[1] == '-' ? 2 : 1);
    std::string v;
    bool has = false;
    size_t eq = a.find('=');
    if (eq != std::string::npos) v = a.substr(eq + 1), a = a.substr(0, eq), has = true;
    if (a == "f16kv" || a == "exactggml") {
      (a == "f16kv" ? f.f16kv : f.exact) = !has || v == "true" || v == "1";
      continue;
    }
    if (!has) {
      if (i + 1 >= argc) die("flag needs an argument: -" + a);
      v = argv[++i];
    }
    if (str.count(a)) {
      *str[a] = v;
    } else if (num.count(a)) {
      char* end;
      long x = strtol(v.c_str(), &end, 10);
      if (*end || v.empty()) die("invalid value \"" + v + "\" for flag -" + a);
      *num[a] = (int)x;
    } else if (a == "tol") {
      f.tol = atof(v.c_str());
    } else {
      die("flag provided but not defined: -" + a);
    }
  }
  return f;
}

std::vector<int32_t> parse_ids(const std::string& s) {
  std::vector<int32_t> out;
  size_t i = 0;
  while (i < s.size()) {
    size_t j = s.find_first_of(", ", i);
    if (j == std::string::npos) j = s.size();
    if (j > i) {
      char* end;
      long x = strtol(s.c_str() + i, &end, 10);
      if (end != s.c_str() + j) die("bad token id list \"" + s + "\"");
      out.push_back((int32_t)x);
    }
    i = j + 1;
  }
  return out;
}

// A fixed synthetic prompt of p ids below vocab (the tool has no tokenizer).
std::vector<int32_t> synthetic_prompt(int p, int vocab) {
  std::vector<int32_t> v(p);
  for (int i = 0; i < p; i++) v[i] = (int32_t)((13 + 7919ull * (uint64_t)i) % (uint64_t)vocab);
  return v;
}

std::string join(const std::vector<int32_t>& v) {
  std::string s = "[";
  for (size_t i = 0; i < v.size(); i++) s += (i ? " " : "") + std::to_string(v[i]);
  return s + "]";
}

// ------------------------------------------------------------ reference files

struct Record {
  uint32_t kind = 0;  // 0 f32, 1 i32
  std::vector<uint32_t> bits;
  std::vector<float> f32() const {
    std::vector<float> v(bits.size());
    memcpy(v.data(), bits.data(), bits.size() * 4);
    return v;
  }
  std::vector<int32_t> i32() const {
    std::vector<int32_t> v(bits.size());
    memcpy(v.data(), bits.data(), bits.size() * 4);
    return v;
  }
};

const char kMagic[8] = {'L', 'L', 'M', 'R', 'E', 'F', '0', '1'};

std::map<std::string, Record> read_ref(const std::string& path) {
  FILE* fp = fopen(path.c_str(), "rb");
  if (!fp) die("cannot open reference file " + path);
  char magic[8];
  if (fread(magic, 1, 8, fp) != 8 || memcmp(magic, kMagic, 8) != 0) die(path + ": not a reference file (LLMREF01)");
  std::map<std::string, Record> out;
  for (;;) {
    uint32_t nl;
    size_t got = fread(&nl, 4, 1, fp);
    if (got == 0) break;
    if (nl == 0 || nl > 256) die(path + ": bad record name length");
    std::string name(nl, '\0');
    Record r;
    uint64_t count;
    if (fread(&name[0], 1, nl, fp) != nl || fread(&r.kind, 4, 1, fp) != 1 || fread(&count, 8, 1, fp) != 1)
      die(path + ": truncated record header");
    if (r.kind > 1 || count > (1ull << 31)) die(path + ": bad record " + name);
    r.bits.resize(count);
    if (count && fread(r.bits.data(), 4, count, fp) != count) die(path + ": truncated record " + name);
    out[name] = std::move(r);
  }
  fclose(fp);
  return out;
}

struct RefWriter {
  FILE* fp;
  explicit RefWriter(const std::string& path) {
    fp = fopen(path.c_str(), "wb");
    if (!fp) die("cannot create " + path);
    fwrite(kMagic, 1, 8, fp);
  }
  void put(const std::string& name, uint32_t kind, const void* data, uint64_t count) {
    uint32_t nl = (uint32_t)name.size();
    fwrite(&nl, 4, 1, fp);
    fwrite(name.data(), 1, nl, fp);
    fwrite(&kind, 4, 1, fp);
    fwrite(&count, 8, 1, fp);
    fwrite(data, 4, count, fp);
  }
  ~RefWriter() {
    if (fclose(fp) != 0) die("writing the reference file failed");
  }
};

// ------------------------------------------------------------ model

struct Model {
  llm_gpu* g = nullptr;
  llmhip_model* m = nullptr;
  llmhip_config cfg{};
  int ctx = 0;
  ~Model() {
    if (g) llm_gpu_free(g);
  }
};

void open_model(const Flags& f, Model* md) {
  auto t0 = std::chrono::steady_clock::now();
  llm_gguf* gf = nullptr;
  int kind = 0;
  check_rc(llm_gguf_parse_file(f.model.c_str(), &gf, &kind));
  uint64_t nt, nkv, doff, align;
  uint32_t ver;
  check_rc(llm_gguf_info(gf, &nt, &nkv, &doff, &align, &ver));
  FILE* fp = fopen(f.model.c_str(), "rb");
  long long size = 0;
  if (fp) {
    fseek(fp, 0, SEEK_END);
    size = ftell(fp);
    fclose(fp);
  }
  printf("header: %llu tensors, %lld bytes, parsed in %.0f ms\n", (unsigned long long)nt, size, ms_since(t0));
  llm_gguf_free(gf);

  int ndev = 0;
  if (llmhip_device_count(&ndev) != 0 || ndev == 0) {
    printf("no GPU: %s\n", ndev == 0 ? "no HIP device" : llmhip_last_error());
    exit(2);
  }
  llmhip_limits lim;
  check_rc(llmhip_device_limits(f.device, &lim));
  printf("limits: workgroup size %u, %u invocations, %u B shared, %u groups/dim, binding %llu, memory %llu\n",
         lim.max_invocations_per_workgroup, lim.max_invocations_per_workgroup, lim.max_workgroup_storage,
         lim.max_workgroups_per_dimension, (unsigned long long)lim.max_binding_size,
         (unsigned long long)lim.memory_budget);
  check_rc(llm_set_decode_batch(f.batch));
  check_rc(llm_set_prefill_batch(f.prefillbatch));
  check_rc(llm_set_f16kv(f.f16kv ? 1 : 0));
  check_rc(llm_set_exact_ggml(f.exact ? 1 : 0));
  t0 = std::chrono::steady_clock::now();
  check_rc(llm_new_gpu(f.device, &lim, f.model.c_str(), f.ctx, &md->g));
  md->m = llm_gpu_model(md->g);
  check_rc(llm_gpu_config(md->g, &md->cfg, &md->ctx));
  llmhip_stats st;
  check_rc(llmhip_model_stats(md->m, &st));
  printf("load: %.0f ms, GPU memory %llu bytes, %lld submits\n", ms_since(t0),
         (unsigned long long)llmhip_model_memory_used(md->m), (long long)st.submits);
  if (!f.skip.empty()) check_rc(llmhip_model_set_skip(md->m, f.skip.c_str()));
}

std::vector<int32_t> prompt_of(const Flags& f, const Model& md) {
  std::vector<int32_t> ids = parse_ids(f.ids);
  for (const std::string& a : f.args) {
    std::vector<int32_t> more = parse_ids(a);
    ids.insert(ids.end(), more.begin(), more.end());
  }
  if (ids.empty()) ids = synthetic_prompt(f.p, md.cfg.vocab);
  return ids;
}

struct Collect {
  std::vector<int32_t> toks;
};

int collect(int32_t tok, void* user) {
  ((Collect*)user)->toks.push_back(tok);
  return 1;
}

std::vector<int32_t> generate(Model& md, const std::vector<int32_t>& prompt, int n, llm_timing* tm) {
  Collect c;
  check_rc(llm_gpu_generate(md.g, prompt.data(), (int)prompt.size(), n, -1, collect, &c, tm));
  return c.toks;
}

std::vector<float> prefill_logits(Model& md, const std::vector<int32_t>& prompt) {
  std::vector<float> out(md.cfg.vocab);
  check_rc(llm_gpu_prefill_logits(md.g, prompt.data(), (int)prompt.size(), out.data()));
  return out;
}

int argmax(const std::vector<float>& l) {  // cpu.go:389-397: the first maximum; NaN never wins
  int best = 0;
  for (size_t i = 0; i < l.size(); i++)
    if (l[i] > l[best]) best = (int)i;
  return best;
}

void report(const llm_timing& tm) {
  double pre = tm.prefill_ns * 1e-6, dec = tm.decode_ns * 1e-6;
  printf("prefill: %lld tokens in %.1f ms = %.1f tok/s\n", (long long)tm.prompt_tokens, pre,
         tm.prompt_tokens / (pre * 1e-3));
  printf("decode: %lld tokens in %.1f ms = %.1f tok/s (%lld submits, %lld dispatches in all)\n",
         (long long)tm.generated, dec, tm.generated / (dec * 1e-3), (long long)tm.submits,
         (long long)tm.dispatches);
  if (tm.generated > 1)
    printf("decode per token: %.2f ms recording, %.2f ms in submit (launch, GPU, read-back)\n",
           tm.record_ns * 1e-6 / (double)(tm.generated - 1), tm.submit_ns * 1e-6 / (double)(tm.generated - 1));
}

// ------------------------------------------------------------ modes

int mode_run(const Flags& f) {
  Model md;
  open_model(f, &md);
  std::vector<int32_t> ids = prompt_of(f, md);
  llm_timing tm;
  std::vector<int32_t> out = generate(md, ids, f.n, &tm);
  printf("prompt: %s\ntokens: %s\n", join(ids).c_str(), join(out).c_str());
  report(tm);
  return 0;
}

int mode_check(const Flags& f) {
  if (f.ref.empty()) die("check needs -ref FILE (the CPU path's logits and tokens)");
  std::map<std::string, Record> ref = read_ref(f.ref);
  if (!ref.count("logits") || !ref.count("tokens")) die(f.ref + ": check needs the records logits and tokens");
  Model md;
  open_model(f, &md);
  std::vector<int32_t> ids = ref.count("prompt") ? ref["prompt"].i32() : prompt_of(f, md);
  std::vector<float> cl = ref["logits"].f32();
  std::vector<int32_t> want = ref["tokens"].i32();
  if ((int)cl.size() != md.cfg.vocab) die("reference logits have " + std::to_string(cl.size()) + " entries, vocab is " +
                                          std::to_string(md.cfg.vocab));
  int n = std::min<int>(f.n, (int)want.size());
  want.resize(n);
  std::vector<float> gl = prefill_logits(md, ids);
  double max_abs = 0, max_ref = 0;
  for (size_t i = 0; i < cl.size(); i++) {
    max_abs = std::max(max_abs, std::fabs((double)gl[i] - (double)cl[i]));
    max_ref = std::max(max_ref, std::fabs((double)cl[i]));
  }
  double rel = max_ref > 0 ? max_abs / max_ref : max_abs;
  printf("logits: max |gpu-cpu| = %.3e, max |cpu| = %.3f, relative %.3e, argmax gpu %d cpu %d\n", max_abs, max_ref, rel,
         argmax(gl), argmax(cl));
  std::vector<int32_t> got = generate(md, ids, n, nullptr);
  int eq = 0;
  while (eq < (int)got.size() && eq < (int)want.size() && got[eq] == want[eq]) eq++;
  printf("gpu tokens: %s\ncpu tokens: %s\nequal prefix: %d of %d\n", join(got).c_str(), join(want).c_str(), eq, n);
  if (rel > f.tol || eq < n) {
    printf("outside tolerance (relative %.1e, all %d tokens equal)\n", f.tol, n);
    return 3;
  }
  return 0;
}

int mode_bench(const Flags& f) {
  Model md;
  open_model(f, &md);
  std::vector<int32_t> prompt = prompt_of(f, md);
  std::vector<double> pre, dec;
  for (int i = 0; i < f.rounds + 1; i++) {  // the first round warms up
    llm_timing tm;
    generate(md, prompt, f.n, &tm);
    if (i == 0) continue;
    pre.push_back(tm.prompt_tokens / (tm.prefill_ns * 1e-9));
    dec.push_back(tm.generated / (tm.decode_ns * 1e-9));
    printf("round %d: prefill %.1f tok/s, decode %.1f tok/s\n", i, pre.back(), dec.back());
    report(tm);
  }
  if (pre.empty()) die("bench needs -rounds >= 1");
  std::sort(pre.begin(), pre.end());
  std::sort(dec.begin(), dec.end());
  printf("bench p=%d n=%d rounds=%d: prefill median %.1f (min %.1f max %.1f) tok/s, decode median %.1f (min %.1f max "
         "%.1f) tok/s\n",
         (int)prompt.size(), f.n, f.rounds, pre[pre.size() / 2], pre.front(), pre.back(), dec[dec.size() / 2],
         dec.front(), dec.back());
  return 0;
}

int mode_trace(const Flags& f) {
  if (f.ref.empty()) die("trace needs -ref FILE (the CPU path's x.<layers> records)");
  std::map<std::string, Record> ref = read_ref(f.ref);
  Model md;
  open_model(f, &md);
  std::vector<int32_t> ids = ref.count("prompt") ? ref["prompt"].i32() : prompt_of(f, md);
  ids.resize(1);
  int traced = 0;
  for (const auto& kv : ref) {
    if (kv.first.rfind("x.", 0) != 0) continue;
    int l = atoi(kv.first.c_str() + 2);
    std::vector<float> want = kv.second.f32();
    if ((int)want.size() != md.cfg.embd) die(kv.first + ": not one residual vector");
    check_rc(llmhip_model_set_layers(md.m, l));
    std::vector<float> logits(md.cfg.vocab);
    int rc = llm_gpu_prefill_logits(md.g, ids.data(), 1, logits.data());
    if (rc != 0 && (l == 0 || l >= md.cfg.layers)) die(llmhip_last_error());
    std::vector<float> got(want.size()), st(2), tk(2);
    check_rc(llm_gpu_peek(md.g, "x", got.data(), got.size()));
    check_rc(llm_gpu_peek(md.g, "state", st.data(), 2));
    check_rc(llm_gpu_peek(md.g, "tokens", tk.data(), 2));
    double max_abs = 0, max_ref = 0;
    for (size_t i = 0; i < want.size(); i++) {
      max_abs = std::max(max_abs, std::fabs((double)got[i] - (double)want[i]));
      max_ref = std::max(max_ref, std::fabs((double)want[i]));
    }
    uint32_t sb[2], tb[2];
    memcpy(sb, st.data(), 8);
    memcpy(tb, tk.data(), 8);
    printf("state bits %x %x tokens bits %x %x\n", sb[0], sb[1], tb[0], tb[1]);
    printf("layers %d: x max |gpu-cpu| = %.3e (max |x| %.3f); gpu [%g %g %g %g] cpu [%g %g %g %g]\n", l, max_abs,
           max_ref, got[0], got[1], got[2], got[3], want[0], want[1], want[2], want[3]);
    traced++;
  }
  check_rc(llmhip_model_set_layers(md.m, 0));
  if (!traced) die(f.ref + ": no x.<layers> records");
  return 0;
}

int mode_dump(const Flags& f) {
  if (f.out.empty()) die("dump needs -out FILE");
  Model md;
  open_model(f, &md);
  std::vector<int32_t> ids = prompt_of(f, md);
  std::vector<float> logits = prefill_logits(md, ids);
  std::vector<int32_t> toks = generate(md, ids, f.n, nullptr);
  std::vector<std::pair<std::string, std::vector<float>>> xs;
  for (int32_t l : parse_ids(f.layers)) {
    check_rc(llmhip_model_set_layers(md.m, l));
    std::vector<float> lg(md.cfg.vocab), x(md.cfg.embd);
    int rc = llm_gpu_prefill_logits(md.g, ids.data(), 1, lg.data());
    if (rc != 0 && (l == 0 || l >= md.cfg.layers)) die(llmhip_last_error());
    check_rc(llm_gpu_peek(md.g, "x", x.data(), x.size()));
    xs.push_back({"x." + std::to_string(l), x});
  }
  check_rc(llmhip_model_set_layers(md.m, 0));
  RefWriter w(f.out);
  w.put("prompt", 1, ids.data(), ids.size());
  w.put("logits", 0, logits.data(), logits.size());
  w.put("tokens", 1, toks.data(), toks.size());
  for (auto& x : xs) w.put(x.first, 0, x.second.data(), x.second.size());
  printf("wrote %s: prompt %zu ids, %zu logits, %zu tokens, %zu residual vectors\n", f.out.c_str(), ids.size(),
         logits.size(), toks.size(), xs.size());
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) die("usage: llm-generate run|check|bench|trace|dump [flags] [TOKEN IDS]");
  std::string mode = argv[1];
  Flags f = parse_flags(argc - 2, argv + 2);
  if (mode == "run") return mode_run(f);
  if (mode == "check") return mode_check(f);
  if (mode == "bench") return mode_bench(f);
  if (mode == "trace") return mode_trace(f);
  if (mode == "dump") return mode_dump(f);
  die("unknown mode \"" + mode + "\"");
}
