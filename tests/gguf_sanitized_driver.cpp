// The GGUF header parser and ConfigFrom (llm_amd/csrc/gguf.cpp), built on its
// own with AddressSanitizer and UndefinedBehaviorSanitizer by
// tests/test_gguf_sanitized.py, then run over every input file named on the
// command line and `mutations` seeded mutations of each (byte flips, 64-bit
// fields overwritten with extreme values, truncations, extensions): every
// input either parses, with every accessor then exercised, or is refused.
// A sanitizer report aborts the run with a non-zero status.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../llm_amd/csrc/gguf.h"

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static uint64_t next() {  // xorshift64*
  g_rng ^= g_rng >> 12;
  g_rng ^= g_rng << 25;
  g_rng ^= g_rng >> 27;
  return g_rng * 0x2545F4914F6CDD1Dull;
}

static int ok = 0, refused = 0;

static void run(const std::vector<uint8_t>& d) {
  llm_gguf* g = nullptr;
  int kind = 0;
  // a copy of exactly the input's length, so that a read past it is reported
  std::vector<uint8_t> exact(d);
  const int rc = llm_gguf_parse_bytes(exact.empty() ? nullptr : exact.data(), exact.size(), &g, &kind);
  if (rc != 0) {
    if (kind < LLM_GGUF_MAGIC || kind > LLM_GGUF_IO) {
      fprintf(stderr, "refusal without a kind: %d (%s)\n", kind, llmhip_last_error());
      exit(3);
    }
    refused++;
    return;
  }
  ok++;
  uint64_t nt, nkv, off, al;
  uint32_t ver;
  llm_gguf_info(g, &nt, &nkv, &off, &al, &ver);
  for (uint64_t i = 0; i < nt; i++) {
    char name[64];
    uint32_t type, nd;
    uint64_t dims[4], toff, size, idx;
    llm_gguf_tensor_info(g, i, name, sizeof name, &type, &nd, dims, &toff, &size);
    if (off + toff + size > d.size()) {
      fprintf(stderr, "tensor %llu lies past the input\n", (unsigned long long)i);
      exit(3);
    }
    (void)llm_gguf_find_tensor(g, name, &idx);
  }
  uint64_t u;
  double f;
  char s[32];
  (void)llm_gguf_meta_uint(g, "llama.block_count", &u);
  (void)llm_gguf_meta_float(g, "llama.rope.freq_base", &f);
  (void)llm_gguf_meta_str(g, "general.architecture", s, sizeof s);
  llmhip_config c;
  (void)llm_config_from(g, &c);
  llm_gguf_free(g);
}

int main(int argc, char** argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: %s mutations file...\n", argv[0]);
    return 2;
  }
  const long muts = atol(argv[1]);
  for (int a = 2; a < argc; a++) {
    FILE* fp = fopen(argv[a], "rb");
    if (!fp) return 2;
    std::vector<uint8_t> base;
    uint8_t buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, fp)) > 0) base.insert(base.end(), buf, buf + n);
    fclose(fp);
    run(base);
    // mutate the header region (the tensor data never reaches the parser)
    const size_t span = std::min<size_t>(base.size(), 1 << 16);
    for (long m = 0; m < muts && span > 0; m++) {
      std::vector<uint8_t> d(base);
      const int flips = 1 + (int)(next() % 5);
      for (int i = 0; i < flips; i++) d[next() % span] = (uint8_t)next();
      if (next() % 4 == 0 && span >= 8) {  // a count, size or offset field set to an extreme
        static const uint64_t extreme[] = {0, 1, 0xFFFFFFFFull, 0x100000000ull, ~0ull, 1ull << 63, 0x7FFFFFFFFFFFFFFFull};
        const uint64_t v = extreme[next() % 7];
        memcpy(&d[next() % (span - 7)], &v, 8);
      }
      const uint64_t r = next() % 10;
      if (r < 3) d.resize(next() % (d.size() + 1));
      else if (r == 3) for (int i = 0; i < 64; i++) d.push_back((uint8_t)next());
      run(d);
    }
  }
  printf("parsed %d, refused %d\n", ok, refused);
  return 0;
}
