// The GGUF header reader, ConfigFrom and their C-ABI (llm_gguf_*,
// llm_config_from).  Host code only (gguf.h).
#include "gguf.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>

namespace llm {

using llmhip::set_error;

namespace gguf {

// gguf.Type.BlockSize, gguf/gguf.go:72-92.
bool block_size(uint32_t t, uint64_t* elems, uint64_t* bytes) {
  switch (t) {
    case 0: *elems = 1; *bytes = 4; return true;
    case 1: *elems = 1; *bytes = 2; return true;
    case 2: *elems = 32; *bytes = 18; return true;
    case 3: *elems = 32; *bytes = 20; return true;
    case 6: *elems = 32; *bytes = 22; return true;
    case 7: *elems = 32; *bytes = 24; return true;
    case 8: *elems = 32; *bytes = 34; return true;
    case 14: *elems = 256; *bytes = 210; return true;
  }
  return false;
}

struct Reader {
  ReaderAt r;
  std::vector<uint8_t> win;
  uint64_t win_off = 0, pos = 0, lim = 0;
  int* kind;
  static constexpr uint64_t ReadAhead = 1 << 20;

  // reader.read, gguf/gguf.go:147-179: bounded by lim, through a window.
  int read(void* p, uint64_t n) {
    if (pos + n > lim) {
      *kind = LLM_GGUF_BOUND;
      return set_error(LLMHIP_ERR_FORMAT, "gguf: a size or count exceeds its bound: header runs past byte %llu",
                       (unsigned long long)lim);
    }
    if (pos < win_off || pos + n > win_off + win.size()) {
      uint64_t want = std::min<uint64_t>(std::max<uint64_t>(ReadAhead, n), lim - pos);
      win.resize(want);
      int64_t got = r(win.data(), want, pos);
      if (got < 0) got = 0;
      win.resize((size_t)got);
      win_off = pos;
      if ((uint64_t)got < n) {
        *kind = LLM_GGUF_IO;
        return set_error(LLMHIP_ERR_IO, "gguf: unexpected EOF");
      }
    }
    memcpy(p, win.data() + (pos - win_off), n);
    pos += n;
    return 0;
  }
  int u32(uint32_t* v) { return read(v, 4); }
  int u64(uint64_t* v) { return read(v, 8); }
  int str(std::string* s) {
    uint64_t n;
    LLM_TRY(u64(&n));
    if (n > MaxString) {
      *kind = LLM_GGUF_BOUND;
      return set_error(LLMHIP_ERR_FORMAT, "gguf: a size or count exceeds its bound: string of %llu bytes",
                       (unsigned long long)n);
    }
    s->resize(n);
    return n ? read(&(*s)[0], n) : 0;
  }
  // reader.value, gguf/gguf.go:210-289
  int value(uint32_t t, int depth, Value* v) {
    uint8_t b1;
    uint16_t b2;
    uint32_t b4;
    uint64_t b8;
    switch (t) {
      case 0: LLM_TRY(read(&b1, 1)); v->kind = K_UINT; v->u = b1; return 0;
      case 1: LLM_TRY(read(&b1, 1)); v->kind = K_INT; v->i = (int8_t)b1; return 0;
      case 7: LLM_TRY(read(&b1, 1)); v->kind = K_BOOL; v->b = b1 != 0; return 0;
      case 2: LLM_TRY(read(&b2, 2)); v->kind = K_UINT; v->u = b2; return 0;
      case 3: LLM_TRY(read(&b2, 2)); v->kind = K_INT; v->i = (int16_t)b2; return 0;
      case 4: LLM_TRY(u32(&b4)); v->kind = K_UINT; v->u = b4; return 0;
      case 5: LLM_TRY(u32(&b4)); v->kind = K_INT; v->i = (int32_t)b4; return 0;
      case 6: {
        LLM_TRY(u32(&b4));
        float f;
        memcpy(&f, &b4, 4);
        v->kind = K_FLOAT;
        v->f = f;
        return 0;
      }
      case 10: LLM_TRY(u64(&b8)); v->kind = K_UINT; v->u = b8; return 0;
      case 11: LLM_TRY(u64(&b8)); v->kind = K_INT; v->i = (int64_t)b8; return 0;
      case 12: LLM_TRY(u64(&b8)); v->kind = K_FLOAT; memcpy(&v->f, &b8, 8); return 0;
      case 8: v->kind = K_STRING; return str(&v->s);
      case 9: {
        if (depth > 0) {
          *kind = LLM_GGUF_FORMAT;
          return set_error(LLMHIP_ERR_FORMAT, "gguf: malformed header: nested array");
        }
        uint32_t et;
        uint64_t n;
        LLM_TRY(u32(&et));
        LLM_TRY(u64(&n));
        if (n > MaxArray) {
          *kind = LLM_GGUF_BOUND;
          return set_error(LLMHIP_ERR_FORMAT, "gguf: a size or count exceeds its bound: array of %llu",
                           (unsigned long long)n);
        }
        if (n > lim - pos) {  // each element takes at least a byte
          *kind = LLM_GGUF_BOUND;
          return set_error(LLMHIP_ERR_FORMAT, "gguf: a size or count exceeds its bound: array of %llu past the header",
                           (unsigned long long)n);
        }
        v->kind = K_ARRAY;
        v->n = n;
        for (uint64_t i = 0; i < n; i++) {
          Value e;
          LLM_TRY(value(et, depth + 1, &e));
        }
        return 0;
      }
    }
    *kind = LLM_GGUF_FORMAT;
    return set_error(LLMHIP_ERR_FORMAT, "gguf: malformed header: value type %u", t);
  }
};

// Parse, gguf/gguf.go:292-407.
int parse(ReaderAt r, uint64_t size, File* f, int* kind) {
  *kind = 0;
  Reader rd{r, {}, 0, 0, std::min(size, MaxHeader), kind};
  char magic[4];
  LLM_TRY(rd.read(magic, 4));
  if (memcmp(magic, "GGUF", 4) != 0) {
    *kind = LLM_GGUF_MAGIC;
    return set_error(LLMHIP_ERR_FORMAT, "gguf: bad magic");
  }
  uint32_t ver;
  LLM_TRY(rd.u32(&ver));
  if (ver != 3) {
    *kind = LLM_GGUF_VERSION;
    return set_error(LLMHIP_ERR_FORMAT, "gguf: unsupported version: %u", ver);
  }
  uint64_t nt, nkv;
  LLM_TRY(rd.u64(&nt));
  LLM_TRY(rd.u64(&nkv));
  if (nt > MaxTensors || nkv > MaxKV) {
    *kind = LLM_GGUF_BOUND;
    return set_error(LLMHIP_ERR_FORMAT, "gguf: a size or count exceeds its bound: %llu tensors, %llu metadata entries",
                     (unsigned long long)nt, (unsigned long long)nkv);
  }
  f->version = ver;
  f->size = size;
  for (uint64_t i = 0; i < nkv; i++) {
    std::string k;
    uint32_t t;
    LLM_TRY(rd.str(&k));
    LLM_TRY(rd.u32(&t));
    Value v;
    LLM_TRY(rd.value(t, 0, &v));
    f->meta[k] = v;
  }
  f->alignment = 32;
  auto al = f->meta.find("general.alignment");
  if (al != f->meta.end()) {
    const Value& a = al->second;
    if (a.kind != K_UINT || a.u == 0 || a.u > MaxAlignment || a.u % 8 != 0) {
      *kind = LLM_GGUF_FORMAT;
      return set_error(LLMHIP_ERR_FORMAT, "gguf: malformed header: general.alignment");
    }
    f->alignment = a.u;
  }
  for (uint64_t i = 0; i < nt; i++) {
    Tensor t;
    LLM_TRY(rd.str(&t.name));
    uint32_t nd;
    LLM_TRY(rd.u32(&nd));
    if (nd == 0 || nd > MaxDims) {
      *kind = LLM_GGUF_FORMAT;
      return set_error(LLMHIP_ERR_FORMAT, "gguf: malformed header: tensor \"%s\" has %u dimensions", t.name.c_str(),
                       nd);
    }
    uint64_t elems = 1;
    for (uint32_t j = 0; j < nd; j++) {
      uint64_t d;
      LLM_TRY(rd.u64(&d));
      if (d == 0 || d > (1ull << 32)) {
        *kind = LLM_GGUF_BOUND;
        return set_error(LLMHIP_ERR_FORMAT, "gguf: a size or count exceeds its bound: tensor \"%s\" dimension %llu",
                         t.name.c_str(), (unsigned long long)d);
      }
      if (elems > (1ull << 62) / d) {
        *kind = LLM_GGUF_BOUND;
        return set_error(LLMHIP_ERR_FORMAT, "gguf: a size or count exceeds its bound: tensor \"%s\" too large",
                         t.name.c_str());
      }
      elems *= d;
      t.dims.push_back(d);
    }
    LLM_TRY(rd.u32(&t.type));
    LLM_TRY(rd.u64(&t.offset));
    uint64_t be, bb;
    if (!block_size(t.type, &be, &bb)) {
      *kind = LLM_GGUF_FORMAT;
      return set_error(LLMHIP_ERR_FORMAT, "gguf: malformed header: tensor \"%s\" has unsupported ggml type %u",
                       t.name.c_str(), t.type);
    }
    if (t.dims[0] % be != 0) {
      *kind = LLM_GGUF_FORMAT;
      return set_error(LLMHIP_ERR_FORMAT, "gguf: malformed header: tensor \"%s\" row of %llu is not a multiple of %llu",
                       t.name.c_str(), (unsigned long long)t.dims[0], (unsigned long long)be);
    }
    t.size = elems / be * bb;
    if (f->by_name.count(t.name)) {
      *kind = LLM_GGUF_FORMAT;
      return set_error(LLMHIP_ERR_FORMAT, "gguf: malformed header: duplicate tensor \"%s\"", t.name.c_str());
    }
    f->by_name[t.name] = f->tensors.size();
    f->tensors.push_back(t);
  }
  f->data_offset = (rd.pos + f->alignment - 1) / f->alignment * f->alignment;
  for (auto& t : f->tensors) {
    if (t.offset % f->alignment != 0) {
      *kind = LLM_GGUF_FORMAT;
      return set_error(LLMHIP_ERR_FORMAT, "gguf: malformed header: tensor \"%s\" offset %llu is not aligned",
                       t.name.c_str(), (unsigned long long)t.offset);
    }
    if (t.offset > size || f->data_offset > size - t.offset || t.size > size - f->data_offset - t.offset) {
      *kind = LLM_GGUF_BOUND;
      return set_error(LLMHIP_ERR_FORMAT, "gguf: a size or count exceeds its bound: tensor \"%s\" lies past the end of the file",
                       t.name.c_str());
    }
  }
  return 0;
}

// File.Uint / Float / Str, gguf/gguf.go:410-432.
bool meta_uint(const File& f, const std::string& k, uint64_t* v) {
  auto it = f.meta.find(k);
  if (it == f.meta.end()) return false;
  if (it->second.kind == K_UINT) {
    *v = it->second.u;
    return true;
  }
  if (it->second.kind == K_INT && it->second.i >= 0) {
    *v = (uint64_t)it->second.i;
    return true;
  }
  return false;
}
bool meta_float(const File& f, const std::string& k, double* v) {
  auto it = f.meta.find(k);
  if (it == f.meta.end() || it->second.kind != K_FLOAT) return false;
  *v = it->second.f;
  return true;
}
bool meta_str(const File& f, const std::string& k, std::string* v) {
  auto it = f.meta.find(k);
  if (it == f.meta.end() || it->second.kind != K_STRING) return false;
  *v = it->second.s;
  return true;
}

}  // namespace gguf

// ConfigFrom, config.go:29-73.
int config_from(const gguf::File& f, llmhip_config* c) {
  std::string arch;
  gguf::meta_str(f, "general.architecture", &arch);
  if (arch != "llama" && arch != "qwen2")
    return set_error(LLMHIP_ERR_FORMAT, "llm: architecture \"%s\" is not supported (llama and qwen2 only)",
                     arch.c_str());
  auto u = [&](const char* k) {
    uint64_t v = 0;
    gguf::meta_uint(f, arch + "." + k, &v);
    return (int64_t)v;
  };
  memset(c, 0, sizeof *c);
  c->arch = arch == "qwen2";
  c->rope_neox = arch == "qwen2";
  int64_t layers = u("block_count"), embd = u("embedding_length"), ff = u("feed_forward_length"),
          heads = u("attention.head_count"), kvh = u("attention.head_count_kv"), ctx = u("context_length");
  if (kvh == 0) kvh = heads;
  if (layers <= 0 || embd <= 0 || ff <= 0 || heads <= 0 || embd % heads != 0 || heads % kvh != 0 ||
      layers > (1 << 20) || embd > (1 << 24) || ff > (1 << 24) || ctx > (1ll << 30))
    return set_error(LLMHIP_ERR_FORMAT, "llm: implausible %s hyperparameters", arch.c_str());
  c->layers = (int32_t)layers;
  c->embd = (int32_t)embd;
  c->ff = (int32_t)ff;
  c->heads = (int32_t)heads;
  c->kv_heads = (int32_t)kvh;
  c->ctx = (int32_t)ctx;
  c->head_dim = c->embd / c->heads;
  int64_t rd = u("rope.dimension_count");
  if (rd != 0 && rd != c->head_dim)
    return set_error(LLMHIP_ERR_FORMAT, "llm: rope.dimension_count %lld differs from the head size %d", (long long)rd,
                     c->head_dim);
  for (const char* k : {".rope.scaling.type", ".rope.scaling.factor"})
    if (f.meta.count(arch + k))
      return set_error(LLMHIP_ERR_FORMAT, "llm: rope scaling (%s%s) is not supported", arch.c_str(), k);
  double rb = 10000, eps = 0;
  gguf::meta_float(f, arch + ".rope.freq_base", &rb);
  gguf::meta_float(f, arch + ".attention.layer_norm_rms_epsilon", &eps);
  c->rope_base = (float)rb;
  c->eps = (float)eps;
  auto te = f.by_name.find("token_embd.weight");
  if (te == f.by_name.end()) return set_error(LLMHIP_ERR_FORMAT, "llm: no token_embd.weight");
  const gguf::Tensor& t = f.tensors[te->second];
  if (t.dims.size() < 2) return set_error(LLMHIP_ERR_FORMAT, "llm: token_embd.weight is not a matrix");
  c->vocab = (int32_t)t.dims[1];
  c->tied_output = f.by_name.count("output.weight") == 0;
  c->bias = f.by_name.count("blk.0.attn_q.bias") != 0;
  if ((c->bias != 0) != (arch == "qwen2"))
    return set_error(LLMHIP_ERR_FORMAT, "llm: %s with biases %s is not supported", arch.c_str(),
                     c->bias ? "true" : "false");
  return 0;
}

}  // namespace llm

using namespace llm;

int llm::parse_fd(int fd, llm_gguf** out, int* kind) {
  struct stat st;
  if (fstat(fd, &st) != 0) return set_error(LLMHIP_ERR_IO, "llm: stat failed");
  llm_gguf* g = new llm_gguf();
  int k = 0;
  int rc = gguf::parse(
      [fd](void* d, uint64_t n, uint64_t off) -> int64_t {
        uint64_t got = 0;
        while (got < n) {
          ssize_t r = pread(fd, (char*)d + got, n - got, (off_t)(off + got));
          if (r <= 0) break;
          got += (uint64_t)r;
        }
        return (int64_t)got;
      },
      (uint64_t)st.st_size, &g->f, &k);
  if (kind) *kind = k;
  if (rc) {
    delete g;
    return rc;
  }
  *out = g;
  return 0;
}

extern "C" {

int llm_gguf_parse_file(const char* path, llm_gguf** out, int* kind) {
  llmhip::clear_error();
  *out = nullptr;
  if (kind) *kind = 0;
  int fd = open(path, O_RDONLY);
  if (fd < 0) {
    if (kind) *kind = LLM_GGUF_IO;
    return set_error(LLMHIP_ERR_IO, "llm: cannot open %s", path);
  }
  int rc = parse_fd(fd, out, kind);
  close(fd);
  return rc;
}

int llm_gguf_parse_bytes(const void* data, uint64_t size, llm_gguf** out, int* kind) {
  llmhip::clear_error();
  *out = nullptr;
  llm_gguf* g = new llm_gguf();
  int k = 0;
  const uint8_t* p = (const uint8_t*)data;
  int rc = gguf::parse(
      [p, size](void* d, uint64_t n, uint64_t off) -> int64_t {
        if (off >= size) return 0;
        uint64_t m = std::min(n, size - off);
        memcpy(d, p + off, m);
        return (int64_t)m;
      },
      size, &g->f, &k);
  if (kind) *kind = k;
  if (rc) {
    delete g;
    return rc;
  }
  *out = g;
  return 0;
}

void llm_gguf_free(llm_gguf* g) { delete g; }

int llm_gguf_info(const llm_gguf* g, uint64_t* ntensors, uint64_t* nkv, uint64_t* data_offset, uint64_t* alignment,
                  uint32_t* version) {
  *ntensors = g->f.tensors.size();
  *nkv = g->f.meta.size();
  *data_offset = g->f.data_offset;
  *alignment = g->f.alignment;
  *version = g->f.version;
  return 0;
}

int llm_gguf_tensor_info(const llm_gguf* g, uint64_t i, char* name, uint64_t name_cap, uint32_t* type,
                         uint32_t* ndims, uint64_t* dims, uint64_t* offset, uint64_t* size) {
  if (i >= g->f.tensors.size()) return set_error(LLMHIP_ERR_ARG, "llm: tensor index %llu", (unsigned long long)i);
  const gguf::Tensor& t = g->f.tensors[i];
  if (name && name_cap) {
    size_t n = std::min<size_t>(t.name.size(), name_cap - 1);
    memcpy(name, t.name.data(), n);
    name[n] = 0;
  }
  *type = t.type;
  *ndims = (uint32_t)t.dims.size();
  for (size_t j = 0; j < 4; j++) dims[j] = j < t.dims.size() ? t.dims[j] : 1;
  *offset = t.offset;
  *size = t.size;
  return 0;
}

int llm_gguf_find_tensor(const llm_gguf* g, const char* name, uint64_t* index) {
  auto it = g->f.by_name.find(name);
  if (it == g->f.by_name.end()) return set_error(LLMHIP_ERR_ARG, "llm: no tensor %s", name);
  *index = it->second;
  return 0;
}

int llm_gguf_meta_uint(const llm_gguf* g, const char* key, uint64_t* v) { return gguf::meta_uint(g->f, key, v); }
int llm_gguf_meta_float(const llm_gguf* g, const char* key, double* v) { return gguf::meta_float(g->f, key, v); }
int llm_gguf_meta_str(const llm_gguf* g, const char* key, char* buf, uint64_t cap) {
  std::string s;
  if (!gguf::meta_str(g->f, key, &s)) return 0;
  if (buf && cap) {
    size_t n = std::min<size_t>(s.size(), cap - 1);
    memcpy(buf, s.data(), n);
    buf[n] = 0;
  }
  return 1;
}

int llm_config_from(const llm_gguf* g, llmhip_config* out) {
  llmhip::clear_error();
  return config_from(g->f, out);
}

}  // extern "C"
