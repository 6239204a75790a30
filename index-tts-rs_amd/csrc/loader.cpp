// Gpt::load_from_path for the gpt_int8 safetensors checkpoint (crates/core/src/models/gpt.rs:522,
// crates/core/src/models/loader.rs:768-856 and read_header 1410-1458).
//
// The file is memory-mapped and every tensor is handed to itts_gpt_create as a pointer into
// the mapping (no host copy): the MLX U32 code words are the uint8 [N][K*bits/8] layout the
// device uses, and the group parameters keep the file's dtype (F32 in the shipped checkpoint,
// F16 accepted).  Validation follows the reference: the 8-byte little-endian header length
// (non-zero, at most 100,000,000 bytes, inside the file), the JSON header, the data section
// ending exactly at the end of the file, then every tensor by name with its exact shape
// (Gpt::from_weights gpt.rs:477-515, Gpt2Block::from_weights 269-323, QuantizedLinear
// 229-247).  The decoder shape is read from the file (the reference fixes it in gpt.rs:31-54).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/itts_hip.h"

namespace itts {
itts_status set_error_text(itts_status st, const char *msg);  // runtime.cpp
}
using itts::set_error_text;

namespace {

constexpr size_t kMaxHeaderBytes = 100000000;  // loader.rs:1402

itts_status weight_error(const std::string &artifact, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  const std::string msg = "weight load error in `" + artifact + "`: " + buf;
  return set_error_text(ITTS_E_WEIGHT, msg.c_str());
}

struct TensorInfo {
  std::string dtype;
  std::vector<size_t> shape;
  size_t begin = 0, end = 0;  // data offsets
};

// Minimal JSON reader for the safetensors header: an object of name -> {"dtype": string,
// "shape": [ints], "data_offsets": [int, int]} plus an optional "__metadata__" object of
// strings.  Anything else is a parse error.
class Header {
 public:
  Header(const char *p, size_t n) : p_(p), e_(p + n) {}
  bool parse(std::map<std::string, TensorInfo> &out, std::string &err) {
    ws();
    if (!eat('{')) return fail(err, "expected '{'");
    ws();
    if (eat('}')) return true;
    while (true) {
      std::string key;
      if (!str(key)) return fail(err, "expected a tensor name");
      ws();
      if (!eat(':')) return fail(err, "expected ':'");
      ws();
      if (key == "__metadata__") {
        if (!skip_string_object()) return fail(err, "bad __metadata__");
      } else {
        TensorInfo t;
        if (!tensor(t)) return fail(err, ("bad entry for tensor `" + key + "`").c_str());
        out[key] = t;
      }
      ws();
      if (eat(',')) {
        ws();
        continue;
      }
      if (eat('}')) break;
      return fail(err, "expected ',' or '}'");
    }
    ws();
    if (p_ != e_) return fail(err, "trailing bytes after the header object");
    return true;
  }

 private:
  const char *p_, *e_;
  bool fail(std::string &err, const char *m) {
    err = m;
    return false;
  }
  void ws() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) p_++;
  }
  bool eat(char c) {
    if (p_ < e_ && *p_ == c) {
      p_++;
      return true;
    }
    return false;
  }
  bool str(std::string &s) {
    if (!eat('"')) return false;
    s.clear();
    while (p_ < e_ && *p_ != '"') {
      if (*p_ == '\\') {
        if (++p_ >= e_) return false;
        const char c = *p_;
        if (c == 'u') return false;  // tensor names are ASCII
        s.push_back(c == 'n' ? '\n' : c == 't' ? '\t' : c);
      } else {
        s.push_back(*p_);
      }
      p_++;
    }
    return eat('"');
  }
  bool uint(size_t &v) {
    if (p_ >= e_ || *p_ < '0' || *p_ > '9') return false;
    v = 0;
    while (p_ < e_ && *p_ >= '0' && *p_ <= '9') {
      const size_t d = (size_t)(*p_ - '0');
      if (v > (SIZE_MAX - d) / 10) return false;
      v = v * 10 + d;
      p_++;
    }
    return true;
  }
  bool uints(std::vector<size_t> &v) {
    if (!eat('[')) return false;
    ws();
    v.clear();
    if (eat(']')) return true;
    while (true) {
      size_t x;
      if (!uint(x)) return false;
      v.push_back(x);
      ws();
      if (eat(',')) {
        ws();
        continue;
      }
      return eat(']');
    }
  }
  bool tensor(TensorInfo &t) {
    if (!eat('{')) return false;
    bool have_dtype = false, have_shape = false, have_off = false;
    ws();
    while (true) {
      std::string k;
      if (!str(k)) return false;
      ws();
      if (!eat(':')) return false;
      ws();
      if (k == "dtype") {
        if (!str(t.dtype)) return false;
        have_dtype = true;
      } else if (k == "shape") {
        if (!uints(t.shape)) return false;
        have_shape = true;
      } else if (k == "data_offsets") {
        std::vector<size_t> o;
        if (!uints(o) || o.size() != 2 || o[1] < o[0]) return false;
        t.begin = o[0];
        t.end = o[1];
        have_off = true;
      } else {
        return false;
      }
      ws();
      if (eat(',')) {
        ws();
        continue;
      }
      if (!eat('}')) return false;
      break;
    }
    return have_dtype && have_shape && have_off;
  }
  bool skip_string_object() {
    if (!eat('{')) return false;
    ws();
    if (eat('}')) return true;
    while (true) {
      std::string k, v;
      if (!str(k)) return false;
      ws();
      if (!eat(':')) return false;
      ws();
      if (!str(v)) return false;
      ws();
      if (eat(',')) {
        ws();
        continue;
      }
      return eat('}');
    }
  }
};

size_t dtype_size(const std::string &d) {
  if (d == "F32" || d == "U32" || d == "I32") return 4;
  if (d == "F16" || d == "BF16") return 2;
  return 0;
}

std::string shape_str(const std::vector<size_t> &s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); i++) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

struct Mapped {
  void *base = MAP_FAILED;
  size_t len = 0;
  ~Mapped() {
    if (base != MAP_FAILED) munmap(base, len);
  }
};

class Checkpoint {
 public:
  std::map<std::string, TensorInfo> tensors;
  const uint8_t *data = nullptr;  // start of the data section

  // The tensor `name` with exactly `shape` and one of the dtypes in `dtypes`
  // (tensor_array_shaped, loader.rs:316-331).
  itts_status get(const std::string &name, const std::vector<size_t> &shape, const char *dtypes,
                  const void **out, std::string *dtype_out = nullptr) const {
    auto it = tensors.find(name);
    if (it == tensors.end()) return weight_error(name, "missing required parameter tensor");
    const TensorInfo &t = it->second;
    if (t.shape != shape)
      return weight_error(name, "expected shape %s, found %s", shape_str(shape).c_str(), shape_str(t.shape).c_str());
    if (!strstr(dtypes, (t.dtype + ",").c_str()))
      return weight_error(name, "unsupported dtype %s (expected %s)", t.dtype.c_str(), dtypes);
    *out = data + t.begin;
    if (dtype_out) *dtype_out = t.dtype;
    return ITTS_OK;
  }
  bool has(const std::string &name) const { return tensors.count(name) != 0; }
  const TensorInfo *info(const std::string &name) const {
    auto it = tensors.find(name);
    return it == tensors.end() ? nullptr : &it->second;
  }
};

}  // namespace

extern "C" itts_status itts_gpt_load_safetensors(const char *path, itts_gpt **out) {
  const std::string artifact = "gpt_int8.safetensors";
  if (!path || !out) return set_error_text(ITTS_E_VALIDATION, "weight_path: null argument");
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return weight_error(artifact, "cannot open %s: %s", path, strerror(errno));
  struct stat st {};
  if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
    close(fd);
    return weight_error(artifact, "%s is not a regular file", path);
  }
  const size_t file_len = (size_t)st.st_size;
  if (file_len < 8) {
    close(fd);
    return weight_error(artifact, "safetensors file smaller than 8-byte header prefix");
  }
  Mapped m;
  m.len = file_len;
  m.base = mmap(nullptr, file_len, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m.base == MAP_FAILED) return weight_error(artifact, "mmap failed: %s", strerror(errno));
  const uint8_t *bytes = static_cast<const uint8_t *>(m.base);
  uint64_t header_len = 0;
  for (int i = 7; i >= 0; i--) header_len = (header_len << 8) | bytes[i];
  if (header_len == 0 || header_len > kMaxHeaderBytes)
    return weight_error(artifact, "invalid safetensors header length %llu", (unsigned long long)header_len);
  const size_t data_base = 8 + (size_t)header_len;
  if (data_base > file_len) return weight_error(artifact, "safetensors header length exceeds file size");
  Checkpoint ck;
  std::string perr;
  if (!Header(reinterpret_cast<const char *>(bytes + 8), (size_t)header_len).parse(ck.tensors, perr))
    return weight_error(artifact, "safetensors header parse failed: %s", perr.c_str());
  size_t data_len = 0;
  for (auto &kv : ck.tensors) {
    const TensorInfo &t = kv.second;
    const size_t es = dtype_size(t.dtype);
    size_t n = 1;
    for (size_t d : t.shape) n *= d;
    if (es && t.end - t.begin != n * es)
      return weight_error(kv.first, "data_offsets span %zu bytes for %s %s", t.end - t.begin, t.dtype.c_str(),
                          shape_str(t.shape).c_str());
    if (t.end > data_len) data_len = t.end;
  }
  if (data_base + data_len != file_len)
    return weight_error(artifact, "safetensors data section length does not match file size");
  ck.data = bytes + data_base;
  // shapes come from the file (the reference's constants, gpt.rs:31-54, for the shipped one)
  const TensorInfo *lnf = ck.info("gpt.ln_f.weight"), *te = ck.info("text_embedding.weight");
  const TensorInfo *le = ck.info("lang_embedding.weight"), *me = ck.info("mel_embedding.weight");
  const TensorInfo *mp = ck.info("mel_pos_embedding.emb.weight"), *tp = ck.info("text_pos_embedding.emb.weight");
  const TensorInfo *fcb = ck.info("gpt.h.0.mlp.c_fc.bias"), *hw = ck.info("mel_head.weight");
  struct Need {
    const TensorInfo *t;
    const char *name;
    size_t rank;
  } needs[] = {{lnf, "gpt.ln_f.weight", 1}, {te, "text_embedding.weight", 2}, {le, "lang_embedding.weight", 2},
               {me, "mel_embedding.weight", 2}, {mp, "mel_pos_embedding.emb.weight", 2},
               {tp, "text_pos_embedding.emb.weight", 2}, {fcb, "gpt.h.0.mlp.c_fc.bias", 1}, {hw, "mel_head.weight", 2}};
  for (const Need &nd : needs) {
    if (!nd.t) return weight_error(nd.name, "missing required parameter tensor");
    if (nd.t->shape.size() != nd.rank) return weight_error(nd.name, "unexpected rank %zu", nd.t->shape.size());
  }
  itts_config c{};
  const size_t d = lnf->shape[0];
  int n_layer = 0;
  while (ck.has("gpt.h." + std::to_string(n_layer) + ".ln_1.weight")) n_layer++;
  c.n_layer = n_layer;
  c.d_model = (int)d;
  c.n_head = (int)(d / 64);
  c.d_ffn = (int)fcb->shape[0];
  c.mel_vocab = (int)me->shape[0];
  c.text_vocab = (int)te->shape[0];
  c.lang_vocab = (int)le->shape[0];
  c.mel_pos_len = (int)mp->shape[0];
  c.text_pos_len = (int)tp->shape[0];
  if (d == 0 || d % 64 != 0) return weight_error("gpt.ln_f.weight", "d_model %zu is not a multiple of 64", d);
  // code width from the packed head: [V][K*bits/32] u32 words
  const size_t packed = hw->shape[1];
  if (packed * 4 == d)
    c.quant_bits = 8;
  else if (packed * 8 == d)
    c.quant_bits = 4;
  else
    return weight_error("mel_head.weight", "packed width %zu fits neither 8-bit nor 4-bit codes of K = %zu", packed, d);
  const TensorInfo *hs = ck.info("mel_head.scales");
  if (!hs) return weight_error("mel_head.scales", "missing required parameter tensor");
  c.param_dtype = hs->dtype == "F16" ? ITTS_F16 : ITTS_F32;
  const char *pdt = c.param_dtype == ITTS_F16 ? "F16," : "F32,";

  itts_weights w{};
  w.config = c;
  std::vector<itts_layer_weights> layers((size_t)n_layer);
  const size_t F = (size_t)c.d_ffn, pw = 32 / (size_t)c.quant_bits;
  auto f32 = [&](const std::string &name, std::vector<size_t> shape, const float **dst) {
    return ck.get(name, shape, "F32,", reinterpret_cast<const void **>(dst));
  };
  // QuantizedLinear::from_weights (gpt.rs:229-247): weight [out][in/pw] U32, scales and
  // biases [out][in/64], bias [out]
  auto ql = [&](const std::string &prefix, size_t in, size_t outf, itts_qlinear *q) -> itts_status {
    if (itts_status s = ck.get(prefix + ".weight", {outf, in / pw}, "U32,", &q->codes)) return s;
    if (itts_status s = ck.get(prefix + ".scales", {outf, in / 64}, pdt, &q->scales)) return s;
    if (itts_status s = ck.get(prefix + ".biases", {outf, in / 64}, pdt, &q->biases)) return s;
    return f32(prefix + ".bias", {outf}, &q->bias);
  };
  itts_status s;
  if ((s = f32("text_embedding.weight", {(size_t)c.text_vocab, d}, &w.text_embedding)) ||
      (s = f32("lang_embedding.weight", {(size_t)c.lang_vocab, d}, &w.lang_embedding)) ||
      (s = f32("mel_embedding.weight", {(size_t)c.mel_vocab, d}, &w.mel_embedding)) ||
      (s = f32("mel_pos_embedding.emb.weight", {(size_t)c.mel_pos_len, d}, &w.mel_pos_embedding)) ||
      (s = f32("text_pos_embedding.emb.weight", {(size_t)c.text_pos_len, d}, &w.text_pos_embedding)))
    return s;
  for (int i = 0; i < n_layer; i++) {
    const std::string p = "gpt.h." + std::to_string(i);
    itts_layer_weights &L = layers[(size_t)i];
    if ((s = f32(p + ".ln_1.weight", {d}, &L.ln1_w)) || (s = f32(p + ".ln_1.bias", {d}, &L.ln1_b)) ||
        (s = ql(p + ".attn.c_attn", d, 3 * d, &L.c_attn)) || (s = ql(p + ".attn.c_proj", d, d, &L.c_proj)) ||
        (s = f32(p + ".ln_2.weight", {d}, &L.ln2_w)) || (s = f32(p + ".ln_2.bias", {d}, &L.ln2_b)) ||
        (s = ql(p + ".mlp.c_fc", d, F, &L.c_fc)) || (s = ql(p + ".mlp.c_proj", F, d, &L.mlp_c_proj)))
      return s;
  }
  w.layers = layers.data();
  if ((s = f32("gpt.ln_f.weight", {d}, &w.ln_f_w)) || (s = f32("gpt.ln_f.bias", {d}, &w.ln_f_b)) ||
      (s = f32("final_norm.weight", {d}, &w.final_norm_w)) || (s = f32("final_norm.bias", {d}, &w.final_norm_b)) ||
      (s = ql("mel_head", d, (size_t)c.mel_vocab, &w.mel_head)))
    return s;
  return itts_gpt_create(&w, out);  // copies every tensor to the device; the mapping goes
}
