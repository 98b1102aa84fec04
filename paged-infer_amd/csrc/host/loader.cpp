// Checkpoint loading: LlamaConfig::from_hf_config (src/model.rs:57-95) and
// ModelLoader::load_weights (src/model.rs:388-447) for bf16 HF Llama safetensors files.
//
// The file is memory-mapped. Its header (8-byte little-endian length, then a JSON object of
// name -> {dtype, shape, data_offsets}) is parsed here; each projection's bf16 bytes are copied
// to a device staging buffer and widened (f32) or quantized (int8, the device quantizer that
// matches quantize_rows_i8 bit for bit) straight into the model's padded, interleaved rows.
// Embeddings stay bf16 on the device; norm weights are widened on the host.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <utility>
#include <vector>

#include "common.h"
#include "host/context.h"

namespace pia {
namespace {

// ---------------------------------------------------------------------------------------
// Minimal JSON reader: objects, arrays, strings, numbers, true / false / null.
// ---------------------------------------------------------------------------------------
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0.0;
  bool uint_literal = false;  // digits only: what serde_json's as_u64 accepts
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json* get(const std::string& key) const {
    if (kind != Obj) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JsonParser {
 public:
  JsonParser(const char* p, const char* end, std::string what) : p_(p), end_(end), what_(std::move(what)) {}

  Json parse_document() {
    Json v = value(0);
    ws();
    if (p_ != end_) error("trailing characters");
    return v;
  }

 private:
  const char* p_;
  const char* end_;
  std::string what_;

  [[noreturn]] void error(const std::string& msg) { fail(PIA_ERR_INVALID, "parsing " + what_ + ": " + msg); }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool eat(char c) {
    ws();
    if (p_ < end_ && *p_ == c) {
      ++p_;
      return true;
    }
    return false;
  }
  void expect(char c) {
    if (!eat(c)) error(std::string("expected '") + c + "'");
  }
  bool literal(const char* s) {
    const size_t n = std::strlen(s);
    if (static_cast<size_t>(end_ - p_) >= n && std::memcmp(p_, s, n) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }
  static void utf8(std::string& out, unsigned cp) {
    if (cp < 0x80) {
      out += static_cast<char>(cp);
    } else if (cp < 0x800) {
      out += static_cast<char>(0xC0 | (cp >> 6));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += static_cast<char>(0xE0 | (cp >> 12));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      out += static_cast<char>(0xF0 | (cp >> 18));
      out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      out += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }
  unsigned hex4() {
    if (end_ - p_ < 4) error("short \\u escape");
    unsigned v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else error("bad \\u escape");
    }
    return v;
  }
  std::string string() {
    expect('"');
    std::string out;
    while (true) {
      if (p_ >= end_) error("unterminated string");
      const char c = *p_++;
      if (c == '"') break;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p_ >= end_) error("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          unsigned cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            p_ += 2;
            const unsigned lo = hex4();
            if (lo < 0xDC00 || lo >= 0xE000) error("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, cp);
          break;
        }
        default: error("bad escape");
      }
    }
    return out;
  }
  Json value(int depth) {
    if (depth > 64) error("nesting too deep");
    ws();
    if (p_ >= end_) error("unexpected end");
    Json v;
    const char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = Json::Obj;
      if (eat('}')) return v;
      do {
        ws();
        std::string k = string();
        expect(':');
        v.obj.emplace_back(std::move(k), value(depth + 1));
      } while (eat(','));
      expect('}');
    } else if (c == '[') {
      ++p_;
      v.kind = Json::Arr;
      if (eat(']')) return v;
      do v.arr.push_back(value(depth + 1));
      while (eat(','));
      expect(']');
    } else if (c == '"') {
      v.kind = Json::Str;
      v.str = string();
    } else if (literal("true")) {
      v.kind = Json::Bool, v.b = true;
    } else if (literal("false")) {
      v.kind = Json::Bool, v.b = false;
    } else if (literal("null")) {
      v.kind = Json::Null;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      const char* s = p_;
      while (p_ < end_ && (std::strchr("+-.eE", *p_) || (*p_ >= '0' && *p_ <= '9'))) ++p_;
      const std::string lit(s, p_);
      char* stop = nullptr;
      v.kind = Json::Num;
      v.num = std::strtod(lit.c_str(), &stop);
      if (stop != lit.c_str() + lit.size()) error("bad number '" + lit + "'");
      v.uint_literal = lit.find_first_not_of("0123456789") == std::string::npos;
    } else {
      error(std::string("unexpected character '") + c + "'");
    }
    return v;
  }
};

// ---------------------------------------------------------------------------------------
// safetensors container.
// ---------------------------------------------------------------------------------------
struct TensorView {
  std::string dtype;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  int64_t bytes = 0;
};

class MappedFile {
 public:
  explicit MappedFile(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) fail(PIA_ERR_INVALID, "cannot open " + path + ": " + std::strerror(errno));
    struct stat st {};
    if (::fstat(fd_, &st) != 0) fail(PIA_ERR_INVALID, "cannot stat " + path);
    size_ = static_cast<size_t>(st.st_size);
    if (size_ == 0) fail(PIA_ERR_INVALID, path + " is empty");
    void* p = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (p == MAP_FAILED) fail(PIA_ERR_INVALID, "cannot map " + path + ": " + std::strerror(errno));
    base_ = static_cast<const uint8_t*>(p);
  }
  ~MappedFile() {
    if (base_) ::munmap(const_cast<uint8_t*>(base_), size_);
    if (fd_ >= 0) ::close(fd_);
  }
  MappedFile(const MappedFile&) = delete;
  MappedFile& operator=(const MappedFile&) = delete;
  const uint8_t* data() const { return base_; }
  size_t size() const { return size_; }

 private:
  int fd_ = -1;
  const uint8_t* base_ = nullptr;
  size_t size_ = 0;
};

class SafeTensors {
 public:
  SafeTensors(const MappedFile& f, const std::string& path) {
    if (f.size() < 8) fail(PIA_ERR_INVALID, path + ": too short for a safetensors header");
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = (hlen << 8) | f.data()[i];
    if (hlen > f.size() - 8) fail(PIA_ERR_INVALID, path + ": header length exceeds the file");
    const char* h = reinterpret_cast<const char*>(f.data() + 8);
    const Json doc = JsonParser(h, h + hlen, path + " header").parse_document();
    if (doc.kind != Json::Obj) fail(PIA_ERR_INVALID, path + ": header is not a JSON object");
    const uint8_t* payload = f.data() + 8 + hlen;
    const uint64_t payload_bytes = f.size() - 8 - hlen;
    for (const auto& kv : doc.obj) {
      if (kv.first == "__metadata__") continue;
      const Json& t = kv.second;
      const Json* dt = t.get("dtype");
      const Json* sh = t.get("shape");
      const Json* off = t.get("data_offsets");
      if (!dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !off || off->kind != Json::Arr ||
          off->arr.size() != 2)
        fail(PIA_ERR_INVALID, path + ": malformed header entry for " + kv.first);
      TensorView v;
      v.dtype = dt->str;
      for (const Json& d : sh->arr) {
        if (d.kind != Json::Num || !d.uint_literal) fail(PIA_ERR_INVALID, path + ": bad shape for " + kv.first);
        v.shape.push_back(static_cast<int64_t>(d.num));
      }
      if (off->arr[0].kind != Json::Num || off->arr[1].kind != Json::Num || !off->arr[0].uint_literal ||
          !off->arr[1].uint_literal)
        fail(PIA_ERR_INVALID, path + ": bad data_offsets for " + kv.first);
      const uint64_t a = static_cast<uint64_t>(off->arr[0].num), b = static_cast<uint64_t>(off->arr[1].num);
      if (a > b || b > payload_bytes) fail(PIA_ERR_INVALID, path + ": data_offsets out of range for " + kv.first);
      v.data = payload + a;
      v.bytes = static_cast<int64_t>(b - a);
      tensors_.emplace_back(kv.first, std::move(v));
    }
  }

  const TensorView* find(const std::string& name) const {
    for (const auto& kv : tensors_)
      if (kv.first == name) return &kv.second;
    return nullptr;
  }

  // ModelLoader::tensor (src/model.rs:449-456) plus the checks the reference leaves to its
  // consumers: bf16 elements and the shape the config implies.
  const TensorView& bf16(const std::string& name, std::vector<int64_t> shape) const {
    const TensorView* v = find(name);
    if (!v) fail(PIA_ERR_INVALID, "missing tensor: " + name);
    if (v->dtype != "BF16") fail(PIA_ERR_INVALID, "tensor " + name + ": dtype " + v->dtype + ", expected BF16");
    if (v->shape != shape) {
      std::ostringstream os;
      os << "tensor " << name << ": shape [";
      for (size_t i = 0; i < v->shape.size(); ++i) os << (i ? ", " : "") << v->shape[i];
      os << "], the config implies [";
      for (size_t i = 0; i < shape.size(); ++i) os << (i ? ", " : "") << shape[i];
      os << "]";
      fail(PIA_ERR_INVALID, os.str());
    }
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    if (v->bytes != 2 * n) fail(PIA_ERR_INVALID, "tensor " + name + ": byte size does not match its shape");
    return *v;
  }

 private:
  std::vector<std::pair<std::string, TensorView>> tensors_;
};

void call(pia_status s) {
  if (s != PIA_OK) fail(s, pia_last_error());
}

std::vector<float> widen_host(const TensorView& v) {
  std::vector<float> out(static_cast<size_t>(v.bytes / 2));
  for (size_t i = 0; i < out.size(); ++i) {
    const uint32_t bits = static_cast<uint32_t>(v.data[2 * i]) | (static_cast<uint32_t>(v.data[2 * i + 1]) << 8);
    const uint32_t w = bits << 16;
    std::memcpy(&out[i], &w, 4);
  }
  return out;
}

}  // namespace
}  // namespace pia

using namespace pia;

extern "C" {

pia_status pia_hf_config_read(const char* path, pia_model_config* out) {
  PIA_API_BEGIN
  PIA_REQUIRE(path && out, "null argument");
  std::ifstream in(path, std::ios::binary);
  if (!in) fail(PIA_ERR_INVALID, std::string("reading ") + path + ": cannot open");
  std::stringstream ss;
  ss << in.rdbuf();
  const std::string text = ss.str();
  const Json doc = JsonParser(text.data(), text.data() + text.size(), path).parse_document();
  // LlamaConfig::default() (src/model.rs:37-53): TinyLlama-1.1B.
  pia_model_config c{2048, 22, 32, 4, 5632, 32000, 1e-5f, 10000.0f, -1};
  auto usize_at = [&](const char* key, int64_t fallback) -> int64_t {
    const Json* v = doc.get(key);
    if (!v || v->kind != Json::Num || !v->uint_literal) return fallback;
    return static_cast<int64_t>(v->num);
  };
  auto f32_at = [&](const char* key, float fallback) -> float {
    const Json* v = doc.get(key);
    if (!v || v->kind != Json::Num) return fallback;
    return static_cast<float>(v->num);
  };
  c.hidden = usize_at("hidden_size", c.hidden);
  c.layers = usize_at("num_hidden_layers", c.layers);
  c.heads = usize_at("num_attention_heads", c.heads);
  c.kv_heads = usize_at("num_key_value_heads", c.heads);  // multi-head checkpoints omit it
  c.inter = usize_at("intermediate_size", c.inter);
  c.vocab = usize_at("vocab_size", c.vocab);
  c.rms_eps = f32_at("rms_norm_eps", c.rms_eps);
  c.rope_theta = f32_at("rope_theta", c.rope_theta);
  *out = c;
  PIA_API_END
}

pia_status pia_model_load_safetensors(pia_model* m, const char* path, int32_t quantization, int32_t lm_head_int8) {
  PIA_API_BEGIN
  PIA_REQUIRE(m && path, "null argument");
  PIA_REQUIRE(quantization == 0 || quantization == 1, "quantization must be 0 (f32) or 1 (int8)");
  PIA_REQUIRE(lm_head_int8 == 0 || lm_head_int8 == 1, "lm_head_int8 must be 0 or 1");
  pia_model_config c{};
  call(pia_model_get_config(m, &c));
  const MappedFile file(path);
  const SafeTensors st(file, path);
  const int64_t hd = c.hidden / c.heads, kvd = c.kv_heads * hd;

  // Resolve every tensor first, so a missing or mis-shaped one leaves the model untouched.
  struct Item {
    const TensorView* v;
    int64_t layer;
    int32_t slot;
    int kind;
  };
  std::vector<Item> projs;
  const TensorView& embed = st.bf16("model.embed_tokens.weight", {c.vocab, c.hidden});
  const TensorView& final_norm = st.bf16("model.norm.weight", {c.hidden});
  const TensorView& lm_head =
      st.find("lm_head.weight") ? st.bf16("lm_head.weight", {c.vocab, c.hidden}) : embed;  // tied embeddings
  projs.push_back({&lm_head, -1, PIA_LM_HEAD, lm_head_int8});
  std::vector<std::pair<const TensorView*, const TensorView*>> norms;
  for (int64_t i = 0; i < c.layers; ++i) {
    const std::string p = "model.layers." + std::to_string(i);
    norms.emplace_back(&st.bf16(p + ".input_layernorm.weight", {c.hidden}),
                       &st.bf16(p + ".post_attention_layernorm.weight", {c.hidden}));
    const struct {
      const char* name;
      int32_t slot;
      int64_t rows, cols;
    } spec[] = {
        {".self_attn.q_proj.weight", PIA_WQ, c.hidden, c.hidden}, {".self_attn.k_proj.weight", PIA_WK, kvd, c.hidden},
        {".self_attn.v_proj.weight", PIA_WV, kvd, c.hidden},      {".self_attn.o_proj.weight", PIA_WO, c.hidden, c.hidden},
        {".mlp.gate_proj.weight", PIA_W1, c.inter, c.hidden},     {".mlp.down_proj.weight", PIA_W2, c.hidden, c.inter},
        {".mlp.up_proj.weight", PIA_W3, c.inter, c.hidden},
    };
    for (const auto& s : spec) projs.push_back({&st.bf16(p + s.name, {s.rows, s.cols}), i, s.slot, quantization});
  }

  call(pia_model_set_embedding(m, reinterpret_cast<const uint16_t*>(embed.data)));
  call(pia_model_set_norm(m, 0, PIA_NORM_FINAL, widen_host(final_norm).data()));
  for (int64_t i = 0; i < c.layers; ++i) {
    call(pia_model_set_norm(m, i, PIA_NORM_ATTN, widen_host(*norms[i].first).data()));
    call(pia_model_set_norm(m, i, PIA_NORM_FFN, widen_host(*norms[i].second).data()));
  }
  DeviceBuffer staging;
  for (const Item& it : projs) {
    staging.ensure(static_cast<size_t>(it.v->bytes));
    PIA_HIP(hipMemcpy(staging.ptr, it.v->data, static_cast<size_t>(it.v->bytes), hipMemcpyHostToDevice));
    model_set_proj_bf16_dev(m, it.layer, it.slot, it.kind, staging.as<uint16_t>(), it.v->shape[0], it.v->shape[1]);
  }
  PIA_API_END
}

}  // extern "C"
