// Hugging Face Llama checkpoint reader: see hf_checkpoint.h.
#include "hf_checkpoint.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <set>
#include <sstream>

namespace aethermind::hf {

// ------------------------------------------------------------------ JSON
const Json* Json::Get(std::string_view key) const {
  if (kind != kObject) return nullptr;
  for (const auto& [k, v] : obj)
    if (k == key) return &v;
  return nullptr;
}

namespace {

class JsonParser {
 public:
  explicit JsonParser(std::string_view t) : t_(t) {}

  StatusOr<Json> Document() {
    Json v;
    AM_RETURN_IF_ERROR(Value(&v, 0));
    Ws();
    if (i_ != t_.size()) return Err("trailing content");
    return v;
  }

 private:
  static constexpr int kMaxDepth = 64;

  Status Err(const std::string& what) const {
    return Status::InvalidArgument("JSON: " + what + " at offset " + std::to_string(i_));
  }
  void Ws() {
    while (i_ < t_.size() && (t_[i_] == ' ' || t_[i_] == '\n' || t_[i_] == '\r' || t_[i_] == '\t')) ++i_;
  }
  bool Lit(std::string_view w) {
    if (t_.substr(i_, w.size()) != w) return false;
    i_ += w.size();
    return true;
  }

  Status Value(Json* out, int depth) {
    if (depth > kMaxDepth) return Err("nesting too deep");
    Ws();
    if (i_ >= t_.size()) return Err("unexpected end");
    const char c = t_[i_];
    if (c == '{') return Object(out, depth);
    if (c == '[') return Array(out, depth);
    if (c == '"') {
      out->kind = Json::kString;
      return String(&out->str);
    }
    if (Lit("true")) {
      out->kind = Json::kBool;
      out->boolean = true;
      return Status::Ok();
    }
    if (Lit("false")) {
      out->kind = Json::kBool;
      return Status::Ok();
    }
    if (Lit("null")) {
      out->kind = Json::kNull;
      return Status::Ok();
    }
    return Number(out);
  }

  Status Object(Json* out, int depth) {
    out->kind = Json::kObject;
    ++i_;
    Ws();
    if (i_ < t_.size() && t_[i_] == '}') {
      ++i_;
      return Status::Ok();
    }
    for (;;) {
      Ws();
      std::string key;
      if (i_ >= t_.size() || t_[i_] != '"') return Err("expected an object key");
      AM_RETURN_IF_ERROR(String(&key));
      Ws();
      if (i_ >= t_.size() || t_[i_] != ':') return Err("expected ':'");
      ++i_;
      Json v;
      AM_RETURN_IF_ERROR(Value(&v, depth + 1));
      out->obj.emplace_back(std::move(key), std::move(v));
      Ws();
      if (i_ < t_.size() && t_[i_] == ',') {
        ++i_;
        continue;
      }
      if (i_ < t_.size() && t_[i_] == '}') {
        ++i_;
        return Status::Ok();
      }
      return Err("expected ',' or '}'");
    }
  }

  Status Array(Json* out, int depth) {
    out->kind = Json::kArray;
    ++i_;
    Ws();
    if (i_ < t_.size() && t_[i_] == ']') {
      ++i_;
      return Status::Ok();
    }
    for (;;) {
      Json v;
      AM_RETURN_IF_ERROR(Value(&v, depth + 1));
      out->arr.push_back(std::move(v));
      Ws();
      if (i_ < t_.size() && t_[i_] == ',') {
        ++i_;
        continue;
      }
      if (i_ < t_.size() && t_[i_] == ']') {
        ++i_;
        return Status::Ok();
      }
      return Err("expected ',' or ']'");
    }
  }

  static void PutUtf8(std::string* s, uint32_t cp) {
    if (cp < 0x80) {
      s->push_back(static_cast<char>(cp));
    } else if (cp < 0x800) {
      s->push_back(static_cast<char>(0xC0 | (cp >> 6)));
      s->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      s->push_back(static_cast<char>(0xE0 | (cp >> 12)));
      s->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      s->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else {
      s->push_back(static_cast<char>(0xF0 | (cp >> 18)));
      s->push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
      s->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      s->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
  }

  Status Hex4(uint32_t* v) {
    if (i_ + 4 > t_.size()) return Err("short \\u escape");
    uint32_t x = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = t_[i_++];
      x <<= 4;
      if (h >= '0' && h <= '9') x |= static_cast<uint32_t>(h - '0');
      else if (h >= 'a' && h <= 'f') x |= static_cast<uint32_t>(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') x |= static_cast<uint32_t>(h - 'A' + 10);
      else return Err("bad \\u escape");
    }
    *v = x;
    return Status::Ok();
  }

  Status String(std::string* out) {
    ++i_;  // opening quote
    for (;;) {
      if (i_ >= t_.size()) return Err("unterminated string");
      const char c = t_[i_++];
      if (c == '"') return Status::Ok();
      if (static_cast<unsigned char>(c) < 0x20) return Err("control character in string");
      if (c != '\\') {
        out->push_back(c);
        continue;
      }
      if (i_ >= t_.size()) return Err("unterminated escape");
      const char e = t_[i_++];
      switch (e) {
        case '"': out->push_back('"'); break;
        case '\\': out->push_back('\\'); break;
        case '/': out->push_back('/'); break;
        case 'b': out->push_back('\b'); break;
        case 'f': out->push_back('\f'); break;
        case 'n': out->push_back('\n'); break;
        case 'r': out->push_back('\r'); break;
        case 't': out->push_back('\t'); break;
        case 'u': {
          uint32_t cp = 0;
          AM_RETURN_IF_ERROR(Hex4(&cp));
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            uint32_t lo = 0;
            if (!Lit("\\u")) return Err("lone high surrogate");
            AM_RETURN_IF_ERROR(Hex4(&lo));
            if (lo < 0xDC00 || lo >= 0xE000) return Err("bad low surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          PutUtf8(out, cp);
          break;
        }
        default: return Err("unknown escape");
      }
    }
  }

  Status Number(Json* out) {
    const size_t b = i_;
    if (i_ < t_.size() && t_[i_] == '-') ++i_;
    bool digits = false, integral = true;
    while (i_ < t_.size() && t_[i_] >= '0' && t_[i_] <= '9') {
      ++i_;
      digits = true;
    }
    if (i_ < t_.size() && t_[i_] == '.') {
      integral = false;
      ++i_;
      while (i_ < t_.size() && t_[i_] >= '0' && t_[i_] <= '9') ++i_;
    }
    if (i_ < t_.size() && (t_[i_] == 'e' || t_[i_] == 'E')) {
      integral = false;
      ++i_;
      if (i_ < t_.size() && (t_[i_] == '+' || t_[i_] == '-')) ++i_;
      while (i_ < t_.size() && t_[i_] >= '0' && t_[i_] <= '9') ++i_;
    }
    if (!digits) return Err("expected a value");
    const std::string tok(t_.substr(b, i_ - b));
    out->kind = Json::kNumber;
    out->number = std::strtod(tok.c_str(), nullptr);
    if (integral && tok[0] != '-') {
      errno = 0;
      const unsigned long long u = std::strtoull(tok.c_str(), nullptr, 10);
      if (errno == 0) {
        out->is_uint = true;
        out->uint = u;
      }
    }
    return Status::Ok();
  }

  std::string_view t_;
  size_t i_ = 0;
};

bool CheckedMul(uint64_t a, uint64_t b, uint64_t* out) {
  if (a != 0 && b > UINT64_MAX / a) return false;
  *out = a * b;
  return true;
}

StDType ParseDType(const std::string& s, uint64_t* elem_bytes) {
  static const std::pair<const char*, uint64_t> kBytes[] = {
      {"F64", 8}, {"F32", 4}, {"F16", 2}, {"BF16", 2}, {"I64", 8}, {"I32", 4}, {"I16", 2}, {"I8", 1},
      {"U64", 8}, {"U32", 4}, {"U16", 2}, {"U8", 1},   {"BOOL", 1}, {"F8_E4M3", 1}, {"F8_E5M2", 1}};
  *elem_bytes = 0;
  for (const auto& [n, b] : kBytes)
    if (s == n) *elem_bytes = b;
  if (s == "F32") return StDType::kF32;
  if (s == "F16") return StDType::kF16;
  if (s == "BF16") return StDType::kBF16;
  if (s == "I32") return StDType::kI32;
  return StDType::kOther;
}

StatusOr<std::string> ReadFile(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return Status::NotFound("cannot open " + path);
  std::ostringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

bool FileExists(const std::string& path) {
  struct stat st {};
  return ::stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

}  // namespace

StatusOr<Json> ParseJson(std::string_view text) { return JsonParser(text).Document(); }

// ------------------------------------------------------------------ safetensors
StatusOr<std::vector<TensorView>> ParseSafetensorsHeader(std::string_view header, const uint8_t* data_base,
                                                         uint64_t data_size) {
  auto doc = ParseJson(header);
  if (!doc.ok()) return doc.status();
  const Json& j = doc.value();
  if (j.kind != Json::kObject) return Status::InvalidArgument("safetensors header must be a JSON object");
  std::vector<TensorView> out;
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  std::set<std::string> names;
  for (const auto& [name, e] : j.obj) {
    if (name == "__metadata__") continue;
    if (!names.insert(name).second) return Status::InvalidArgument("duplicate safetensors tensor name '" + name + "'");
    if (e.kind != Json::kObject) return Status::InvalidArgument("safetensors tensor '" + name + "': entry is not an object");
    const Json* dt = e.Get("dtype");
    const Json* shape = e.Get("shape");
    const Json* offs = e.Get("data_offsets");
    if (dt == nullptr || dt->kind != Json::kString)
      return Status::InvalidArgument("safetensors tensor '" + name + "': missing 'dtype'");
    if (offs == nullptr || offs->kind != Json::kArray || offs->arr.size() != 2 || !offs->arr[0].is_uint ||
        !offs->arr[1].is_uint)
      return Status::InvalidArgument("safetensors tensor '" + name + "': missing or malformed 'data_offsets'");
    TensorView v;
    v.name = name;
    v.dtype_text = dt->str;
    uint64_t eb = 0;
    v.dtype = ParseDType(dt->str, &eb);
    if (eb == 0) return Status::InvalidArgument("safetensors tensor '" + name + "': unknown dtype '" + dt->str + "'");
    uint64_t numel = 1;
    if (shape != nullptr) {
      if (shape->kind != Json::kArray) return Status::InvalidArgument("safetensors tensor '" + name + "': bad 'shape'");
      for (const Json& d : shape->arr) {
        if (!d.is_uint || d.uint > static_cast<uint64_t>(INT64_MAX))
          return Status::InvalidArgument("safetensors tensor '" + name + "': negative or non-integer shape");
        if (!CheckedMul(numel, d.uint, &numel))
          return Status::OutOfRange("safetensors tensor '" + name + "': shape overflows");
        v.shape.push_back(static_cast<int64_t>(d.uint));
      }
    }
    const uint64_t b = offs->arr[0].uint, en = offs->arr[1].uint;
    if (b > en) return Status::InvalidArgument("safetensors tensor '" + name + "': data_offsets begin > end");
    if (en > data_size) return Status::OutOfRange("safetensors tensor '" + name + "': data outside the file");
    uint64_t nbytes = 0;
    if (!CheckedMul(numel, eb, &nbytes)) return Status::OutOfRange("safetensors tensor '" + name + "': size overflows");
    if (nbytes != en - b)
      return Status::InvalidArgument("safetensors tensor '" + name + "': shape and dtype do not match data_offsets");
    v.data = data_base + b;
    v.bytes = nbytes;
    ranges.emplace_back(b, en);
    out.push_back(std::move(v));
  }
  std::sort(ranges.begin(), ranges.end());
  uint64_t at = 0;
  for (const auto& [b, e] : ranges) {
    if (b != at) return Status::InvalidArgument("safetensors data_offsets overlap or leave gaps");
    at = e;
  }
  if (at != data_size) return Status::InvalidArgument("safetensors tensors do not cover the whole data region");
  return out;
}

StatusOr<std::unique_ptr<MappedFile>> MappedFile::Open(const std::string& path) {
  const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return Status::NotFound("cannot open " + path + ": " + std::strerror(errno));
  struct stat st {};
  if (::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
    ::close(fd);
    return Status::InvalidArgument(path + " is not a regular file");
  }
  std::unique_ptr<MappedFile> f(new MappedFile());
  f->size_ = static_cast<uint64_t>(st.st_size);
  if (f->size_ > 0) {
    void* p = ::mmap(nullptr, f->size_, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      ::close(fd);
      return Status::Internal("mmap failed for " + path);
    }
    (void)::madvise(p, f->size_, MADV_SEQUENTIAL);  // tensors are streamed in file order
    f->data_ = static_cast<const uint8_t*>(p);
  }
  ::close(fd);
  return f;
}

MappedFile::~MappedFile() {
  if (data_ != nullptr) (void)::munmap(const_cast<uint8_t*>(data_), size_);
}

// ------------------------------------------------------------------ config
namespace {
StatusOr<int64_t> PosInt(const Json& cfg, const char* key, bool required, int64_t dflt) {
  const Json* v = cfg.Get(key);
  if (v == nullptr || v->kind == Json::kNull) {
    if (required) return Status::InvalidArgument(std::string("config.json: missing '") + key + "'");
    return dflt;
  }
  // the runtime keeps every dimension in int32, so 2^31 - 1 is the largest accepted
  if (!v->is_uint || v->uint == 0 || v->uint > static_cast<uint64_t>(INT32_MAX))
    return Status::InvalidArgument(std::string("config.json: '") + key + "' must be a positive integer below 2^31");
  return static_cast<int64_t>(v->uint);
}
}  // namespace

namespace {
// quantization_config -> GptqConfig (4-bit GPTQ only)
Status ParseGptq(const Json& q, GptqConfig* g) {
  if (q.kind != Json::kObject) return Status::InvalidArgument("config.json: quantization_config must be an object");
  const Json* m = q.Get("quant_method");
  if (m == nullptr || m->kind != Json::kString || m->str != "gptq")
    return Status::Unimplemented("config.json: only quant_method \"gptq\" checkpoints can be ingested");
  const Json* bits = q.Get("bits");
  if (bits == nullptr || !bits->is_uint || bits->uint != 4)
    return Status::Unimplemented("config.json: only 4-bit GPTQ checkpoints can be ingested");
  const Json* gs = q.Get("group_size");
  if (gs == nullptr || gs->kind != Json::kNumber) return Status::InvalidArgument("config.json: GPTQ group_size missing");
  if (gs->number == -1.0) {
    g->group_size = -1;
  } else if (gs->is_uint && gs->uint > 0 && gs->uint % 8 == 0 && gs->uint <= static_cast<uint64_t>(INT32_MAX)) {
    g->group_size = static_cast<int64_t>(gs->uint);
  } else {
    return Status::InvalidArgument("config.json: GPTQ group_size must be -1 or a positive multiple of 8");
  }
  for (const char* k : {"desc_act", "sym"}) {
    const Json* b = q.Get(k);
    if (b == nullptr || b->kind == Json::kNull) continue;
    if (b->kind != Json::kBool) return Status::InvalidArgument(std::string("config.json: GPTQ ") + k + " must be a bool");
    (std::string(k) == "desc_act" ? g->desc_act : g->sym) = b->boolean;
  }
  g->zero_offset = 1;
  if (const Json* f = q.Get("checkpoint_format"); f != nullptr && f->kind != Json::kNull) {
    if (f->kind != Json::kString || (f->str != "gptq" && f->str != "gptq_v2"))
      return Status::Unimplemented("config.json: GPTQ checkpoint_format must be \"gptq\" or \"gptq_v2\"");
    g->zero_offset = f->str == "gptq" ? 1 : 0;
  }
  g->present = true;
  return Status::Ok();
}
}  // namespace

StatusOr<LlamaConfig> ParseLlamaConfig(std::string_view text, const LoadRules& rules) {
  auto doc = ParseJson(text);
  if (!doc.ok()) return doc.status();
  const Json& c = doc.value();
  if (c.kind != Json::kObject) return Status::InvalidArgument("config.json must be a JSON object");
  const Json* mt = c.Get("model_type");
  if (mt == nullptr || mt->kind != Json::kString) return Status::InvalidArgument("config.json: 'model_type' must be provided");
  if (mt->str != "llama") return Status::InvalidArgument("config.json: only model_type=llama is supported");
  LlamaConfig m;
  auto get = [&](const char* k, bool req, int64_t d, int64_t* out) -> Status {
    auto v = PosInt(c, k, req, d);
    if (!v.ok()) return v.status();
    *out = v.value();
    return Status::Ok();
  };
  AM_RETURN_IF_ERROR(get("hidden_size", true, 0, &m.hidden));
  AM_RETURN_IF_ERROR(get("intermediate_size", true, 0, &m.ffn));
  AM_RETURN_IF_ERROR(get("num_hidden_layers", true, 0, &m.num_layers));
  AM_RETURN_IF_ERROR(get("num_attention_heads", true, 0, &m.num_q_heads));
  AM_RETURN_IF_ERROR(get("num_key_value_heads", false, m.num_q_heads, &m.num_kv_heads));
  AM_RETURN_IF_ERROR(get("vocab_size", true, 0, &m.vocab));
  if (m.hidden % m.num_q_heads != 0)
    return Status::InvalidArgument("config.json: hidden_size must be divisible by num_attention_heads");
  AM_RETURN_IF_ERROR(get("head_dim", false, m.hidden / m.num_q_heads, &m.head_dim));
  if (m.head_dim != m.hidden / m.num_q_heads)
    return Status::InvalidArgument("config.json: head_dim must equal hidden_size / num_attention_heads");
  if (m.num_kv_heads > m.num_q_heads || m.num_q_heads % m.num_kv_heads != 0)
    return Status::InvalidArgument("config.json: num_attention_heads must be a multiple of num_key_value_heads");
  // rms_norm_eps has no default: the reference reads 0 when it is absent and rejects
  // anything that is not positive (hf_model_validator.cpp:523-525)
  const Json* eps = c.Get("rms_norm_eps");
  if (eps == nullptr || eps->kind != Json::kNumber || !(eps->number > 0.0))
    return Status::InvalidArgument("config.json: rms_norm_eps must be a positive number");
  m.rms_eps = eps->number;
  AM_RETURN_IF_ERROR(get("max_position_embeddings", true, 0, &m.max_position_embeddings));
  if (m.ffn < m.hidden)
    return Status::InvalidArgument("config.json: intermediate_size must be at least hidden_size");
  // RoPE: a top-level rope_theta and a rope_scaling / rope_parameters object (the form
  // recent transformers versions write: {"rope_theta": .., "rope_type": "default"}) are
  // read in file order, so a later key overrides an earlier theta, as in the reference
  // reader (hf_directory_reader.cpp:141-155, 170-219).  A scaling factor or a scaling
  // type other than "" / "default" is RoPE scaling, which Phase 1 rejects
  // (hf_model_validator.cpp:561-564; hf_model_config.h:28-41).
  for (const auto& [key, val] : c.obj) {
    if (key == "rope_theta") {
      if (val.kind != Json::kNumber || !(val.number > 0.0)) return Status::InvalidArgument("config.json: rope_theta must be positive");
      m.rope_theta = val.number;
    } else if (key == "rope_scaling" || key == "rope_parameters") {
      if (val.kind == Json::kNull) continue;
      if (val.kind != Json::kObject) return Status::InvalidArgument("config.json: " + key + " must be an object or null");
      for (const auto& [rk, rv] : val.obj) {
        if (rk == "factor") {
          if (rv.kind != Json::kNumber) return Status::InvalidArgument("config.json: " + key + ".factor must be a number");
          return Status::InvalidArgument("config.json: RoPE scaling is not supported");
        }
        if (rk == "type" || rk == "rope_type") {
          if (rv.kind != Json::kString) return Status::InvalidArgument("config.json: " + key + "." + rk + " must be a string");
          if (!rv.str.empty() && rv.str != "default") return Status::InvalidArgument("config.json: RoPE scaling is not supported");
        } else if (rk == "rope_theta") {
          if (rv.kind != Json::kNumber || !(rv.number > 0.0))
            return Status::InvalidArgument("config.json: " + key + ".rope_theta must be positive");
          m.rope_theta = rv.number;
        }
      }
    }
  }
  if (const Json* t = c.Get("tie_word_embeddings"); t != nullptr && t->kind == Json::kBool) m.tie_word_embeddings = t->boolean;
  for (const char* k : {"attention_bias", "mlp_bias"})
    if (const Json* b = c.Get(k); b != nullptr && b->kind == Json::kBool && b->boolean)
      return Status::InvalidArgument(std::string("config.json: ") + k + " is not supported");
  // the weight dtype hint: absent, "auto" or a dense float type the loader converts
  // (hf_directory_reader.cpp:221-240; hf_model_validator.cpp:30-38, 587-589)
  for (const char* k : {"torch_dtype", "dtype"}) {
    const Json* h = c.Get(k);
    if (h == nullptr || h->kind == Json::kNull) continue;
    if (h->kind != Json::kString) return Status::InvalidArgument(std::string("config.json: ") + k + " must be a string");
    static constexpr std::string_view kDense[] = {"auto", "float32", "float", "float16", "half", "bfloat16"};
    bool ok = false;
    for (std::string_view d : kDense) ok = ok || h->str == d;
    if (!ok) return Status::InvalidArgument("config.json: only dense float torch_dtype hints are supported (got '" + h->str + "')");
  }
  if (const Json* a = c.Get("hidden_act"); a != nullptr && a->kind == Json::kString && a->str != "silu")
    return Status::InvalidArgument("config.json: hidden_act must be silu");
  if (const Json* q = c.Get("quantization_config"); q != nullptr && q->kind != Json::kNull) {
    if (!rules.allow_quantized_tensors)
      return Status::InvalidArgument(
          "config.json: quantization_config describes a quantized checkpoint; loading it needs allow_quantized_tensors");
    AM_RETURN_IF_ERROR(ParseGptq(*q, &m.gptq));
  }
  return m;
}

std::string LayerName(int64_t layer, std::string_view suffix) {
  return "model.layers." + std::to_string(layer) + std::string(suffix);
}

// ------------------------------------------------------------------ checkpoint
namespace {
Status AddFile(const std::string& path, std::vector<std::unique_ptr<MappedFile>>* files,
               std::map<std::string, TensorView>* tensors, const std::map<std::string, std::string>* owner,
               const std::string& shard_name) {
  auto mf = MappedFile::Open(path);
  if (!mf.ok()) return mf.status();
  const MappedFile& f = *mf.value();
  if (f.size() < 8) return Status::InvalidArgument(path + ": too small for a safetensors header");
  uint64_t hl = 0;
  for (int i = 0; i < 8; ++i) hl |= static_cast<uint64_t>(f.data()[i]) << (8 * i);
  if (hl > f.size() - 8) return Status::InvalidArgument(path + ": header length exceeds the file");
  const std::string_view header(reinterpret_cast<const char*>(f.data() + 8), static_cast<size_t>(hl));
  auto views = ParseSafetensorsHeader(header, f.data() + 8 + hl, f.size() - 8 - hl);
  if (!views.ok()) return Status::InvalidArgument(path + ": " + views.status().message());
  for (auto& v : views.value()) {
    if (owner != nullptr) {
      const auto it = owner->find(v.name);
      if (it == owner->end())
        return Status::InvalidArgument(path + ": tensor '" + v.name + "' is not listed in the index");
      if (it->second != shard_name)
        return Status::FailedPrecondition("the index assigns '" + v.name + "' to " + it->second + ", found in " + shard_name);
    }
    const std::string name = v.name;
    if (!tensors->emplace(name, std::move(v)).second)
      return Status::AlreadyExists("tensor '" + name + "' appears in more than one shard");
  }
  files->push_back(std::move(mf.value()));
  return Status::Ok();
}

Status ExpectTensor(const std::map<std::string, TensorView>& t, const std::string& name, std::vector<int64_t> shape) {
  const auto it = t.find(name);
  if (it == t.end()) return Status::InvalidArgument("checkpoint is missing required weight '" + name + "'");
  const TensorView& v = it->second;
  if (v.dtype != StDType::kF32 && v.dtype != StDType::kF16 && v.dtype != StDType::kBF16)
    return Status::InvalidArgument("tensor " + name + ": dtype " + v.dtype_text + " (expected F32, F16 or BF16)");
  if (v.shape != shape) {
    std::string want, got;
    for (int64_t d : shape) want += std::to_string(d) + ",";
    for (int64_t d : v.shape) got += std::to_string(d) + ",";
    return Status::InvalidArgument("tensor " + name + ": shape [" + got + "] (expected [" + want + "])");
  }
  return Status::Ok();
}
}  // namespace

namespace {
bool EndsWithComponent(const std::string& name, std::string_view comp) {
  if (name.size() < comp.size() || name.compare(name.size() - comp.size(), comp.size(), comp) != 0) return false;
  return name.size() == comp.size() || name[name.size() - comp.size() - 1] == '.';
}

// layer index of "model.layers.<i>.<rest>" (-1 for other names, -2 when malformed)
int64_t LayerIndexOf(const std::string& name) {
  static constexpr std::string_view kPre = "model.layers.";
  if (name.compare(0, kPre.size(), kPre) != 0) return -1;
  int64_t v = 0;
  size_t i = kPre.size();
  if (i >= name.size() || name[i] < '0' || name[i] > '9') return -2;
  for (; i < name.size() && name[i] >= '0' && name[i] <= '9'; ++i) {
    v = v * 10 + (name[i] - '0');
    if (v > INT32_MAX) return -2;
  }
  return i < name.size() && name[i] == '.' ? v : -2;
}

// Tensors no Llama-dense kernel can run, whatever the rules (hf_model_validator.cpp:168-243):
// mixture-of-experts, bias and LoRA/adapter weights; quantized components unless allowed.
Status CheckSupported(const std::string& name, const LoadRules& rules) {
  for (std::string_view p : {"experts", "router", "moe"})
    if (name.find(p) != std::string::npos) return Status::InvalidArgument("tensor " + name + ": MoE weights are not supported");
  for (std::string_view p : {".q_proj.bias", ".k_proj.bias", ".v_proj.bias", ".o_proj.bias", ".gate_proj.bias",
                             ".up_proj.bias", ".down_proj.bias", "lm_head.bias"})
    if (name.find(p) != std::string::npos) return Status::InvalidArgument("tensor " + name + ": bias weights are not supported");
  for (std::string_view p : {"lora_A", "lora_B", "adapter", "peft"})
    if (name.find(p) != std::string::npos)
      return Status::InvalidArgument("tensor " + name + ": LoRA/adapter weights are not supported");
  if (!rules.allow_quantized_tensors)
    for (std::string_view p : {"qweight", "qzeros", "scales", "g_idx", "bits", "group_size"})
      if (EndsWithComponent(name, p))
        return Status::InvalidArgument("tensor " + name + ": quantized tensors need allow_quantized_tensors");
  return Status::Ok();
}

std::string ShapeText(const std::vector<int64_t>& s) {
  std::string t = "[";
  for (size_t i = 0; i < s.size(); ++i) t += (i ? "," : "") + std::to_string(s[i]);
  return t + "]";
}

// The GPTQ set of projection prefix [n][k] (all of qweight / qzeros / scales present).
Status CheckGptq(const std::map<std::string, TensorView>& t, const std::string& prefix, int64_t n, int64_t k,
                 const GptqConfig& g, GptqLinear* out) {
  auto find = [&](const char* sfx) -> const TensorView* {
    const auto it = t.find(prefix + sfx);
    return it == t.end() ? nullptr : &it->second;
  };
  out->qweight = find(".qweight");
  out->qzeros = find(".qzeros");
  out->scales = find(".scales");
  out->g_idx = find(".g_idx");
  if (!out->qweight || !out->qzeros || !out->scales)
    return Status::InvalidArgument("checkpoint is missing required weight '" + prefix + ".weight' (or its GPTQ "
                                   "qweight / qzeros / scales)");
  const int64_t group = g.group_size == -1 ? k : g.group_size;
  if (k % 8 != 0 || n % 8 != 0 || k % group != 0)
    return Status::InvalidArgument(prefix + ": GPTQ needs in/out features divisible by 8 and in_features by group_size");
  out->n = n;
  out->k = k;
  out->group = group;
  out->groups = k / group;
  auto expect = [&](const TensorView* v, std::vector<int64_t> shape, bool int32) -> Status {
    if (int32 ? v->dtype != StDType::kI32 : (v->dtype == StDType::kI32 || v->dtype == StDType::kOther))
      return Status::InvalidArgument("tensor " + v->name + ": dtype " + v->dtype_text +
                                     (int32 ? " (expected I32)" : " (expected F16, BF16 or F32)"));
    if (v->shape != shape)
      return Status::InvalidArgument("tensor " + v->name + ": shape " + ShapeText(v->shape) + " (expected " +
                                     ShapeText(shape) + ")");
    return Status::Ok();
  };
  AM_RETURN_IF_ERROR(expect(out->qweight, {k / 8, n}, true));
  AM_RETURN_IF_ERROR(expect(out->qzeros, {out->groups, n / 8}, true));
  AM_RETURN_IF_ERROR(expect(out->scales, {out->groups, n}, false));
  if (out->g_idx) {
    AM_RETURN_IF_ERROR(expect(out->g_idx, {k}, true));
    const int32_t* gi = reinterpret_cast<const int32_t*>(out->g_idx->data);
    for (int64_t i = 0; i < k; ++i)
      if (gi[i] < 0 || gi[i] >= out->groups)
        return Status::InvalidArgument("tensor " + out->g_idx->name + ": group index out of range at " + std::to_string(i));
  }
  return Status::Ok();
}
}  // namespace

StatusOr<std::unique_ptr<Checkpoint>> Checkpoint::Open(const std::string& dir, const LoadRules& rules) {
  std::unique_ptr<Checkpoint> ck(new Checkpoint());
  auto cfg_text = ReadFile(dir + "/config.json");
  if (!cfg_text.ok()) return cfg_text.status();
  auto cfg = ParseLlamaConfig(cfg_text.value(), rules);
  if (!cfg.ok()) return cfg.status();
  ck->cfg_ = cfg.value();
  const std::string single = dir + "/model.safetensors", index = dir + "/model.safetensors.index.json";
  if (FileExists(index)) {
    auto idx_text = ReadFile(index);
    if (!idx_text.ok()) return idx_text.status();
    auto idx = ParseJson(idx_text.value());
    if (!idx.ok()) return Status::InvalidArgument("model.safetensors.index.json: " + idx.status().message());
    const Json* wm = idx.value().Get("weight_map");
    if (wm == nullptr || wm->kind != Json::kObject)
      return Status::InvalidArgument("model.safetensors.index.json: missing 'weight_map'");
    std::map<std::string, std::string> owner;
    std::set<std::string> shards;
    for (const auto& [name, file] : wm->obj) {
      if (file.kind != Json::kString) return Status::InvalidArgument("weight_map: shard name must be a string");
      // a shard is a plain file name inside the model directory
      if (file.str.empty() || file.str.find('/') != std::string::npos || file.str == "." || file.str == "..")
        return Status::InvalidArgument("weight_map: shard '" + file.str + "' escapes the model directory");
      owner[name] = file.str;
      shards.insert(file.str);
    }
    for (const auto& s : shards) AM_RETURN_IF_ERROR(AddFile(dir + "/" + s, &ck->files_, &ck->tensors_, &owner, s));
    for (const auto& [name, s] : owner)
      if (ck->tensors_.find(name) == ck->tensors_.end())
        return Status::NotFound("tensor '" + name + "' listed in the index is missing from " + s);
  } else if (FileExists(single)) {
    AM_RETURN_IF_ERROR(AddFile(single, &ck->files_, &ck->tensors_, nullptr, ""));
  } else {
    return Status::NotFound(dir + ": neither model.safetensors nor model.safetensors.index.json");
  }

  // names, dtypes and shapes against the config (hf_weight_resolver.cpp:17-110,
  // hf_model_validator.cpp:168-644)
  const LlamaConfig& c = ck->cfg_;
  for (const auto& [name, v] : ck->tensors_) {
    AM_RETURN_IF_ERROR(CheckSupported(name, rules));
    const int64_t li = LayerIndexOf(name);
    if (li == -2) return Status::InvalidArgument("tensor " + name + ": malformed layer index");
    if (li >= c.num_layers)
      return Status::InvalidArgument("tensor " + name + " has layer index " + std::to_string(li) +
                                     " but num_hidden_layers is " + std::to_string(c.num_layers));
  }
  const int64_t H = c.hidden, Q = c.num_q_heads * c.head_dim, KV = c.num_kv_heads * c.head_dim;
  std::set<std::string> known;
  // rotary inv_freq buffers some exporters save: ignored under every rule
  // (hf_model_validator.cpp:340-355)
  std::set<std::string> ignorable = {"model.rotary_emb.inv_freq"};
  auto need = [&](const std::string& n, std::vector<int64_t> shape) -> Status {
    known.insert(n);
    return ExpectTensor(ck->tensors_, n, std::move(shape));
  };
  // a projection [n][k]: dense .weight, or (quantized checkpoints) its GPTQ set
  auto proj = [&](const std::string& prefix, int64_t n, int64_t k) -> Status {
    if (ck->tensors_.count(prefix + ".weight") || !c.gptq.present) return need(prefix + ".weight", {n, k});
    GptqLinear g;
    AM_RETURN_IF_ERROR(CheckGptq(ck->tensors_, prefix, n, k, c.gptq, &g));
    for (const TensorView* v : {g.qweight, g.qzeros, g.scales, g.g_idx})
      if (v) known.insert(v->name);
    ck->gptq_[prefix] = g;
    return Status::Ok();
  };
  AM_RETURN_IF_ERROR(need("model.embed_tokens.weight", {c.vocab, H}));
  AM_RETURN_IF_ERROR(need("model.norm.weight", {H}));
  if (ck->tensors_.count("lm_head.weight")) {
    AM_RETURN_IF_ERROR(need("lm_head.weight", {c.vocab, H}));
  } else if (!c.tie_word_embeddings) {
    return Status::InvalidArgument("required weight 'lm_head.weight' is missing and tie_word_embeddings is false");
  }
  for (int64_t l = 0; l < c.num_layers; ++l) {
    ignorable.insert(LayerName(l, ".self_attn.rotary_emb.inv_freq"));
    AM_RETURN_IF_ERROR(need(LayerName(l, ".input_layernorm.weight"), {H}));
    AM_RETURN_IF_ERROR(need(LayerName(l, ".post_attention_layernorm.weight"), {H}));
    AM_RETURN_IF_ERROR(proj(LayerName(l, ".self_attn.q_proj"), Q, H));
    AM_RETURN_IF_ERROR(proj(LayerName(l, ".self_attn.k_proj"), KV, H));
    AM_RETURN_IF_ERROR(proj(LayerName(l, ".self_attn.v_proj"), KV, H));
    AM_RETURN_IF_ERROR(proj(LayerName(l, ".self_attn.o_proj"), H, Q));
    AM_RETURN_IF_ERROR(proj(LayerName(l, ".mlp.gate_proj"), c.ffn, H));
    AM_RETURN_IF_ERROR(proj(LayerName(l, ".mlp.up_proj"), c.ffn, H));
    AM_RETURN_IF_ERROR(proj(LayerName(l, ".mlp.down_proj"), H, c.ffn));
  }
  // tensors outside the model: ignored by default, errors under strict names or
  // without allow_unknown_tensors (hf_model_validator.cpp:364-385); they are dropped
  for (auto it = ck->tensors_.begin(); it != ck->tensors_.end();) {
    if (known.count(it->first)) {
      ++it;
      continue;
    }
    if (!ignorable.count(it->first) && (rules.strict_tensor_names || !rules.allow_unknown_tensors))
      return Status::InvalidArgument("unexpected tensor found: " + it->first);
    it = ck->tensors_.erase(it);
  }
  // The embedding, the head and every dense projection share one dtype (the
  // reference's default require_uniform_linear_dtype, hf_model_validator.cpp:433-500);
  // a present head of a tied model has the embedding's dtype.  Norm gains may differ.
  const TensorView& embed = ck->Get("model.embed_tokens.weight");
  if (const TensorView* head = ck->Find("lm_head.weight"); head != nullptr && c.tie_word_embeddings &&
                                                             head->dtype != embed.dtype)
    return Status::InvalidArgument("tied embedding dtype mismatch: lm_head.weight is " + head->dtype_text +
                                   ", model.embed_tokens.weight is " + embed.dtype_text);
  auto same_as_embed = [&](const std::string& n) -> Status {
    const TensorView* v = ck->Find(n);
    if (v == nullptr) return Status::Ok();  // a GPTQ projection
    if (v->dtype != embed.dtype)
      return Status::InvalidArgument("mixed linear tensor dtype: " + n + " is " + v->dtype_text + ", expected " +
                                     embed.dtype_text);
    return Status::Ok();
  };
  AM_RETURN_IF_ERROR(same_as_embed("lm_head.weight"));
  for (int64_t l = 0; l < c.num_layers; ++l)
    for (const char* sfx : {".self_attn.q_proj.weight", ".self_attn.k_proj.weight", ".self_attn.v_proj.weight",
                            ".self_attn.o_proj.weight", ".mlp.gate_proj.weight", ".mlp.up_proj.weight",
                            ".mlp.down_proj.weight"})
      AM_RETURN_IF_ERROR(same_as_embed(LayerName(l, sfx)));
  return ck;
}

const GptqLinear* Checkpoint::Gptq(const std::string& prefix) const {
  const auto it = gptq_.find(prefix);
  return it == gptq_.end() ? nullptr : &it->second;
}

const TensorView* Checkpoint::Find(const std::string& name) const {
  const auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

const TensorView& Checkpoint::LmHead() const {
  const TensorView* h = Find("lm_head.weight");
  return h != nullptr ? *h : Get("model.embed_tokens.weight");
}

uint64_t Checkpoint::max_tensor_bytes() const {
  uint64_t b = 0;
  for (const auto& [n, v] : tensors_) b = std::max(b, v.bytes);
  return b;
}

uint64_t Checkpoint::total_bytes() const {
  uint64_t b = 0;
  for (const auto& [n, v] : tensors_) b += v.bytes;
  return b;
}

}  // namespace aethermind::hf
