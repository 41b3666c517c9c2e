// Hugging Face Llama checkpoint reader (config.json + safetensors, single file or
// sharded with model.safetensors.index.json), the counterpart of the reference's
// HfDirectoryReader / HfSafetensorsFile / HfModelValidator / ResolveWeights
// (src/model/formats/hf/hf_directory_reader.cpp:333-412, hf_safetensors_file.cpp:64-382,
// hf_model_validator.cpp:168-644, hf_weight_resolver.cpp:17-110).
//
// Files are memory-mapped read-only; a tensor is a view (pointer, bytes, dtype, shape)
// into its shard.  Nothing here touches a device: the runtime streams the views to HBM.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

#include "am_core.h"

namespace aethermind::hf {

// ---- minimal JSON (config.json, the shard index, safetensors headers) ----
struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject };
  Kind kind = kNull;
  bool boolean = false;
  double number = 0.0;
  bool is_uint = false;  // the number was a non-negative integer literal
  uint64_t uint = 0;     // its exact value
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;  // keys in file order

  const Json* Get(std::string_view key) const;
};
StatusOr<Json> ParseJson(std::string_view text);

// ---- safetensors ----
enum class StDType { kF32, kF16, kBF16, kOther };
struct TensorView {
  std::string name;
  StDType dtype = StDType::kOther;
  std::string dtype_text;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;
  uint64_t bytes = 0;
};

// Parses and validates a safetensors header against a data region of data_size bytes
// at data_base: dtype / shape / data_offsets per tensor, offsets contiguous from 0 and
// covering the region, byte sizes matching shape x dtype, no duplicate names.
StatusOr<std::vector<TensorView>> ParseSafetensorsHeader(std::string_view header, const uint8_t* data_base,
                                                         uint64_t data_size);

class MappedFile {
 public:
  static StatusOr<std::unique_ptr<MappedFile>> Open(const std::string& path);
  ~MappedFile();
  const uint8_t* data() const { return data_; }
  uint64_t size() const { return size_; }

 private:
  MappedFile() = default;
  const uint8_t* data_ = nullptr;
  uint64_t size_ = 0;
};

// ---- model ----
struct LlamaConfig {
  int64_t num_layers = 0, hidden = 0, num_q_heads = 0, num_kv_heads = 0, head_dim = 0, ffn = 0, vocab = 0;
  int64_t max_position_embeddings = 0;
  double rms_eps = 0.0, rope_theta = 10000.0;
  bool tie_word_embeddings = false;
};
// config.json -> LlamaConfig with the reference's Phase-1 rules (model_type llama,
// positive integer dimensions below 2^31, rms_norm_eps and max_position_embeddings
// present, no bias, no RoPE scaling, head_dim = hidden / heads, heads divisible by kv
// heads, intermediate_size >= hidden_size, a dense float dtype hint).
StatusOr<LlamaConfig> ParseLlamaConfig(std::string_view config_json);

class Checkpoint {
 public:
  // Reads model_dir/config.json and model.safetensors (or the shards named by
  // model.safetensors.index.json), then checks every tensor name, dtype (F32, F16,
  // BF16) and shape against the config; lm_head.weight may be absent only when
  // tie_word_embeddings is true; the embedding, head and projections share a dtype.
  static StatusOr<std::unique_ptr<Checkpoint>> Open(const std::string& model_dir);

  const LlamaConfig& config() const { return cfg_; }
  const TensorView* Find(const std::string& name) const;
  const TensorView& Get(const std::string& name) const { return *Find(name); }
  // lm_head.weight, or the embedding when the head is tied
  const TensorView& LmHead() const;
  size_t num_tensors() const { return tensors_.size(); }
  uint64_t total_bytes() const;
  uint64_t max_tensor_bytes() const;  // the largest single tensor (device staging size)

 private:
  LlamaConfig cfg_{};
  std::vector<std::unique_ptr<MappedFile>> files_;
  std::map<std::string, TensorView> tensors_;
};

std::string LayerName(int64_t layer, std::string_view suffix);

}  // namespace aethermind::hf
