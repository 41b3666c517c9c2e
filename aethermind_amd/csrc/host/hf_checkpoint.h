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
enum class StDType { kF32, kF16, kBF16, kI32, kOther };
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

// The reference's ModelValidationOptions (model_validation_options.h:7-16) that this
// reader honours, with the reference's defaults.  Bias, LoRA/adapter and MoE tensors
// and RoPE scaling are always rejected (allow_bias / allow_lora_or_adapter /
// allow_rope_scaling have no kernels behind them here).
struct LoadRules {
  bool strict_tensor_names = false;     // any tensor outside the model is an error
  bool allow_unknown_tensors = true;    // otherwise unknown tensors are ignored
  bool allow_quantized_tensors = false; // GPTQ checkpoints (see GptqConfig)
};

// quantization_config of a GPTQ checkpoint (AutoGPTQ / optimum layout, 4 bits), read
// only under allow_quantized_tensors.  A quantized linear P is stored as
//   P.qweight  I32 [k/8][n]   nibble t of word (i, j) = q[8i + t][j]       (0..15)
//   P.qzeros   I32 [g][n/8]   nibble t of word (i, j) = stored zero of column 8j + t
//   P.scales   F16/BF16/F32 [g][n]
//   P.g_idx    I32 [k]        group of input feature k (optional: k / group_size)
// and means w[j][k] = scales[g_idx[k]][j] * (q[k][j] - z), z = (stored + zero_offset) & 15.
struct GptqConfig {
  bool present = false;
  int64_t group_size = 0;    // -1: one group over each linear's in_features
  bool desc_act = false;
  bool sym = true;
  int32_t zero_offset = 1;   // checkpoint_format "gptq" stores z - 1; "gptq_v2" stores z
};

struct LlamaConfig {
  int64_t num_layers = 0, hidden = 0, num_q_heads = 0, num_kv_heads = 0, head_dim = 0, ffn = 0, vocab = 0;
  int64_t max_position_embeddings = 0;
  double rms_eps = 0.0, rope_theta = 10000.0;
  bool tie_word_embeddings = false;
  GptqConfig gptq;
};
// config.json -> LlamaConfig with the reference's Phase-1 rules (model_type llama,
// positive integer dimensions below 2^31, rms_norm_eps and max_position_embeddings
// present, no bias, no RoPE scaling, head_dim = hidden / heads, heads divisible by kv
// heads, intermediate_size >= hidden_size, a dense float dtype hint).  A
// quantization_config is refused unless rules.allow_quantized_tensors, and then must
// describe 4-bit GPTQ.
StatusOr<LlamaConfig> ParseLlamaConfig(std::string_view config_json, const LoadRules& rules = {});

// The tensors of one GPTQ-quantized linear of shape [n][k] (views into the shards).
struct GptqLinear {
  const TensorView* qweight = nullptr;
  const TensorView* qzeros = nullptr;
  const TensorView* scales = nullptr;
  const TensorView* g_idx = nullptr;  // may be null
  int64_t n = 0, k = 0, group = 0, groups = 0;
};

class Checkpoint {
 public:
  // Reads model_dir/config.json and model.safetensors (or the shards named by
  // model.safetensors.index.json), then checks every tensor name, dtype (F32, F16,
  // BF16) and shape against the config; lm_head.weight may be absent only when
  // tie_word_embeddings is true; the embedding, head and dense projections share a
  // dtype.  MoE, bias and LoRA/adapter tensors and layer indices past num_layers are
  // errors; quantized tensors are errors unless rules.allow_quantized_tensors; other
  // unknown tensors follow strict_tensor_names / allow_unknown_tensors
  // (hf_model_validator.cpp:168-385).  Under allow_quantized_tensors a projection
  // without a dense .weight must have a complete GPTQ set.
  static StatusOr<std::unique_ptr<Checkpoint>> Open(const std::string& model_dir, const LoadRules& rules = {});

  const LlamaConfig& config() const { return cfg_; }
  // The GPTQ tensors of projection `prefix` (e.g. "model.layers.0.self_attn.q_proj"),
  // or null when it is stored dense (prefix + ".weight").
  const GptqLinear* Gptq(const std::string& prefix) const;
  bool has_gptq() const { return !gptq_.empty(); }
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
  std::map<std::string, GptqLinear> gptq_;
};

std::string LayerName(int64_t layer, std::string_view suffix);

}  // namespace aethermind::hf
