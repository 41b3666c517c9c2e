/*
 * Session-level C ABI for the gfx950 Llama prefill/decode path.
 *
 * No counterpart exists in the reference code: its generate API is design-only
 * (docs/products/aethermind_prd.md:298-320 sketches am_runtime_create /
 * am_model_load / am_session_generate; docs/designs/executor_design.md:226-256
 * describes PrepareSession / Prefill / DecodeStep).  These entry points implement that
 * design on one GPU: one HIP stream per runtime, weights repacked into HBM at model
 * creation, a device-resident static KV cache, and a frozen decode plan replayed as a
 * HIP graph with device-resident position/token state (no host sync per token).
 *
 * Two layers: the PRD's own Phase-1 interface (am_runtime_create(config),
 * am_model_load, am_session_create(config), am_session_generate with uint32 token ids,
 * am_error_t) at the end of this file, and the extended interface it is built on
 * (am_runtime_open, am_model_create_synthetic / am_model_load_hf, am_session_open,
 * prefill / decode / batched rows / profiling; int64 token ids, the graph input dtype of
 * model_graph_builder.cpp:339-342).
 */
#ifndef AM_RUNTIME_H
#define AM_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#include "am_c_api.h"
#include "am_gfx950.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct am_runtime am_runtime;
typedef struct am_model am_model;
typedef struct am_session am_session;

typedef struct am_model_config {
  int32_t num_layers, hidden, num_q_heads, num_kv_heads, head_dim, ffn, vocab;
  float rms_eps;
  double rope_theta;
  int32_t act_dtype;         /* AM_DT_F32 or AM_DT_BF16 */
  int32_t weight_format;     /* am_weight_format */
  int32_t group_size;        /* INT4 group (SPEC: 128) */
  int32_t max_tokens;        /* static KV capacity (positions) */
  int32_t max_prefill_chunk; /* rows per prefill pass; prompts are chunked to this */
} am_model_config;

/* Weight roles for am_model_weight (per-weight identity = (layer, role)). */
typedef enum am_weight_role {
  AM_ROLE_QKV = 0,     /* rows q (hq*d), k (hkv*d), v (hkv*d) */
  AM_ROLE_O = 1,
  AM_ROLE_GATE_UP = 2, /* rows gate (ffn) then up (ffn) */
  AM_ROLE_DOWN = 3,
  AM_ROLE_LM_HEAD = 4, /* layer ignored */
  AM_ROLE_Q = 5,       /* row views into QKV / GATE_UP */
  AM_ROLE_K = 6,
  AM_ROLE_V = 7,
  AM_ROLE_GATE = 8,
  AM_ROLE_UP = 9
} am_weight_role;

typedef enum am_model_buffer_kind {
  AM_BUF_EMBED = 0,     /* [vocab][hidden] act dtype */
  AM_BUF_IN_NORM = 1,   /* [hidden] act dtype, per layer */
  AM_BUF_POST_NORM = 2, /* per layer */
  AM_BUF_FINAL_NORM = 3,
  AM_BUF_ROPE_COS = 4, /* [max_tokens][d/2] f32 */
  AM_BUF_ROPE_SIN = 5
} am_model_buffer_kind;

am_status_code am_runtime_open(int32_t device, am_runtime** out);
void am_runtime_destroy(am_runtime* rt);
void* am_runtime_stream(am_runtime* rt); /* hipStream_t */
/* Blocks until all work enqueued on the runtime's stream has finished; reports an
 * asynchronous device error as AM_STATUS_INTERNAL. */
am_status_code am_runtime_synchronize(am_runtime* rt);

/* Prompt ids of the synthetic-data SPEC computed on the host (same integer stream
 * as am_gfx950_synth_token_ids): uniform in [0, vocab). */
am_status_code am_synth_token_ids_host(uint64_t seed, uint64_t stream, int64_t vocab, int64_t n, int64_t* out);

/* Synthetic Llama-dense weights of the build SPEC (seeded normal(0, 0.02), norm gains
 * 1.0) generated and repacked on the device. */
am_status_code am_model_create_synthetic(am_runtime* rt, const am_model_config* cfg, uint64_t seed,
                                         am_model** out);
void am_model_destroy(am_model* m);
/* Loads a Hugging Face Llama checkpoint directory (config.json plus model.safetensors
 * or model.safetensors.index.json with its shards; F32/F16/BF16 tensors) straight into
 * HBM, converted to the requested activation dtype and weight format (quantized on the
 * device).  The reference's HF reader / validator / weight resolver contract
 * (hf_directory_reader.cpp:333-412, hf_model_validator.cpp:168-644,
 * hf_weight_resolver.cpp:17-110): model_type llama, no bias, no RoPE scaling, every
 * layer tensor present with its exact shape, lm_head.weight absent only with
 * tie_word_embeddings (the embedding is then the head); the validation rules are those
 * of flags 0 in am_model_load_hf_ex (below). */
typedef struct am_model_load_options {
  int32_t act_dtype;         /* AM_DT_F32 or AM_DT_BF16 */
  int32_t weight_format;     /* am_weight_format */
  int32_t group_size;        /* INT4 group (SPEC: 128) */
  int32_t max_tokens;        /* static KV capacity (positions) */
  int32_t max_prefill_chunk; /* rows per prefill pass */
} am_model_load_options;
am_status_code am_model_load_hf(am_runtime* rt, const char* model_dir, const am_model_load_options* opt,
                                am_model** out);
/* Host only (no device work): reads and validates the checkpoint directory and fills
 * the shape fields of cfg (num_layers .. rope_theta), the tensor count and bytes. */
am_status_code am_hf_inspect(const char* model_dir, am_model_config* cfg, int64_t* n_tensors, int64_t* total_bytes);

/* Checkpoint validation rules: the reference's ModelValidationOptions
 * (model_validation_options.h:7-16).  0 = the reference's defaults, which
 * am_model_load_hf / am_hf_inspect use: tensors outside the model are ignored,
 * quantized tensors are refused (hf_model_validator.cpp:196-243, 364-385).  MoE, bias
 * and LoRA/adapter tensors and RoPE scaling are refused under every flag. */
typedef enum am_load_flags {
  AM_LOAD_STRICT_TENSOR_NAMES = 1,    /* strict_tensor_names: any tensor outside the model is an error */
  AM_LOAD_REJECT_UNKNOWN_TENSORS = 2, /* allow_unknown_tensors = false */
  AM_LOAD_ALLOW_QUANTIZED_TENSORS = 4 /* allow_quantized_tensors: a config.json quantization_config of
                                         4-bit GPTQ (checkpoint_format "gptq" or "gptq_v2") is accepted
                                         and each projection may be stored as its GPTQ set
                                         (qweight / qzeros / scales / optional g_idx) instead of .weight.
                                         INT4 targets with the same group size, F16 scales, in-order
                                         groups and all zeros 8 are repacked exactly; every other case is
                                         dequantized exactly (s * (q - z) in fp32) and converted to the
                                         requested format (see am_gfx950_gptq_unpack). */
} am_load_flags;
am_status_code am_model_load_hf_ex(am_runtime* rt, const char* model_dir, const am_model_load_options* opt,
                                   uint32_t flags, am_model** out);
am_status_code am_hf_inspect_ex(const char* model_dir, uint32_t flags, am_model_config* cfg, int64_t* n_tensors,
                                int64_t* total_bytes);
/* On-disk packed-weight cache: SavePackedCache / LoadPackedCache of the reference's
 * weight-packing design (model_weight_packing_strategy.md:390-394; design-only there).
 * The file is the model's repacked device weights exactly as they sit in HBM (embedding,
 * norms, q|k|v, o, gate|up, down, lm_head in the model's activation dtype and weight
 * format) behind a 256-byte header naming the shape, formats, device architecture and
 * layout version, with checksums of header and payload.  Loading reads it sequentially
 * through a pinned ring straight into HBM: no conversion, no quantization.
 *   save:    writes path + ".tmp" and renames it when complete.
 *   inspect: host only; checks the header and that the file holds the whole payload
 *            (NOT_FOUND, INVALID_ARGUMENT bad magic, FAILED_PRECONDITION other version /
 *            architecture / layout, DATA_LOSS checksum or size mismatch).
 *   load:    opt->act_dtype / weight_format (/ group_size for INT4) must equal the
 *            cache's (INVALID_ARGUMENT otherwise); max_tokens and max_prefill_chunk come
 *            from opt; a payload checksum mismatch is DATA_LOSS. */
am_status_code am_model_save_packed_cache(am_model* m, const char* path);
am_status_code am_packed_cache_inspect(const char* path, am_model_config* cfg, int64_t* payload_bytes);
am_status_code am_model_load_packed_cache(am_runtime* rt, const char* path, const am_model_load_options* opt,
                                          am_model** out);
am_status_code am_model_weight(am_model* m, int32_t layer, int32_t role, am_gfx950_weight* out);
am_status_code am_model_buffer(am_model* m, int32_t kind, int32_t layer, void** ptr, int64_t* bytes);
int64_t am_model_weight_bytes_total(am_model* m); /* repacked linear weights incl. scales */

typedef struct am_session_options {
  int32_t fused_decode; /* 1: fused decode plan (default), 0: one kernel per reference node */
  int32_t use_graph;    /* 1: replay decode steps as a HIP graph */
  int32_t batch;        /* sequences decoded together, 1..16 (0 means 1); > 1 needs the
                           fused plan, bf16 activations and bf16/int8/int4 weights */
  int32_t persistent_decode; /* 1: batch-1 fused decode as one persistent launch for
                                all layers (am_gfx950_decode_layers); session creation
                                fails when the model does not qualify.  0 or -1: the
                                per-op fused plan (default) */
  int32_t kv_block_size;     /* 0: each sequence owns a contiguous KV slot of max_tokens
                                positions (default).  > 0: paged KV (am_gfx950_kv_pages)
                                with blocks of this many positions (a power of two, at
                                least 32; bf16 activations, not with persistent_decode):
                                a sequence holds blocks only for the positions it has
                                reached, taken from one pool at prefill and as decode
                                grows it, and returned when the row is prefilled again or
                                the session ends */
  int32_t kv_pool_blocks;    /* paged KV: blocks in the pool (0: enough for every
                                sequence at max_tokens).  A prefill or decode that would
                                need more returns AM_STATUS_RESOURCE_EXHAUSTED before any
                                work is enqueued */
} am_session_options;

am_status_code am_session_open(am_model* m, const am_session_options* opt, am_session** out);
void am_session_destroy(am_session* s);
/* Prefill the prompt (host ids) from position 0; returns the first generated token.
 * In a batched session this prefills sequence 0. */
am_status_code am_session_prefill(am_session* s, const int64_t* prompt, int64_t n, int64_t* first_token);
/* Prefill sequence `row` (0 <= row < batch) of a batched session from position 0, in
 * its own KV reservation; the other sequences keep their caches and positions. */
am_status_code am_session_prefill_row(am_session* s, int64_t row, const int64_t* prompt, int64_t n,
                                      int64_t* first_token);
/* Number of sequences the session decodes together. */
int64_t am_session_batch(am_session* s);
/* Run n decode steps (enqueued, no host sync between steps); copies the n generated
 * tokens to tokens_out (host) at the end: [batch][n], sequence-major.  Every
 * sequence must have been prefilled. */
am_status_code am_session_decode(am_session* s, int64_t n, int64_t* tokens_out);
/* Enqueue n decode steps without reading anything back (benchmark timing). */
am_status_code am_session_decode_async(am_session* s, int64_t n);
/* Prefill + greedy decode up to max_new tokens (stops after eos if eos >= 0).
 * Single-sequence sessions only. */
am_status_code am_session_generate_ids(am_session* s, const int64_t* prompt, int64_t n_prompt, int64_t max_new,
                                   int64_t eos, int64_t* tokens_out, int64_t* n_out);
/* fp32 logits [batch][vocab] of the most recent step (host copy). */
am_status_code am_session_logits(am_session* s, float* out);
/* Current position (tokens committed to the KV cache) of sequence 0. */
int64_t am_session_position(am_session* s);
/* Current position of sequence `row` (-1 for a bad row). */
int64_t am_session_row_position(am_session* s, int64_t row);
/* Number of kernels launched per decode step by the active decode plan. */
int64_t am_session_decode_plan_size(am_session* s);
/* 1 when the session decodes with the persistent all-layers kernel, else 0. */
int32_t am_session_persistent_decode(am_session* s);

/* Per-op-type kernel time of eager decode steps, measured with HIP events on the
 * session stream around every step of the decode plan.  Runs n steps eagerly and
 * writes, for each executed step type, total milliseconds into ms_by_op[op_type]
 * (array of at least 64 doubles, indexed by OpType) and launch counts into
 * count_by_op. */
am_status_code am_session_profile_decode(am_session* s, int64_t n, double* ms_by_op, int64_t* count_by_op);

/* Process-wide counts of the device memory (hipMalloc / hipFree) and pinned host
 * memory (hipHostMalloc / hipHostFree) this library has taken and returned, and of the
 * HIP graphs it has instantiated (an instantiation takes device memory of its own).
 * A debug query with no counterpart in the reference: it shows that steady-state
 * decode allocates nothing, the PRD's "zero allocations in steady state"
 * (docs/products/aethermind_prd.md:152).  Memory torch or a caller allocates is not
 * counted. */
typedef struct am_alloc_stats {
  int64_t device_allocs, device_frees, device_bytes_live;
  int64_t pinned_allocs, pinned_frees, pinned_bytes_live;
  int64_t graph_instantiations;
} am_alloc_stats;
am_status_code am_debug_alloc_stats(am_alloc_stats* out);

/* ---------------- the PRD's Phase-1 C ABI (aethermind_prd.md:298-320) ----------------
 * Token ids are the only data boundary and are uint32 (prd.md:158-185).  Config structs
 * start with struct_size and only grow at the end (the PRD's ABI v1.x rules,
 * prd.md:322-327).  Errors: am_runtime_create / am_session_create return NULL (the text
 * is in am_last_error_message()); am_model_load and am_session_generate also fill
 * *error (when error != NULL) with an error object of this library, read with
 * am_gfx950_error_code / am_gfx950_error_message and released with am_error_free.  (The
 * PRD's am_error_message reads the reference library's own error objects, c_api.h:88.) */
typedef am_runtime* am_runtime_t;
typedef am_model* am_model_t;
typedef am_session* am_session_t;
typedef am_error_handle am_error_t;

typedef struct am_config {
  uint32_t struct_size;      /* sizeof(am_config_t) */
  int32_t device;            /* HIP device index */
  int32_t act_dtype;         /* activations of loaded models: AM_DT_BF16 or AM_DT_F32 */
  int32_t weight_format;     /* am_weight_format the loader converts / quantizes to */
  int32_t group_size;        /* INT4 group along k (128) */
  int32_t max_tokens;        /* static KV capacity per sequence (positions) */
  int32_t max_prefill_chunk; /* rows per prefill pass */
  /* grown at the end (a struct_size that stops before a field leaves its default) */
  uint32_t load_flags;       /* am_load_flags for am_model_load (default 0) */
} am_config_t;

typedef struct am_session_config {
  uint32_t struct_size;  /* sizeof(am_session_config_t) */
  uint32_t max_tokens;   /* GenerationConfig.max_tokens: tokens per generate call, 0 = no limit */
  int64_t eos_token_id;  /* GenerationConfig.eos_token_id, -1 = none */
  int32_t use_graph;     /* 1: decode steps replayed as a HIP graph (default) */
} am_session_config_t;

/* Runtime on config->device (NULL config: device 0, bf16 activations, INT4 g128
 * weights, 4096 positions, 512-row prefill chunks). */
am_runtime_t am_runtime_create(const am_config_t* config);
/* A Hugging Face checkpoint directory (see am_model_load_hf), converted to the
 * runtime's activation dtype and weight format. */
am_model_t am_model_load(am_runtime_t runtime, const char* path, am_error_t* error);
void am_model_unload(am_model_t model);
/* Single-sequence session with the fused decode plan (NULL config: graph on, no token
 * limit, no eos). */
am_session_t am_session_create(am_model_t model, const am_session_config_t* config);
/* Prefill input_tokens from position 0 and decode greedily: up to output_capacity
 * tokens, the session's max_tokens and the KV capacity left after the prompt,
 * stopping after eos_token_id.  Writes *output_len; returns an am_status_code. */
int am_session_generate(am_session_t session, const uint32_t* input_tokens, size_t input_len,
                        uint32_t* output_tokens, size_t output_capacity, size_t* output_len,
                        am_error_t* error);
void am_error_free(am_error_t error);

#ifdef __cplusplus
}
#endif
#endif
