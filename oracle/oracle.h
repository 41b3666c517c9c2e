/*
 * CPU ORACLE -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is a plain C++ restatement of the reference (fengjiran/AetherMind)
 * CPU semantics for the Llama prefill/decode path, plus the build's own SPEC for
 * the parts the reference never implemented (quant formats, RoPE, attention,
 * SiLU-Mul kernel, argmax tie-break, synthetic weights).  It exists to CHECK the
 * gfx950 library.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path never links or calls it.
 *
 * It shares no source with the product (aethermind_amd/csrc): every formula is
 * written out again here so a mistake in one side shows up as a parity failure.
 *
 * Parity status per function (what pins it besides the GPU comparison):
 *   orc_bf16_*           reference bfloat16.cpp:20-32; bit patterns from
 *                        tests/unit/numeric/test_bfloat16.cpp
 *   orc_f16_*            IEEE binary16 RNE; pinned by exhaustive round trip
 *   orc_synth_*          build SPEC; pinned by moment checks + closed forms of
 *                        the portable log/sin/cos/rsqrt against libm
 *   orc_embedding        reference embedding_entry.cpp:32-126 + KATs
 *                        (test_cpu_embedding_kernel.cpp:61-211)
 *   orc_rmsnorm_scalar   reference rmsnorm_fp32_scalar.cpp:10-63 + KATs
 *                        (test_cpu_rmsnorm_kernel.cpp:65-288)
 *   orc_rmsnorm_avx2     reference rmsnorm_fp32_avx2.cpp:15-122; pinned against
 *                        the scalar form at 1e-6 (test_cpu_rmsnorm_kernel.cpp:290-346)
 *   orc_dot_avx2         reference cpu_dot_product_avx2.cpp:8-40
 *   orc_linear           reference LinearOp design loop
 *                        (docs/designs/kernel_dev/LinearOp...v1.0.md:415-437),
 *                        double accumulation; pinned by brute-force fp64 sums
 *                        and identity / one-hot matrices
 *   orc_quant_int8/int4  build SPEC (reference has no format: prd.md:216);
 *                        pinned by closed forms and brute force over all codes
 *   orc_rope             reference RoPE design (RoPEOp...v1.0.md:588-622);
 *                        pinned by pos=0 identity, pair-norm preservation and
 *                        known angles
 *   orc_attention        textbook GQA SDPA (attention_op.cpp:11-169 contract);
 *                        pinned by one-position (out=V), uniform-score (mean V)
 *                        and GQA group equivalence
 *   orc_silu_mul         reference const_eval_silu_mul.cpp:18-31; pinned by
 *                        silu(0)=0 and asymptotes
 *   orc_argmax           build SPEC (lowest index wins, NaN ignored); brute force
 *   orc_model_*          node order of model_graph_builder.cpp:133-415
 */
#ifndef AM_ORACLE_H
#define AM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numerics ---- */
uint16_t orc_f32_to_bf16(float v);
float orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_f16(float v);
float orc_f16_to_f32(uint16_t h);
double orc_portable_log(double x);
void orc_portable_sincos_turns(double turns, double* s, double* c);
double orc_portable_sqrt(double x);

/* ---- synthetic data (build SPEC) ---- */
uint64_t orc_splitmix64(uint64_t x);
uint64_t orc_tensor_key(uint64_t seed, uint64_t tensor_id);
/* elements [offset, offset+n) of the N(0, std) stream of (seed, tensor_id) */
void orc_synth_normal_f32(uint64_t seed, uint64_t tensor_id, double stddev,
                          int64_t offset, int64_t n, float* out);
void orc_synth_normal_bf16(uint64_t seed, uint64_t tensor_id, double stddev,
                           int64_t offset, int64_t n, uint16_t* out);
void orc_synth_token_ids(uint64_t seed, uint64_t stream, int64_t vocab, int64_t n,
                         int64_t* out);

/* ---- quantization (build SPEC) ---- */
int orc_quant_int8(const float* w, int64_t n, int64_t k, int8_t* q, float* scales);
int orc_dequant_int8(const int8_t* q, const float* scales, int64_t n, int64_t k, float* w);
int orc_quant_int4(const float* w, int64_t n, int64_t k, int64_t group, uint8_t* packed,
                   uint16_t* scales_f16);
int orc_dequant_int4(const uint8_t* packed, const uint16_t* scales_f16, int64_t n, int64_t k,
                     int64_t group, float* w);

/* ---- ops (fp32 storage; act_bf16 != 0 rounds results through bf16) ---- */
int orc_embedding_i64(const int64_t* ids, int64_t n_tokens, const float* table, int64_t vocab,
                      int64_t hidden, float* out);
int orc_rmsnorm_scalar(const float* x, const float* w, int64_t rows, int64_t hidden, float eps,
                       float* out);
int orc_rmsnorm_avx2(const float* x, const float* w, int64_t rows, int64_t hidden, float eps,
                     float* out);
float orc_dot_avx2(const float* a, const float* b, int64_t n);
void orc_linear(const float* x, const float* w, int64_t m, int64_t n, int64_t k, float* out);
void orc_linear_avx2(const float* x, const float* w, int64_t m, int64_t n, int64_t k, float* out);
void orc_rope_table(int64_t max_pos, int64_t head_dim, double theta, float* cos_tab,
                    float* sin_tab);
void orc_rope(float* x, int64_t seq, int64_t heads, int64_t head_dim, const int64_t* pos,
              const float* cos_tab, const float* sin_tab);
void orc_attention(const float* q, const float* kc, const float* vc, int64_t seq,
                   int64_t hq, int64_t hkv, int64_t head_dim, int64_t cap, int64_t start_pos,
                   float* out);
void orc_silu_mul(const float* gate, const float* up, int64_t n, float* out);
int64_t orc_argmax(const float* x, int64_t n);
void orc_round_bf16_inplace(float* x, int64_t n);

/* ---- whole model (Llama dense) ---- */
typedef struct orc_model_config {
  int32_t num_layers, hidden, num_q_heads, num_kv_heads, head_dim, ffn, vocab;
  int32_t act_bf16;      /* 0: fp32 activations, 1: bf16 activations */
  int32_t weight_format; /* 0 fp32, 1 bf16, 2 int8 per-channel, 3 int4 g128 */
  int32_t group_size;
  int32_t max_tokens;
  float rms_eps;
  double rope_theta;
} orc_model_config;

typedef struct orc_model orc_model;
orc_model* orc_model_create_synthetic(const orc_model_config* cfg, uint64_t seed, int32_t threads);
void orc_model_destroy(orc_model* m);
/* prompt of n_prompt ids, then greedy decode; writes n_prompt-th.. tokens:
 * out_tokens[0] = argmax after prefill, then n_new-1 more decode steps. */
int orc_model_generate(orc_model* m, const int64_t* prompt, int64_t n_prompt, int64_t n_new,
                       int64_t* out_tokens, float* last_logits);
/* one forward over `n` tokens at positions [pos, pos+n): fills logits of the last token */
int orc_model_forward(orc_model* m, const int64_t* ids, int64_t n, int64_t pos, float* logits);
/* use the AVX2 fp32 kernels (the reference's fast path) instead of the fp64 scalar forms */
void orc_model_set_fast(orc_model* m, int32_t fast);
/* Plant one composition mistake (tests only: they show that the pins of the
 * composition reject it).  0 = none. */
enum {
  ORC_SLIP_NONE = 0,
  ORC_SLIP_RESIDUAL_NORMED = 1, /* attention residual added to the normed input, not h */
  ORC_SLIP_ROPE_AFTER_KV = 2,   /* keys written to the cache without RoPE */
  ORC_SLIP_GQA_MODULO = 3,      /* q head h reads kv head h % hkv instead of h / group */
  ORC_SLIP_NO_FINAL_NORM = 4,   /* final RMSNorm skipped before the head */
  ORC_SLIP_SWAP_NORM_GAINS = 5, /* each layer's input and post-attention gains swapped */
  ORC_SLIP_FINAL_GAIN_FROM_LAYER = 6, /* final norm applies the last layer's post-attention gain */
  ORC_SLIP_DROP_INPUT_GAIN = 7  /* input norms applied without their gain */
};
void orc_model_set_slip(orc_model* m, int32_t slip);
/* Replace a norm gain vector (hidden floats): kind 0 = input norm of `layer`, 1 =
 * post-attention norm of `layer`, 2 = final norm (layer ignored).  Synthetic models
 * start with every gain 1.0.  Returns 3 for a bad kind or layer. */
int orc_model_set_norm_gain(orc_model* m, int32_t kind, int32_t layer, const float* gain);
/* Per-shape decode GEMV of the CPU baseline: an n x k weight in format fmt (1 bf16,
 * 2 int8 per-channel, 3 int4 of `group`) filled with cheap deterministic bytes (timing
 * only: the values are not the synthetic-data SPEC's), and y = W x through the model's
 * Linear path (rows dequantized on the fly, AVX2 dot product), on the OpenMP threads
 * set by orc_set_threads.  orc_qweight_bytes: weight + scale bytes. */
typedef struct orc_qweight orc_qweight;
orc_qweight* orc_qweight_create(int64_t n, int64_t k, int32_t fmt, int64_t group, uint64_t seed);
void orc_qweight_destroy(orc_qweight* q);
int64_t orc_qweight_bytes(const orc_qweight* q);
void orc_qweight_gemv(const orc_qweight* q, const float* x, float* y);
/* OpenMP threads used by the oracle's parallel loops (cpu_baseline uses 1). */
void orc_set_threads(int32_t n);

#ifdef __cplusplus
}
#endif
#endif
