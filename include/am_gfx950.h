/*
 * gfx950 (MI355X) kernel C ABI for the AetherMind Llama prefill/decode path.
 *
 * Every entry point has the shape
 *     am_status_code am_gfx950_<op>(const am_gfx950_<op>_args* args, void* hip_stream);
 * All pointers inside the args are DEVICE pointers unless a field says otherwise.
 * Work is enqueued on `hip_stream` (NULL = the default stream) and the call returns
 * without synchronising, except where a field asks for a checked (synchronous) mode.
 * Argument validation happens on the host before any launch; a rejected call enqueues
 * nothing.  These functions replace the reference's CPU KernelFunc bodies: the C++
 * backend in aethermind_amd/csrc/host registers one KernelFunc per op through the
 * reference's KernelRegistry shape (kernel_descriptor.h:12-21) that unpacks its
 * params and calls the matching function here.
 *
 * Data layouts (row-major unless stated):
 *   activations  [rows][cols], dtype AM_DT_F32 or AM_DT_BF16
 *   KV cache     one plane per layer and K/V: [kv_heads][capacity][head_dim]
 *                (the reference KVCacheLayout, kv_cache_view.cpp:41-75)
 *   weights      see am_gfx950_weight
 */
#ifndef AM_GFX950_H
#define AM_GFX950_H

#include <stdint.h>

#include "am_c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum am_dtype {
  AM_DT_F32 = 0,
  AM_DT_BF16 = 1,
  AM_DT_F16 = 2,
  AM_DT_I8 = 3,
  AM_DT_I4 = 4,
  AM_DT_I32 = 5,
  AM_DT_I64 = 6,
  AM_DT_U32 = 7,
  AM_DT_U8 = 8
} am_dtype;

/* Device weight formats (WeightFormat of kernel_selector.h:26-31 of the reference,
 * with the two quantized formats given a concrete layout). */
typedef enum am_weight_format {
  AM_WF_F32 = 0,  /* fp32 [n][k]                                                  */
  AM_WF_BF16 = 1, /* bf16 [n][k]                                                  */
  AM_WF_INT8 = 2, /* uint8 [n][k] holding q+128, fp32 scale per row [n]           */
  AM_WF_INT4 = 3  /* uint8 [n][k/2] nibbles holding q+8 (device tile order below), */
                  /* fp16 scales [n][k/group]                                     */
} am_weight_format;

/* INT4 device tile order: each 32-bit word of a row holds k = 8w..8w+7 with
 * nibble j (bits 4j..4j+3) = k 8w + {0,2,4,6,1,3,5,7}[j], so that
 * (word >> 4t) & 0x000F000F yields the pair (k 8w+2t, k 8w+2t+1).  The logical
 * interchange format (low nibble = even k, two's complement) converts to it with
 * am_gfx950_pack_int4 and back with am_gfx950_dequant. */
typedef struct am_gfx950_weight {
  const void* data;
  const void* scales; /* NULL for F32/BF16 */
  int64_t n;          /* out_features */
  int64_t k;          /* in_features  */
  int32_t format;     /* am_weight_format */
  int32_t group_size; /* INT4 only (SPEC: 128) */
} am_gfx950_weight;

/* ---------------- per-op kernels (one reference OpType each) ---------------- */

/* OpType::kEmbedding (embedding_entry.cpp:32-126): out[t,:] = table[ids[t],:].
 * ids dtype I32/I64/U32.  An id outside [0, vocab) writes a zero row and sets
 * *err_flag (if non-NULL) to 1; with check != 0 the call synchronises the stream
 * and returns AM_STATUS_OUT_OF_RANGE in that case, like the reference kernel. */
typedef struct am_gfx950_embedding_args {
  const void* ids;
  int32_t ids_dtype;
  int64_t n_tokens;
  const void* table;
  int32_t table_dtype; /* F32 / BF16 */
  int64_t vocab, hidden;
  void* out;
  int32_t out_dtype;
  int32_t* err_flag;
  int32_t check;
} am_gfx950_embedding_args;
am_status_code am_gfx950_embedding(const am_gfx950_embedding_args* args, void* hip_stream);

/* OpType::kRmsNorm (rmsnorm_fp32_avx2.cpp:15-122): y = x * rsqrt(mean(x^2)+eps) * w,
 * fp32 accumulation, one rounding to out_dtype. */
typedef struct am_gfx950_rmsnorm_args {
  const void* x;
  const void* w;
  void* out;
  int64_t rows, hidden;
  int64_t x_stride, out_stride; /* elements between rows */
  float eps;
  int32_t x_dtype, w_dtype, out_dtype;
} am_gfx950_rmsnorm_args;
am_status_code am_gfx950_rmsnorm(const am_gfx950_rmsnorm_args* args, void* hip_stream);

/* OpType::kLinear (linear_op.h:87-92): out[m,:] = x[m,:] @ W^T (+ residual[m,:]).
 * fp32 accumulation; out rounded once to out_dtype, and with a residual the sum is
 * rounded again (two op boundaries: Linear then Add).  residual may alias out.
 * mode: 0 auto (bf16 activations with 2 <= m <= 16 -> batched decode GEMV when the
 * weight format allows it; otherwise m <= 8 -> GEMV, else MFMA GEMM), 1 GEMV per row,
 * 2 GEMM, 3 batched decode GEMV (m <= 16, bf16 activations, bf16/int8 weights or
 * int4 with group 128; when m rows of k values do not fit one block's LDS the rows
 * run in groups that do, each group reading the weights again). */
typedef struct am_gfx950_linear_args {
  const void* x;
  int32_t x_dtype;
  int64_t m;
  am_gfx950_weight w;
  void* out;
  int32_t out_dtype;
  const void* residual; /* optional, out_dtype */
  int32_t mode;
  void* workspace;      /* optional (NULL): am_gfx950_gemm_workspace_bytes(m, n, k, group) bytes,
                           16-byte aligned, zero before the first call (left zero); lets the
                           MFMA GEMM split K when its tiles alone leave CUs idle */
  int64_t workspace_bytes;
} am_gfx950_linear_args;
am_status_code am_gfx950_linear(const am_gfx950_linear_args* args, void* hip_stream);

/* Prefill fusions of Linear with the next reference node, on the MFMA GEMM (m rows of
 * bf16 activations; INT4 weights with group a multiple of 64, INT8 per-channel or bf16
 * weights with k a multiple of 128; fp32 weights return AM_STATUS_UNIMPLEMENTED and
 * take am_gfx950_linear per node):
 *   AM_PREFILL_SPLIT     one weight whose row ranges are several Linears (q|k|v):
 *                        columns [0, split[0]) -> out[0] [m][split[0]], [split[0],
 *                        split[1]) -> out[1], [split[1], n) -> out[2]; each rounded
 *                        to bf16 as its own Linear's output
 *   AM_PREFILL_SILU_MUL  Linear gate|up (rows [0, n/2) gate, [n/2, n) up) -> SiluMul:
 *                        out[0] [m][n/2] = round(silu(round(gate)) * round(up))
 *   AM_PREFILL_QKV_ROPE_KV  Linear q|k|v -> RoPE -> KVCacheUpdate for one sequence
 *                        (rope_op.cpp:11-223, kvcache_update_op.cpp:50-138): row i is
 *                        position *rope_kv->start_pos_dev + i; out[0] [m][hq*d] gets
 *                        the rotated q; k (rotated) and v go straight into the cache
 *                        planes (pages: the sequence's block-table row).  Rows whose
 *                        position is outside [0, capacity) write no cache row, keep
 *                        q unrotated and set *err_flag (when not NULL).
 * (model_graph_builder.cpp:133-290 node order; SiluMul formula const_eval_silu_mul.cpp:18-31) */
typedef enum am_gfx950_prefill_epilogue {
  AM_PREFILL_SPLIT = 0,
  AM_PREFILL_SILU_MUL = 1,
  AM_PREFILL_QKV_ROPE_KV = 2
} am_gfx950_prefill_epilogue;
typedef struct am_gfx950_prefill_rope_kv {
  const float* cos_tab;          /* [max_pos][head_dim/2], am_gfx950_rope_table */
  const float* sin_tab;
  int64_t max_pos;               /* at least capacity */
  const int64_t* start_pos_dev;  /* device: position of row 0 */
  void* k_cache;                 /* the layer's planes [hkv][capacity][d] (or block pools) */
  void* v_cache;
  int64_t hq, hkv, head_dim, capacity;
  const struct am_gfx950_kv_pages* pages; /* NULL: contiguous planes (struct defined below) */
  int32_t* err_flag;             /* optional */
} am_gfx950_prefill_rope_kv;
typedef struct am_gfx950_prefill_linear_args {
  const void* x;
  int64_t m;
  am_gfx950_weight w;
  int32_t epilogue;
  void* out[3];
  int64_t split[2];
  void* workspace;      /* optional, as in am_gfx950_linear_args */
  int64_t workspace_bytes;
  const am_gfx950_prefill_rope_kv* rope_kv; /* AM_PREFILL_QKV_ROPE_KV only */
} am_gfx950_prefill_linear_args;
am_status_code am_gfx950_prefill_linear(const am_gfx950_prefill_linear_args* args, void* hip_stream);

/* Workspace bytes with which the prefill GEMM of an m x n x k product may split K
 * (group_size: the INT4 group; 128 for INT8 and bf16 weights, whose splits are whole
 * 128-value ranges of k): split s of an output tile sums a contiguous range of whole
 * groups, and the tile's last split block adds the fp32 partials in
 * split order (results are independent of block scheduling).  0: the shape never
 * splits (its tiles already fill the device).  The first 4096 bytes are the tickets
 * (one u32 per tile of the launch), which must be zero before the first call and are
 * left zero; the region has the same size for every shape, so one workspace sized for
 * the largest shape serves launches of different shapes in turn. */
int64_t am_gfx950_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int64_t group_size);

/* OpType::kRoPE (rope_op.cpp:202-223; RoPEOp design :588-622): split-half rotation of
 * q [seq][hq*d] and k [seq][hkv*d] at positions pos[seq] (I64, device) using the
 * fp32 tables cos_tab/sin_tab [max_pos][d/2] built by am_gfx950_rope_table.
 * Outputs may alias inputs. */
typedef struct am_gfx950_rope_args {
  const void* q;
  const void* k;
  void* q_out;
  void* k_out;
  const int64_t* pos;
  const float* cos_tab;
  const float* sin_tab;
  int64_t seq, hq, hkv, head_dim, max_pos;
  int32_t dtype;
} am_gfx950_rope_args;
am_status_code am_gfx950_rope(const am_gfx950_rope_args* args, void* hip_stream);

/* Host-side helper: fills the host arrays cos_tab/sin_tab [max_pos][d/2] with
 * inv_freq = 1/theta^(2i/d), angle = pos*inv_freq (double), cast to float. */
am_status_code am_gfx950_rope_table(int64_t max_pos, int64_t head_dim, double theta,
                                    float* cos_tab_host, float* sin_tab_host);

/* Paged (block) KV cache.  The PRD's Phase-2 direction (aethermind_prd.md:437-444;
 * kv_cache_design.md 6.7 and 10: "replace the storage and offset resolution under a
 * stable logical view").  With pages, k_cache / v_cache of a layer are pools of
 * num_blocks blocks, each [hkv][block_size][head_dim] elements, and position pos of
 * sequence b lives in block block_table[b * table_stride + pos / block_size] at row
 * pos % block_size.  capacity stays the logical position limit per sequence (at most
 * table_stride * block_size); cache_batch_stride is unused.  Block ids outside
 * [0, num_blocks) are clamped into it on the device (the runtime never writes one).
 * Without pages (pages == NULL) a sequence's cache is contiguous: head g's rows start
 * g * capacity * head_dim elements into its planes. */
typedef struct am_gfx950_kv_pages {
  const int32_t* block_table; /* device [batch][table_stride] */
  int32_t block_size;         /* positions per block: a power of two, at least 32 */
  int32_t table_stride;       /* table entries per sequence */
  int64_t num_blocks;         /* blocks in each pool */
  /* grown at the end (zero-initialise the struct): optional device flag the KV writers
   * (kv_update, the fused q/k/v decode epilogues, the prefill q|k|v RoPE+KV epilogue)
   * set to 1 when the table entry of a position they write lies outside
   * [0, num_blocks), e.g. an unassigned block (-1); that row is then not written.
   * Readers clamp such an entry into the pool.  kv_update and the prefill epilogue
   * also report into their own err_flag when this one is NULL. */
  int32_t* err_flag;
} am_gfx950_kv_pages;

/* OpType::kKVCacheUpdate (kvcache_update_op.cpp:50-138): writes k/v [seq][hkv*d]
 * into the layer planes at positions [start, start+seq), start = *start_pos_dev if
 * start_pos_dev != NULL else start_pos.  Rows past capacity are rejected on the host
 * when start is a host value, and skipped (err_flag set) when it is a device value.
 * pages != NULL: the sequence's table row is pages->block_table (bf16 or f32). */
typedef struct am_gfx950_kv_update_args {
  const void* k;
  const void* v;
  void* k_cache;
  void* v_cache;
  int64_t seq, hkv, head_dim, capacity;
  int64_t start_pos;
  const int64_t* start_pos_dev;
  int32_t dtype;
  int32_t* err_flag;
  const am_gfx950_kv_pages* pages; /* NULL: contiguous planes */
} am_gfx950_kv_update_args;
am_status_code am_gfx950_kv_update(const am_gfx950_kv_update_args* args, void* hip_stream);

/* OpType::kAttention (attention_op.cpp:11-169): causal GQA SDPA.  Query row s sits at
 * position start+s and attends to cache positions [0, start+s]; q head h reads kv
 * head h/(hq/hkv); scale 1/sqrt(d); fp32 online softmax.  The cache rows for the new
 * positions must already be written (KVCacheUpdate precedes Attention).
 * workspace: device scratch of am_gfx950_attention_workspace_bytes(...) bytes (0 when
 * no split is possible), whose first 4*hkv*batch*seq bytes (split tickets) must be
 * zero before the first call; the kernel leaves them zero.  Decode rows are split
 * over positions when the context is long; the last block of each (row, kv head)
 * merges the partial records, so one launch produces the output.
 * batch > 1 stacks independent sequences: q [batch][seq][hq*d], caches
 * [batch] planes of cache_batch_stride elements, start positions start_pos_dev[b].
 * pages != NULL (bf16 only): paged caches, sequence b's table row b. */
typedef struct am_gfx950_attention_args {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  void* out;
  int64_t seq, hq, hkv, head_dim, capacity;
  int64_t start_pos;
  const int64_t* start_pos_dev;
  int64_t batch;
  int64_t cache_batch_stride;
  int32_t dtype;
  int32_t num_splits; /* 0 = choose */
  void* workspace;
  int64_t workspace_bytes;
  const am_gfx950_kv_pages* pages; /* NULL: contiguous planes */
} am_gfx950_attention_args;
am_status_code am_gfx950_attention(const am_gfx950_attention_args* args, void* hip_stream);
int64_t am_gfx950_attention_workspace_bytes(int64_t batch, int64_t seq, int64_t hq, int64_t hkv,
                                            int64_t head_dim, int64_t capacity, int32_t num_splits);

/* am_gfx950_attention without a caller workspace and without any allocation: the
 * split tickets and records live in a file-scope device array of
 * am_gfx950_attention_noalloc_max_bytes() bytes (8 MiB) that each device holds until
 * the process ends.  No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid hipMalloc).
 * args->workspace must be NULL and args->workspace_bytes 0; a shape whose
 * am_gfx950_attention_workspace_bytes exceeds the maximum is rejected with
 * AM_STATUS_RESOURCE_EXHAUSTED.  Each call clears its tickets with a kernel on
 * hip_stream (no memset), then launches the same kernels as am_gfx950_attention.
 * Every call on one device shares that device's array: calls that overlap on one
 * device (different streams, concurrently) race and must not be issued. */
am_status_code am_gfx950_attention_noalloc(const am_gfx950_attention_args* args, void* hip_stream);
int64_t am_gfx950_attention_noalloc_max_bytes(void);

/* OpType::kSiluMul (silu_mul_op.cpp:32-61; formula const_eval_silu_mul.cpp:18-31). */
typedef struct am_gfx950_silu_mul_args {
  const void* gate;
  const void* up;
  void* out;
  int64_t n;
  int32_t dtype;
} am_gfx950_silu_mul_args;
am_status_code am_gfx950_silu_mul(const am_gfx950_silu_mul_args* args, void* hip_stream);

/* OpType::kAdd (add_entry.cpp): out = a + b, same shape (no broadcast on this path). */
typedef struct am_gfx950_add_args {
  const void* a;
  const void* b;
  void* out;
  int64_t n;
  int32_t dtype;
} am_gfx950_add_args;
am_status_code am_gfx950_add(const am_gfx950_add_args* args, void* hip_stream);

/* OpType::kArgmax (argmax_op.cpp:6-45), axis -1: out[r] = first index of the maximum
 * of x[r,:] (NaN never selected; an all-NaN row gives 0).  x dtype F32/BF16, out I64.
 * workspace: am_gfx950_argmax_workspace_bytes(rows) bytes, first 4*rows bytes zero
 * before the first call (left zero). */
typedef struct am_gfx950_argmax_args {
  const void* x;
  int32_t dtype;
  int64_t rows, n;
  int64_t* out;
  void* workspace;
  int64_t workspace_bytes;
} am_gfx950_argmax_args;
am_status_code am_gfx950_argmax(const am_gfx950_argmax_args* args, void* hip_stream);
int64_t am_gfx950_argmax_workspace_bytes(int64_t rows);

/* ---------------- weight loader / repack (WeightPrepackPlanner + prepacker) -------- */

/* Quantize a device fp32/bf16/fp16 matrix src [n][k] into a device weight of `format`
 * (INT8 per-channel or INT4 group) following the build SPEC:
 *   INT8: s = max|w|/127 (1 for an all-zero row), q = clamp(rint(w/s), -127, 127)
 *   INT4: s = fp16(max|w|/7) per group, q = clamp(rint(w/s), -8, 7), q = 0 if s == 0
 * dst->data / dst->scales must point at buffers of am_gfx950_weight_bytes(...). */
typedef struct am_gfx950_quantize_args {
  const void* src;
  int32_t src_dtype;
  int64_t src_rows;     /* rows of src, each dst.k long */
  am_gfx950_weight dst; /* data/scales written through (cast away const) */
  int64_t dst_row_offset; /* src row r goes to dst row offset + r * stride */
  int64_t dst_row_stride; /* 1 = contiguous rows; 2 = interleave (gate/up pairs) */
} am_gfx950_quantize_args;
am_status_code am_gfx950_quantize(const am_gfx950_quantize_args* args, void* hip_stream);

/* Copies a device fp32/bf16/fp16 matrix into an F32/BF16 device weight (one RNE
 * rounding when narrowing), same row mapping as am_gfx950_quantize
 * (dst_row_offset / dst_row_stride). */
am_status_code am_gfx950_pack_plain(const am_gfx950_quantize_args* args, void* hip_stream);

/* Converts the logical INT4 interchange format (uint8 [n][k/2], low nibble = even k,
 * two's complement; fp16 scales [n][k/group]) into the device tile order. */
typedef struct am_gfx950_pack_int4_args {
  const uint8_t* logical;
  const uint16_t* scales;
  am_gfx950_weight dst;
} am_gfx950_pack_int4_args;
am_status_code am_gfx950_pack_int4(const am_gfx950_pack_int4_args* args, void* hip_stream);

/* GPTQ (4-bit, AutoGPTQ / optimum layout) -> this library's weight inputs.  No
 * counterpart kernel in the reference, whose validator only admits such tensors under
 * allow_quantized_tensors (hf_model_validator.cpp:196-243, model_validation_options.h:12).
 *   qweight [k/8][n] I32: nibble t of word (i, j) = q[8i + t][j] in 0..15
 *   qzeros  [groups][n/8] I32: nibble t of word (g, j) = stored zero of column 8j + t;
 *           z = (stored + zero_offset) & 15 (zero_offset 1 for checkpoint_format "gptq",
 *           which stores z - 1; 0 for "gptq_v2")
 *   scales  [groups][n], scales_dtype AM_DT_F16, AM_DT_BF16 or AM_DT_F32
 *   g_idx   [k] group of input feature k (NULL: k / group_size); out-of-range entries
 *           are clamped to the last group (the loader rejects them beforehand)
 * Exactly one output:
 *   out_f32     [n][k]: w[j][kk] = s * (q - z), one fp32 multiply of exact operands
 *               (exact: |q - z| <= 15 and s has at most 24 significant bits);
 *   out_logical [n][k/2] + out_scales [n][groups] fp16: the logical INT4 interchange of
 *               am_gfx950_pack_int4 (q - z as a two's complement nibble, low nibble =
 *               even k).  Meaningful only when every z is 8, g_idx is trivial and the
 *               scales are F16; then it is exact (same q - z and the same fp16 scale). */
typedef struct am_gfx950_gptq_args {
  const int32_t* qweight;
  const int32_t* qzeros;
  const void* scales;
  int32_t scales_dtype;
  int32_t zero_offset;
  const int32_t* g_idx;
  int64_t n, k, group_size;
  float* out_f32;
  uint8_t* out_logical;
  uint16_t* out_scales;
} am_gfx950_gptq_args;
am_status_code am_gfx950_gptq_unpack(const am_gfx950_gptq_args* args, void* hip_stream);

/* Dequantizes a device weight to fp32 [n][k] in logical k order:
 * w = float(q) * float(scale), one fp32 multiply (bit-exact SPEC). */
typedef struct am_gfx950_dequant_args {
  am_gfx950_weight w;
  float* out;
} am_gfx950_dequant_args;
am_status_code am_gfx950_dequant(const am_gfx950_dequant_args* args, void* hip_stream);

/* Bytes of data and scales for a weight of this shape/format. */
am_status_code am_gfx950_weight_bytes(int64_t n, int64_t k, int32_t format, int32_t group_size,
                                      int64_t* data_bytes, int64_t* scale_bytes);

/* Synthetic N(0, stddev) data of the build SPEC (SplitMix64 + Box-Muller with
 * portable arithmetic), elements [offset, offset+n) of stream (seed, tensor_id).
 * out dtype F32 or BF16 (RNE of the fp32 value). */
typedef struct am_gfx950_synth_args {
  uint64_t seed, tensor_id;
  double stddev;
  int64_t offset, n;
  void* out;
  int32_t dtype;
} am_gfx950_synth_args;
am_status_code am_gfx950_synth_normal(const am_gfx950_synth_args* args, void* hip_stream);

/* Synthetic token ids (I64) of the build SPEC, uniform in [0, vocab). */
am_status_code am_gfx950_synth_token_ids(uint64_t seed, uint64_t stream, int64_t vocab,
                                         int64_t n, int64_t* out, void* hip_stream);

/* Fill `n` elements of dtype F32/BF16 with a constant (norm gains = 1.0). */
am_status_code am_gfx950_fill(void* out, int32_t dtype, int64_t n, float value,
                              void* hip_stream);

/* ---------------- fused decode kernels (fusion of reference node runs) ------------- */

/* RmsNorm(input_layernorm) -> Linear q|k|v (one concatenated weight, rows q then k
 * then v) -> RoPE(q, k) -> KVCacheUpdate(k_rope, v), for one token at position *pos
 * (device).  Rounds at every reference op boundary.
 * rows > 1 (up to 16, bf16 activations): one token of each of `rows` independent
 * sequences: h [rows][hidden], pos [rows], q_out [rows][hq*d], and sequence r's cache
 * planes start cache_batch_stride elements after sequence r-1's.  rows 0 means 1.
 * pages != NULL (bf16): paged caches, sequence r's table row r. */
typedef struct am_gfx950_fused_qkv_args {
  const void* h;
  const void* norm_w;
  float eps;
  am_gfx950_weight w_qkv;
  const float* cos_tab;
  const float* sin_tab;
  const int64_t* pos;
  void* q_out;
  void* k_cache;
  void* v_cache;
  int64_t hq, hkv, head_dim, capacity;
  int32_t dtype;
  int64_t rows;
  int64_t cache_batch_stride;
  const am_gfx950_kv_pages* pages; /* NULL: contiguous planes */
} am_gfx950_fused_qkv_args;
am_status_code am_gfx950_fused_qkv(const am_gfx950_fused_qkv_args* args, void* hip_stream);

/* Linear (x @ W^T) -> Add(residual): h = round(h + round(W x)), in place on h.
 * rows > 1 (up to 16, bf16): x [rows][k], h [rows][n].  rows 0 means 1. */
typedef struct am_gfx950_fused_linear_residual_args {
  const void* x;
  am_gfx950_weight w;
  void* h;
  int32_t dtype;
  int64_t rows;
} am_gfx950_fused_linear_residual_args;
am_status_code am_gfx950_fused_linear_residual(const am_gfx950_fused_linear_residual_args* a,
                                               void* hip_stream);

/* RmsNorm(post_attention_layernorm) -> Linear gate, up (one weight: rows [0, F) are
 * gate, rows [F, 2F) are up) -> SiluMul.
 * rows > 1 (up to 16, bf16): h [rows][hidden], act_out [rows][F].  rows 0 means 1. */
typedef struct am_gfx950_fused_gate_up_args {
  const void* h;
  const void* norm_w;
  float eps;
  am_gfx950_weight w_gate_up;
  void* act_out;
  int32_t dtype;
  int64_t rows;
} am_gfx950_fused_gate_up_args;
am_status_code am_gfx950_fused_gate_up(const am_gfx950_fused_gate_up_args* a, void* hip_stream);

/* RmsNorm(final) -> Linear lm_head (fp32 logits) -> Argmax.  Writes logits [vocab]
 * (if non-NULL) and token_out[0]; with tokens_hist != NULL also tokens_hist[*step]
 * = token and increments *pos and *step (device-resident decode state).
 * workspace: am_gfx950_lm_head_workspace_bytes() bytes, first 4 bytes zero before
 * the first call (left zero).
 * rows > 1 (up to 16, bf16): h [rows][hidden], logits [rows][vocab] (required),
 * token_out [rows], pos [rows]; tokens_hist row r starts hist_stride elements after
 * row r-1 and *step is shared (incremented once).  The first 256 bytes of the
 * workspace must be zero before the first call (left zero).  rows 0 means 1. */
typedef struct am_gfx950_fused_lm_head_args {
  const void* h;
  const void* norm_w;
  float eps;
  am_gfx950_weight w;
  float* logits;
  int64_t* token_out;
  int64_t* tokens_hist;
  int64_t* pos;
  int64_t* step;
  int32_t dtype;
  void* workspace;
  int64_t workspace_bytes;
  int64_t rows;
  int64_t hist_stride;
} am_gfx950_fused_lm_head_args;
am_status_code am_gfx950_fused_lm_head(const am_gfx950_fused_lm_head_args* a, void* hip_stream);
int64_t am_gfx950_lm_head_workspace_bytes(void);

/* Embedding of the single token *token (device) into h (decode step input). */
am_status_code am_gfx950_embed_token(const int64_t* token, const void* table, int32_t dtype,
                                     int64_t vocab, int64_t hidden, void* h, int32_t* err_flag,
                                     void* hip_stream);

/* End of an unfused decode step (after Argmax): tokens_hist[*step] = *token,
 * ++*step, ++*pos.  The fused lm_head kernel does the same in its epilogue. */
am_status_code am_gfx950_decode_advance(const int64_t* token, int64_t* tokens_hist, int64_t* pos,
                                        int64_t* step, void* hip_stream);

/* The same for `rows` sequences decoded together: for each r, tokens_hist[r *
 * hist_stride + *step] = token[r] (when tokens_hist != NULL) and ++pos[r]; then
 * ++*step once. */
am_status_code am_gfx950_decode_advance_rows(const int64_t* token, int64_t rows, int64_t* tokens_hist,
                                             int64_t hist_stride, int64_t* pos, int64_t* step,
                                             void* hip_stream);

/* ---------------- persistent decode of all layers (one launch per token) ----------
 * The per-layer node sequence of model_graph_builder.cpp:133-290 (RmsNorm -> Linear
 * q|k|v -> RoPE -> KVCacheUpdate -> Attention -> Linear o -> Add -> RmsNorm -> Linear
 * gate|up -> SiluMul -> Linear down -> Add) for every layer of one token (batch 1),
 * with the roundings of the fused kernels above.  Replaces the per-layer sequence of
 * am_gfx950_fused_qkv / am_gfx950_attention / am_gfx950_fused_linear_residual /
 * am_gfx950_fused_gate_up / am_gfx950_fused_linear_residual (the executor's steps,
 * layer_runner.cpp:24-67) by one grid of one block per CU that exchanges step
 * outputs through the workspace.  Scope: bf16 activations, INT4 group-128 weights,
 * head_dim 128, hidden = q heads x 128 in {2048, 4096}, ffn a multiple of 128 up to
 * 16384, q heads <= 8 x kv heads, a 256-CU device (else UNIMPLEMENTED). */
typedef struct am_gfx950_decode_layer {
  am_gfx950_weight w_qkv;     /* [(hq + 2 hkv) * 128, hidden], rows q then k then v */
  am_gfx950_weight w_o;       /* [hidden, hq * 128] */
  am_gfx950_weight w_gate_up; /* [2 ffn, hidden], rows gate then up */
  am_gfx950_weight w_down;    /* [hidden, ffn] */
  const void* in_norm;        /* [hidden] input_layernorm gain */
  const void* post_norm;      /* [hidden] post_attention_layernorm gain */
  void* k_cache;              /* this layer's key plane [hkv][capacity][128] */
  void* v_cache;              /* this layer's value plane */
} am_gfx950_decode_layer;

typedef struct am_gfx950_decode_layers_args {
  const am_gfx950_decode_layer* layers; /* DEVICE array of num_layers entries */
  int64_t num_layers, hidden, hq, hkv, head_dim, ffn, capacity;
  float eps;
  const float* cos_tab; /* [capacity][64] */
  const float* sin_tab;
  const int64_t* pos; /* device: position of the token (KV row written) */
  void* h;            /* [hidden] bf16: the embedding in, the last layer's output out */
  void* workspace;    /* am_gfx950_decode_layers_workspace_bytes(), 256-byte aligned,
                         zero-filled once before the first call; calls on one
                         workspace must not overlap */
  int64_t workspace_bytes;
  int32_t dtype;  /* AM_DT_BF16 */
  void* timeline; /* optional (NULL = off): uint64 [num_layers][256 blocks][16] wall-clock
                     stamps (100 MHz) per block at the step points: 0 layer entry,
                     1 h gathered, 2 q|k|v done, 3 attention output gathered, 4 o done,
                     5 h gathered for the MLP, 6 gate|up done, 7 SiLU-Mul gathered;
                     attention blocks: 8 q|k|v flags seen, 9 q gathered, 10 partials
                     published; merge blocks: 11 partial flags seen, 12 partials read,
                     13 output published; 14 output flags seen (o step) */
} am_gfx950_decode_layers_args;
am_status_code am_gfx950_decode_layers(const am_gfx950_decode_layers_args* args, void* hip_stream);
int64_t am_gfx950_decode_layers_workspace_bytes(int64_t hidden, int64_t hq, int64_t hkv, int64_t head_dim,
                                                int64_t ffn);
/* Host-side check of the scalar arguments and (when host_layers != NULL, a host copy
 * of args->layers) of every layer's weight formats, shapes and alignment. */
am_status_code am_gfx950_decode_layers_validate(const am_gfx950_decode_layers_args* args,
                                                const am_gfx950_decode_layer* host_layers);
/* *out = 1 when a launch on this workspace ended early because a cross-block wait
 * timed out (the grid was not resident at once); the workspace must then be
 * zero-filled again.  Synchronous. */
am_status_code am_gfx950_decode_layers_aborted(const void* workspace, int32_t* out);

/* Host-side record of the last kernel an entry point of this library launched on the
 * calling thread: kernel family and template variant (e.g.
 * "gemv<bf16,int4,gate_up,norm=1,jm=2,p=1,nw=8,one=0>"), grid size in blocks,
 * threads per block and dynamic LDS bytes.  No counterpart in the reference (its
 * kernels are plain CPU functions): it lets a caller or a test confirm which kernel
 * variant a shape reached. */
typedef struct am_gfx950_launch_info {
  char kernel[96];
  int64_t grid;
  int32_t block_threads;
  int32_t lds_bytes;
} am_gfx950_launch_info;
am_status_code am_gfx950_last_launch(am_gfx950_launch_info* out);

/* Library / device information. */
int32_t am_gfx950_device_count(void);
const char* am_gfx950_version(void);

#ifdef __cplusplus
}
#endif
#endif
