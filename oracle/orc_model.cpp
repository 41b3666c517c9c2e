// CPU ORACLE -- test infrastructure only (see oracle.h).
//
// Whole-model Llama-dense forward in the node order of the reference graph builder
// (src/model/model_graph_builder.cpp:133-290 per layer, :356-415 around the layers):
//   Embedding
//   per layer: RmsNorm, Linear q/k/v, RoPE, KVCacheUpdate, Attention, Linear o, Add,
//              RmsNorm, Linear gate/up, SiluMul, Linear down, Add
//   RmsNorm(final), Linear lm_head, Argmax
// With act_bf16 every op output is rounded to bf16 (RNE) at the op boundary; the
// lm_head emits fp32 logits (build SPEC).

#include "oracle.h"

#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

namespace {

enum Role : uint64_t { kQ = 1, kK, kV, kO, kGate, kUp, kDown };
constexpr uint64_t kEmbedId = 0x01;
constexpr uint64_t kLmHeadId = 0x02;
inline uint64_t LayerTensorId(int layer, Role r) {
  return (static_cast<uint64_t>(layer + 1) << 8) | static_cast<uint64_t>(r);
}

struct QWeight {
  int64_t n = 0, k = 0;
  int fmt = 0;
  std::vector<float> f32;
  std::vector<uint16_t> bf16;
  std::vector<int8_t> q8;
  std::vector<float> s8;
  std::vector<uint8_t> q4;
  std::vector<uint16_t> s4;
  int64_t group = 128;

  void row(int64_t r, float* out) const {
    switch (fmt) {
      case 0: std::memcpy(out, f32.data() + r * k, sizeof(float) * static_cast<size_t>(k)); break;
      case 1:
        for (int64_t j = 0; j < k; ++j) out[j] = orc_bf16_to_f32(bf16[static_cast<size_t>(r * k + j)]);
        break;
      case 2: orc_dequant_int8(q8.data() + r * k, s8.data() + r, 1, k, out); break;
      default:
        orc_dequant_int4(q4.data() + r * (k / 2), s4.data() + r * (k / group), 1, k, group, out);
        break;
    }
  }
};

QWeight MakeWeight(uint64_t seed, uint64_t tid, int64_t n, int64_t k, int fmt, int64_t group) {
  QWeight w;
  w.n = n;
  w.k = k;
  w.fmt = fmt;
  w.group = group;
  const size_t count = static_cast<size_t>(n * k);
  if (fmt == 0) {
    w.f32.resize(count);
    orc_synth_normal_f32(seed, tid, 0.02, 0, n * k, w.f32.data());
    return w;
  }
  std::vector<uint16_t> b(count);
  // Generation is per element; split across threads (deterministic per index).
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; ++r) orc_synth_normal_bf16(seed, tid, 0.02, r * k, k, b.data() + r * k);
  if (fmt == 1) {
    w.bf16 = std::move(b);
    return w;
  }
  std::vector<float> f(count);
  for (size_t i = 0; i < count; ++i) f[i] = orc_bf16_to_f32(b[i]);
  // Rows are independent: quantize them in parallel (same result as one call).
  if (fmt == 2) {
    w.q8.resize(count);
    w.s8.resize(static_cast<size_t>(n));
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r) orc_quant_int8(f.data() + r * k, 1, k, w.q8.data() + r * k, w.s8.data() + r);
  } else {
    w.q4.resize(count / 2);
    w.s4.resize(static_cast<size_t>(n * (k / group)));
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r)
      orc_quant_int4(f.data() + r * k, 1, k, group, w.q4.data() + r * (k / 2), w.s4.data() + r * (k / group));
  }
  return w;
}

struct Layer {
  QWeight q, k, v, o, gate, up, down;
  std::vector<float> in_norm, post_norm;
  std::vector<float> kc, vc;  // [hkv][cap][d]
};

}  // namespace

struct orc_model {
  orc_model_config cfg{};
  std::vector<float> embed;  // [vocab][hidden] (bf16 values for bf16 models)
  std::vector<Layer> layers;
  std::vector<float> final_norm;
  std::vector<float> unit_gain;  // all 1.0 (ORC_SLIP_DROP_INPUT_GAIN)
  QWeight lm_head;
  std::vector<float> cos_tab, sin_tab;
  int fast = 0;
  int slip = 0;  // planted composition mistake for the tests that check the pins (0 = none)
};

namespace {

void LinearImpl(bool fast, const float* x, int64_t rows, const QWeight& w, float* out) {
  // Output columns in blocks of 16 dequantized rows: each token row is then read once
  // per block instead of once per column (the same dot per output either way).
  const int64_t n = w.n, k = w.k;
  constexpr int64_t kBlock = 16;
#pragma omp parallel
  {
    std::vector<float> buf(static_cast<size_t>(kBlock * k));
#pragma omp for schedule(dynamic, 1)
    for (int64_t c0 = 0; c0 < n; c0 += kBlock) {
      const int64_t nb = std::min<int64_t>(kBlock, n - c0);
      for (int64_t j = 0; j < nb; ++j) w.row(c0 + j, buf.data() + j * k);
      for (int64_t r = 0; r < rows; ++r) {
        const float* xr = x + r * k;
        for (int64_t j = 0; j < nb; ++j) {
          const float* wr = buf.data() + j * k;
          if (fast) {
            out[r * n + c0 + j] = orc_dot_avx2(xr, wr, k);
          } else {
            double acc = 0.0;
            for (int64_t i = 0; i < k; ++i) acc += static_cast<double>(xr[i]) * wr[i];
            out[r * n + c0 + j] = static_cast<float>(acc);
          }
        }
      }
    }
  }
}

void Linear(const orc_model* m, const float* x, int64_t rows, const QWeight& w, float* out) {
  LinearImpl(m->fast != 0, x, rows, w, out);
}

void MaybeRound(const orc_model* m, float* x, int64_t n) {
  if (m->cfg.act_bf16) orc_round_bf16_inplace(x, n);
}

void Norm(const orc_model* m, const float* x, const float* w, int64_t rows, float* out) {
  if (m->fast)
    orc_rmsnorm_avx2(x, w, rows, m->cfg.hidden, m->cfg.rms_eps, out);
  else
    orc_rmsnorm_scalar(x, w, rows, m->cfg.hidden, m->cfg.rms_eps, out);
  MaybeRound(m, out, rows * m->cfg.hidden);
}

}  // namespace

extern "C" {

orc_model* orc_model_create_synthetic(const orc_model_config* cfg, uint64_t seed, int32_t threads) {
  (void)threads;
  if (cfg == nullptr || cfg->num_layers <= 0 || cfg->hidden <= 0 || cfg->head_dim <= 0 ||
      cfg->num_q_heads % cfg->num_kv_heads != 0)
    return nullptr;
  auto* m = new orc_model();
  m->cfg = *cfg;
  const int64_t H = cfg->hidden, V = cfg->vocab, F = cfg->ffn, d = cfg->head_dim;
  const int64_t hq = cfg->num_q_heads, hkv = cfg->num_kv_heads;
  const int fmt = cfg->weight_format;
  const int64_t g = cfg->group_size > 0 ? cfg->group_size : 128;

  // The embedding table is stored in the activation dtype (SPEC): fp32 values for
  // fp32 activations, bf16 (RNE of the same fp32 stream) for bf16 activations.
  m->embed.resize(static_cast<size_t>(V * H));
  if (!cfg->act_bf16) {
    orc_synth_normal_f32(seed, kEmbedId, 0.02, 0, V * H, m->embed.data());
  } else {
    std::vector<uint16_t> b(static_cast<size_t>(V * H));
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < V; ++r) orc_synth_normal_bf16(seed, kEmbedId, 0.02, r * H, H, b.data() + r * H);
    for (size_t i = 0; i < b.size(); ++i) m->embed[i] = orc_bf16_to_f32(b[i]);
  }
  m->layers.resize(static_cast<size_t>(cfg->num_layers));
  for (int l = 0; l < cfg->num_layers; ++l) {
    Layer& L = m->layers[static_cast<size_t>(l)];
    L.q = MakeWeight(seed, LayerTensorId(l, kQ), hq * d, H, fmt, g);
    L.k = MakeWeight(seed, LayerTensorId(l, kK), hkv * d, H, fmt, g);
    L.v = MakeWeight(seed, LayerTensorId(l, kV), hkv * d, H, fmt, g);
    L.o = MakeWeight(seed, LayerTensorId(l, kO), H, hq * d, fmt, g);
    L.gate = MakeWeight(seed, LayerTensorId(l, kGate), F, H, fmt, g);
    L.up = MakeWeight(seed, LayerTensorId(l, kUp), F, H, fmt, g);
    L.down = MakeWeight(seed, LayerTensorId(l, kDown), H, F, fmt, g);
    L.in_norm.assign(static_cast<size_t>(H), 1.0f);
    L.post_norm.assign(static_cast<size_t>(H), 1.0f);
    L.kc.assign(static_cast<size_t>(hkv * cfg->max_tokens * d), 0.0f);
    L.vc.assign(static_cast<size_t>(hkv * cfg->max_tokens * d), 0.0f);
  }
  m->final_norm.assign(static_cast<size_t>(H), 1.0f);
  m->unit_gain.assign(static_cast<size_t>(H), 1.0f);
  m->lm_head = MakeWeight(seed, kLmHeadId, V, H, fmt, g);
  m->cos_tab.resize(static_cast<size_t>(cfg->max_tokens * (d / 2)));
  m->sin_tab.resize(m->cos_tab.size());
  orc_rope_table(cfg->max_tokens, d, cfg->rope_theta, m->cos_tab.data(), m->sin_tab.data());
  return m;
}

void orc_model_destroy(orc_model* m) { delete m; }

void orc_model_set_fast(orc_model* m, int32_t fast) { m->fast = fast; }

void orc_model_set_slip(orc_model* m, int32_t slip) { m->slip = slip; }

int orc_model_set_norm_gain(orc_model* m, int32_t kind, int32_t layer, const float* gain) {
  std::vector<float>* dst = nullptr;
  if (kind == 2) {
    dst = &m->final_norm;
  } else if ((kind == 0 || kind == 1) && layer >= 0 && layer < m->cfg.num_layers) {
    Layer& L = m->layers[static_cast<size_t>(layer)];
    dst = kind == 0 ? &L.in_norm : &L.post_norm;
  }
  if (dst == nullptr || gain == nullptr) return 3;
  std::memcpy(dst->data(), gain, sizeof(float) * dst->size());
  return 0;
}

void orc_set_threads(int32_t n) { omp_set_num_threads(n > 0 ? n : 1); }

int orc_model_forward(orc_model* m, const int64_t* ids, int64_t n, int64_t pos, float* logits) {
  const orc_model_config& c = m->cfg;
  const int64_t H = c.hidden, F = c.ffn, d = c.head_dim, hq = c.num_q_heads, hkv = c.num_kv_heads;
  const int64_t cap = c.max_tokens;
  if (n <= 0 || pos < 0 || pos + n > cap) return 11;
  std::vector<float> h(static_cast<size_t>(n * H)), xn(h.size()), tmp(h.size());
  std::vector<float> q(static_cast<size_t>(n * hq * d)), k(static_cast<size_t>(n * hkv * d)),
      v(k.size()), attn(q.size());
  std::vector<float> gt(static_cast<size_t>(n * F)), up(gt.size()), act(gt.size());
  std::vector<int64_t> positions(static_cast<size_t>(n));
  for (int64_t s = 0; s < n; ++s) positions[static_cast<size_t>(s)] = pos + s;

  if (int rc = orc_embedding_i64(ids, n, m->embed.data(), c.vocab, H, h.data()); rc != 0) return rc;

  for (Layer& L : m->layers) {
    {
      // which gain the input norm applies (the slips are planted composition mistakes)
      const std::vector<float>& g = m->slip == ORC_SLIP_SWAP_NORM_GAINS ? L.post_norm
                                    : m->slip == ORC_SLIP_DROP_INPUT_GAIN ? m->unit_gain
                                                                          : L.in_norm;
      Norm(m, h.data(), g.data(), n, xn.data());
    }
    Linear(m, xn.data(), n, L.q, q.data());
    MaybeRound(m, q.data(), n * hq * d);
    Linear(m, xn.data(), n, L.k, k.data());
    MaybeRound(m, k.data(), n * hkv * d);
    Linear(m, xn.data(), n, L.v, v.data());
    MaybeRound(m, v.data(), n * hkv * d);
    orc_rope(q.data(), n, hq, d, positions.data(), m->cos_tab.data(), m->sin_tab.data());
    MaybeRound(m, q.data(), n * hq * d);
    if (m->slip != ORC_SLIP_ROPE_AFTER_KV) {
      orc_rope(k.data(), n, hkv, d, positions.data(), m->cos_tab.data(), m->sin_tab.data());
      MaybeRound(m, k.data(), n * hkv * d);
    }
    for (int64_t s = 0; s < n; ++s)
      for (int64_t g = 0; g < hkv; ++g) {
        std::memcpy(&L.kc[static_cast<size_t>((g * cap + pos + s) * d)], &k[static_cast<size_t>((s * hkv + g) * d)],
                    sizeof(float) * static_cast<size_t>(d));
        std::memcpy(&L.vc[static_cast<size_t>((g * cap + pos + s) * d)], &v[static_cast<size_t>((s * hkv + g) * d)],
                    sizeof(float) * static_cast<size_t>(d));
      }
    if (m->slip == ORC_SLIP_GQA_MODULO) {
      // q head h reads kv head h % hkv: reorder the heads so the contiguous-group
      // attention below sees that mapping, then put the outputs back
      const int64_t grp = hq / hkv;
      std::vector<float> qp(q.size()), ap(attn.size());
      auto slot = [&](int64_t h) { return (h % hkv) * grp + h / hkv; };
      for (int64_t s = 0; s < n; ++s)
        for (int64_t hh = 0; hh < hq; ++hh)
          std::memcpy(&qp[static_cast<size_t>((s * hq + slot(hh)) * d)], &q[static_cast<size_t>((s * hq + hh) * d)],
                      sizeof(float) * static_cast<size_t>(d));
      orc_attention(qp.data(), L.kc.data(), L.vc.data(), n, hq, hkv, d, cap, pos, ap.data());
      for (int64_t s = 0; s < n; ++s)
        for (int64_t hh = 0; hh < hq; ++hh)
          std::memcpy(&attn[static_cast<size_t>((s * hq + hh) * d)], &ap[static_cast<size_t>((s * hq + slot(hh)) * d)],
                      sizeof(float) * static_cast<size_t>(d));
    } else {
      orc_attention(q.data(), L.kc.data(), L.vc.data(), n, hq, hkv, d, cap, pos, attn.data());
    }
    MaybeRound(m, attn.data(), n * hq * d);
    Linear(m, attn.data(), n, L.o, tmp.data());
    MaybeRound(m, tmp.data(), n * H);
    if (m->slip == ORC_SLIP_RESIDUAL_NORMED)
      for (size_t i = 0; i < h.size(); ++i) h[i] = xn[i] + tmp[i];
    else
      for (size_t i = 0; i < h.size(); ++i) h[i] += tmp[i];
    MaybeRound(m, h.data(), n * H);

    Norm(m, h.data(), (m->slip == ORC_SLIP_SWAP_NORM_GAINS ? L.in_norm : L.post_norm).data(), n, xn.data());
    Linear(m, xn.data(), n, L.gate, gt.data());
    MaybeRound(m, gt.data(), n * F);
    Linear(m, xn.data(), n, L.up, up.data());
    MaybeRound(m, up.data(), n * F);
    orc_silu_mul(gt.data(), up.data(), n * F, act.data());
    MaybeRound(m, act.data(), n * F);
    Linear(m, act.data(), n, L.down, tmp.data());
    MaybeRound(m, tmp.data(), n * H);
    for (size_t i = 0; i < h.size(); ++i) h[i] += tmp[i];
    MaybeRound(m, h.data(), n * H);
  }
  // Only the last row's logits feed the next token.
  if (m->slip == ORC_SLIP_NO_FINAL_NORM)
    std::memcpy(xn.data(), h.data() + (n - 1) * H, sizeof(float) * static_cast<size_t>(H));
  else
    Norm(m, h.data() + (n - 1) * H,
         (m->slip == ORC_SLIP_FINAL_GAIN_FROM_LAYER ? m->layers.back().post_norm : m->final_norm).data(), 1,
         xn.data());
  Linear(m, xn.data(), 1, m->lm_head, logits);
  return 0;
}

int orc_model_generate(orc_model* m, const int64_t* prompt, int64_t n_prompt, int64_t n_new,
                       int64_t* out_tokens, float* last_logits) {
  if (n_prompt <= 0 || n_new <= 0) return 3;
  std::vector<float> logits(static_cast<size_t>(m->cfg.vocab));
  int rc = orc_model_forward(m, prompt, n_prompt, 0, logits.data());
  if (rc != 0) return rc;
  int64_t tok = orc_argmax(logits.data(), m->cfg.vocab);
  out_tokens[0] = tok;
  for (int64_t i = 1; i < n_new; ++i) {
    rc = orc_model_forward(m, &tok, 1, n_prompt + i - 1, logits.data());
    if (rc != 0) return rc;
    tok = orc_argmax(logits.data(), m->cfg.vocab);
    out_tokens[i] = tok;
  }
  if (last_logits != nullptr)
    std::memcpy(last_logits, logits.data(), sizeof(float) * logits.size());
  return 0;
}

// ---------------- per-shape GEMV of the CPU baseline ----------------
// A weight of one format filled with cheap deterministic bytes (the timing does not
// depend on the values, and the seeded normal generator would cost seconds per GB),
// multiplied by one activation row through the model's own Linear path: rows
// dequantized on the fly in blocks of 16, each dotted with the AVX2 kernel.
struct orc_qweight {
  QWeight w;
};

orc_qweight* orc_qweight_create(int64_t n, int64_t k, int32_t fmt, int64_t group, uint64_t seed) {
  if (n <= 0 || k <= 0 || fmt < 1 || fmt > 3 || (fmt == 3 && (group <= 0 || k % group != 0))) return nullptr;
  auto* q = new orc_qweight();
  QWeight& w = q->w;
  w.n = n;
  w.k = k;
  w.fmt = fmt;
  w.group = group;
  const size_t count = static_cast<size_t>(n * k);
  auto bits = [seed](uint64_t i) { return orc_splitmix64(seed ^ (i * 0x9E3779B97F4A7C15ull)); };
  if (fmt == 1) {
    w.bf16.resize(count);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i) {
      // 2^-7 <= |value| < 2^-4: exponent 0x78..0x7A, random sign and mantissa
      const uint64_t b = bits(static_cast<uint64_t>(i));
      w.bf16[static_cast<size_t>(i)] =
          static_cast<uint16_t>(((b >> 8) & 0x8000u) | ((0x78u + (b & 1u) + ((b >> 1) & 1u)) << 7) | ((b >> 16) & 0x7Fu));
    }
  } else if (fmt == 2) {
    w.q8.resize(count);
    w.s8.assign(static_cast<size_t>(n), 0.02f / 127.0f);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count); ++i)
      w.q8[static_cast<size_t>(i)] = static_cast<int8_t>(static_cast<int>(bits(static_cast<uint64_t>(i)) % 255u) - 127);
  } else {
    w.q4.resize(count / 2);
    w.s4.assign(static_cast<size_t>(n * (k / group)), orc_f32_to_f16(0.02f / 7.0f));
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < static_cast<int64_t>(count / 2); ++i)
      w.q4[static_cast<size_t>(i)] = static_cast<uint8_t>(bits(static_cast<uint64_t>(i)));
  }
  return q;
}

void orc_qweight_destroy(orc_qweight* q) { delete q; }

int64_t orc_qweight_bytes(const orc_qweight* q) {
  const QWeight& w = q->w;
  if (w.fmt == 1) return w.n * w.k * 2;
  if (w.fmt == 2) return w.n * w.k + w.n * 4;
  return w.n * w.k / 2 + w.n * (w.k / w.group) * 2;
}

void orc_qweight_gemv(const orc_qweight* q, const float* x, float* y) { LinearImpl(true, x, 1, q->w, y); }

}  // extern "C"
