// oracle/model.cpp — restatement of src/model.rs (forward pass, KV cache),
// src/sampler.rs and the bench protocol of src/main.rs.
// TEST INFRASTRUCTURE ONLY (the parity oracle / CPU baseline).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "cpu_ref.h"
#include "internal.h"

using namespace orc;

struct Weight {  // model.rs:36-53: a borrowed view resolved at load time
  uint32_t ty = 0;
  const uint8_t* data = nullptr;
  size_t cols = 0, rows = 0;
  bool present() const { return data != nullptr; }
};

struct LayerW {  // model.rs:56-71
  std::vector<float> attn_norm, ffn_norm, attn_q_norm, attn_k_norm, bq, bk, bv;
  Weight attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down;
};

struct orc_model {
  orc_config cfg;
  std::vector<LayerW> layers;
  Weight token_embd, output;
  std::vector<float> output_norm;
  std::vector<float> rope_inv_freq;  // model.rs:221-227
};

struct orc_cache {  // model.rs:107-134 (KvCache + Workspace)
  size_t max_ctx = 0, len = 0;
  std::vector<std::vector<float>> k, v;
  std::vector<float> x, xb, q, kk, vv, attn, gate, up, scores;
  float* dump = nullptr;
  size_t dump_max_tokens = 0;
};

static std::vector<float> to_f32(uint32_t ty, const void* bytes, size_t n) {  // tensor.rs:65-77
  std::vector<float> out(n);
  dequant_row(ty, (const uint8_t*)bytes, n, out.data());
  return out;
}

extern "C" {

orc_model* orc_model_create(const orc_config* cfg) {
  orc_model* m = new orc_model();
  m->cfg = *cfg;
  m->layers.resize(cfg->n_layer);
  return m;
}

int orc_model_set_tensor(orc_model* m, int kind, int layer, uint32_t ty, const void* bytes, size_t n_cols,
                         size_t n_rows) {
  if (block_size(ty) == 0) return -1;
  if (kind >= ORC_T_ATTN_NORM && (layer < 0 || (size_t)layer >= m->layers.size())) return -2;
  Weight w{ty, (const uint8_t*)bytes, n_cols, n_rows};
  size_t n = n_cols * n_rows;
  LayerW* L = kind >= ORC_T_ATTN_NORM ? &m->layers[layer] : nullptr;
  switch (kind) {
    case ORC_T_TOKEN_EMBD: m->token_embd = w; break;
    case ORC_T_OUTPUT_NORM: m->output_norm = to_f32(ty, bytes, n); break;
    case ORC_T_OUTPUT: m->output = w; break;
    case ORC_T_ATTN_NORM: L->attn_norm = to_f32(ty, bytes, n); break;
    case ORC_T_ATTN_Q: L->attn_q = w; break;
    case ORC_T_ATTN_K: L->attn_k = w; break;
    case ORC_T_ATTN_V: L->attn_v = w; break;
    case ORC_T_ATTN_OUTPUT: L->attn_output = w; break;
    case ORC_T_ATTN_Q_NORM: L->attn_q_norm = to_f32(ty, bytes, n); break;
    case ORC_T_ATTN_K_NORM: L->attn_k_norm = to_f32(ty, bytes, n); break;
    case ORC_T_FFN_NORM: L->ffn_norm = to_f32(ty, bytes, n); break;
    case ORC_T_FFN_GATE: L->ffn_gate = w; break;
    case ORC_T_FFN_UP: L->ffn_up = w; break;
    case ORC_T_FFN_DOWN: L->ffn_down = w; break;
    case ORC_T_ATTN_Q_BIAS: L->bq = to_f32(ty, bytes, n); break;
    case ORC_T_ATTN_K_BIAS: L->bk = to_f32(ty, bytes, n); break;
    case ORC_T_ATTN_V_BIAS: L->bv = to_f32(ty, bytes, n); break;
    default: return -3;
  }
  return 0;
}

int orc_model_finalize(orc_model* m) {
  const orc_config& c = m->cfg;
  size_t half = c.head_dim / 2;
  m->rope_inv_freq.resize(half);
  for (size_t i = 0; i < half; i++) {  // model.rs:222-227
    float e = -2.0f * (float)i / (float)c.head_dim;
    m->rope_inv_freq[i] = std::pow(c.rope_theta, e);
  }
  if (!m->token_embd.present() || m->output_norm.size() != c.n_embd) return -1;
  for (auto& L : m->layers) {
    if (!L.attn_q.present() || !L.attn_k.present() || !L.attn_v.present() || !L.attn_output.present() ||
        !L.ffn_gate.present() || !L.ffn_up.present() || !L.ffn_down.present() || L.attn_norm.empty() ||
        L.ffn_norm.empty())
      return -1;
    if (c.has_qk_norm && (L.attn_q_norm.empty() || L.attn_k_norm.empty())) return -1;
  }
  return 0;
}

void orc_model_destroy(orc_model* m) { delete m; }

orc_cache* orc_cache_create(orc_model* m, size_t max_ctx) {
  const orc_config& c = m->cfg;
  if (max_ctx > c.n_ctx) max_ctx = c.n_ctx;  // model.rs:340
  orc_cache* kc = new orc_cache();
  size_t kv_dim = (size_t)c.n_head_kv * c.head_dim, q_dim = (size_t)c.n_head * c.head_dim;
  kc->max_ctx = max_ctx;
  kc->k.assign(c.n_layer, std::vector<float>(max_ctx * kv_dim, 0.f));
  kc->v.assign(c.n_layer, std::vector<float>(max_ctx * kv_dim, 0.f));
  kc->x.resize(c.n_embd);
  kc->xb.resize(c.n_embd);
  kc->q.resize(q_dim);
  kc->kk.resize(kv_dim);
  kc->vv.resize(kv_dim);
  kc->attn.resize(q_dim);
  kc->gate.resize(c.n_ff);
  kc->up.resize(c.n_ff);
  kc->scores.resize(max_ctx);
  return kc;
}
void orc_cache_reset(orc_cache* c) { c->len = 0; }
size_t orc_cache_len(const orc_cache* c) { return c->len; }
size_t orc_cache_max_ctx(const orc_cache* c) { return c->max_ctx; }
void orc_cache_destroy(orc_cache* c) { delete c; }
void orc_set_hidden_dump(orc_cache* c, float* buf, size_t max_tokens) {
  c->dump = buf;
  c->dump_max_tokens = max_tokens;
}
const float* orc_cache_k(const orc_cache* c, int layer) { return c->k[layer].data(); }
const float* orc_cache_v(const orc_cache* c, int layer) { return c->v[layer].data(); }

}  // extern "C"

static void mm(const Weight& w, const float* x, float* y, int mode) { matmul(w.ty, w.data, w.rows, w.cols, x, y, mode); }
static void mmb(const Weight& w, const float* xs, size_t n, float* ys, int mode) {
  matmul_batch(w.ty, w.data, w.rows, w.cols, xs, n, ys, mode);
}
static void embed_row(const Weight& w, uint32_t tok, float* out) {  // tensor.rs:59-62
  size_t rb = (size_t)type_size(w.ty) * (w.cols / (size_t)block_size(w.ty));
  dequant_row(w.ty, w.data + (size_t)tok * rb, w.cols, out);
}

// One (head, query) attention row: model.rs:674-689 / 693-710 / 525-543.
static void attend_head(const float* qh, const float* kc, const float* vc, size_t t, size_t kv_dim, size_t kvh,
                        size_t hd, float scale, float* scores, float* ah, int mode) {
  for (size_t j = 0; j < t; j++) scores[j] = dot(qh, kc + j * kv_dim + kvh * hd, hd) * scale;
  if (mode & ORC_MODE_SPLIT_ATTN) {
    // NOT the reference: the softmax sum and the PV sums taken over four
    // contiguous position splits, each in order, then combined pairwise (the
    // order a split-K decode kernel uses); everything else unchanged
    float mx = scores[0];
    for (size_t j = 1; j < t; j++)
      if (scores[j] > mx) mx = scores[j];
    for (size_t j = 0; j < t; j++) scores[j] = std::exp(scores[j] - mx);
    const size_t q = (t + 3) / 4;
    float part[4] = {0.f, 0.f, 0.f, 0.f};
    for (size_t j = 0; j < t; j++) part[j / q] += scores[j];
    const float sum = (part[0] + part[1]) + (part[2] + part[3]);
    if (sum > 0.0f) {
      const float inv = 1.0f / sum;
      for (size_t j = 0; j < t; j++) scores[j] *= inv;
    }
    for (size_t i = 0; i < hd; i++) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (size_t j = 0; j < t; j++) acc[j / q] += scores[j] * vc[j * kv_dim + kvh * hd + i];
      ah[i] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    return;
  }
  softmax_inplace(scores, t);
  for (size_t i = 0; i < hd; i++) ah[i] = 0.0f;
  for (size_t j = 0; j < t; j++) saxpy(ah, scores[j], vc + j * kv_dim + kvh * hd, hd);
}

// model.rs:585-738
static void forward_one(orc_model* m, uint32_t token, size_t pos, orc_cache* c, float* logits, int mode) {
  const orc_config& cfg = m->cfg;
  size_t E = cfg.n_embd, hd = cfg.head_dim, H = cfg.n_head, K = cfg.n_head_kv, F = cfg.n_ff;
  size_t kv_dim = K * hd;
  float eps = cfg.rms_eps;
  size_t t = pos + 1;
  embed_row(m->token_embd, token, c->x.data());
  float scale = 1.0f / std::sqrt((float)hd);
  size_t group = H / K;
  if (group < 1) group = 1;
  for (size_t l = 0; l < cfg.n_layer; l++) {
    LayerW& L = m->layers[l];
    rmsnorm(c->xb.data(), c->x.data(), L.attn_norm.data(), E, eps, mode);
    mm(L.attn_q, c->xb.data(), c->q.data(), mode);
    mm(L.attn_k, c->xb.data(), c->kk.data(), mode);
    mm(L.attn_v, c->xb.data(), c->vv.data(), mode);
    for (size_t i = 0; i < L.bq.size(); i++) c->q[i] += L.bq[i];
    for (size_t i = 0; i < L.bk.size(); i++) c->kk[i] += L.bk[i];
    for (size_t i = 0; i < L.bv.size(); i++) c->vv[i] += L.bv[i];
    if (!L.attn_q_norm.empty() && !L.attn_k_norm.empty()) {
      for (size_t h = 0; h < H; h++) rmsnorm_head(c->q.data() + h * hd, L.attn_q_norm.data(), hd, eps, mode);
      for (size_t h = 0; h < K; h++) rmsnorm_head(c->kk.data() + h * hd, L.attn_k_norm.data(), hd, eps, mode);
    }
    rope_neox_freqs(c->q.data(), H, hd, pos, m->rope_inv_freq.data());
    rope_neox_freqs(c->kk.data(), K, hd, pos, m->rope_inv_freq.data());
    std::memcpy(c->k[l].data() + pos * kv_dim, c->kk.data(), kv_dim * sizeof(float));
    std::memcpy(c->v[l].data() + pos * kv_dim, c->vv.data(), kv_dim * sizeof(float));
    const float* kc = c->k[l].data();
    const float* vc = c->v[l].data();
    if (t * H >= 1024) {  // model.rs:668-690 (parallel heads; same arithmetic)
      parallel_for(H, [&](size_t h) {
        std::vector<float> scores(t);
        attend_head(c->q.data() + h * hd, kc, vc, t, kv_dim, h / group, hd, scale, scores.data(),
                    c->attn.data() + h * hd, mode);
      });
    } else {
      for (size_t h = 0; h < H; h++)
        attend_head(c->q.data() + h * hd, kc, vc, t, kv_dim, h / group, hd, scale, c->scores.data(),
                    c->attn.data() + h * hd, mode);
    }
    mm(L.attn_output, c->attn.data(), c->xb.data(), mode);
    for (size_t i = 0; i < E; i++) c->x[i] += c->xb[i];
    rmsnorm(c->xb.data(), c->x.data(), L.ffn_norm.data(), E, eps, mode);
    mm(L.ffn_gate, c->xb.data(), c->gate.data(), mode);
    mm(L.ffn_up, c->xb.data(), c->up.data(), mode);
    for (size_t i = 0; i < F; i++) c->gate[i] = silu(c->gate[i]) * c->up[i];
    mm(L.ffn_down, c->gate.data(), c->xb.data(), mode);
    for (size_t i = 0; i < E; i++) c->x[i] += c->xb[i];
    if (c->dump && c->dump_max_tokens >= 1) std::memcpy(c->dump + l * c->dump_max_tokens * E, c->x.data(), E * 4);
  }
  c->len = t;
  if (logits) {
    rmsnorm(c->xb.data(), c->x.data(), m->output_norm.data(), E, eps, mode);
    const Weight& w = m->output.present() ? m->output : m->token_embd;
    mm(w, c->xb.data(), logits, mode);
  }
}

// model.rs:384-583
static void forward_batch(orc_model* m, const uint32_t* tokens, size_t n_in, size_t start_pos, orc_cache* c,
                          float* out, int mode) {
  const orc_config& cfg = m->cfg;
  size_t n = std::min(n_in, c->max_ctx > start_pos ? c->max_ctx - start_pos : (size_t)0);
  if (n == 0) return;
  size_t E = cfg.n_embd, hd = cfg.head_dim, H = cfg.n_head, K = cfg.n_head_kv, F = cfg.n_ff;
  size_t kv_dim = K * hd, q_dim = H * hd;
  float eps = cfg.rms_eps;
  std::vector<float> xs(n * E);
  for (size_t i = 0; i < n; i++) embed_row(m->token_embd, tokens[i], xs.data() + i * E);
  std::vector<float> xb_all(n * E), q_all(n * q_dim), k_all(n * kv_dim), v_all(n * kv_dim), attn_all(n * q_dim),
      gate_all(n * F), up_all(n * F);
  float scale = 1.0f / std::sqrt((float)hd);
  size_t group = H / K;
  if (group < 1) group = 1;
  for (size_t l = 0; l < cfg.n_layer; l++) {
    LayerW& L = m->layers[l];
    for (size_t i = 0; i < n; i++) rmsnorm(xb_all.data() + i * E, xs.data() + i * E, L.attn_norm.data(), E, eps, mode);
    mmb(L.attn_q, xb_all.data(), n, q_all.data(), mode);
    mmb(L.attn_k, xb_all.data(), n, k_all.data(), mode);
    mmb(L.attn_v, xb_all.data(), n, v_all.data(), mode);
    if (!L.bq.empty())
      for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < q_dim; j++) q_all[i * q_dim + j] += L.bq[j];
    if (!L.bk.empty())
      for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < kv_dim; j++) k_all[i * kv_dim + j] += L.bk[j];
    if (!L.bv.empty())
      for (size_t i = 0; i < n; i++)
        for (size_t j = 0; j < kv_dim; j++) v_all[i * kv_dim + j] += L.bv[j];
    if (!L.attn_q_norm.empty() && !L.attn_k_norm.empty()) {
      for (size_t i = 0; i < n; i++) {
        for (size_t h = 0; h < H; h++)
          rmsnorm_head(q_all.data() + i * q_dim + h * hd, L.attn_q_norm.data(), hd, eps, mode);
        for (size_t h = 0; h < K; h++)
          rmsnorm_head(k_all.data() + i * kv_dim + h * hd, L.attn_k_norm.data(), hd, eps, mode);
      }
    }
    for (size_t i = 0; i < n; i++) {
      size_t pos = start_pos + i;
      rope_neox_freqs(q_all.data() + i * q_dim, H, hd, pos, m->rope_inv_freq.data());
      rope_neox_freqs(k_all.data() + i * kv_dim, K, hd, pos, m->rope_inv_freq.data());
      std::memcpy(c->k[l].data() + pos * kv_dim, k_all.data() + i * kv_dim, kv_dim * 4);
      std::memcpy(c->v[l].data() + pos * kv_dim, v_all.data() + i * kv_dim, kv_dim * 4);
    }
    const float* kc = c->k[l].data();
    const float* vc = c->v[l].data();
    parallel_for(n, [&](size_t i) {  // model.rs:520-545
      std::vector<float> scores(start_pos + n);
      size_t t = start_pos + i + 1;
      for (size_t h = 0; h < H; h++)
        attend_head(q_all.data() + i * q_dim + h * hd, kc, vc, t, kv_dim, h / group, hd, scale, scores.data(),
                    attn_all.data() + i * q_dim + h * hd, mode & ~ORC_MODE_SPLIT_ATTN);
    });
    mmb(L.attn_output, attn_all.data(), n, xb_all.data(), mode);
    for (size_t i = 0; i < n * E; i++) xs[i] += xb_all[i];
    for (size_t i = 0; i < n; i++) rmsnorm(xb_all.data() + i * E, xs.data() + i * E, L.ffn_norm.data(), E, eps, mode);
    mmb(L.ffn_gate, xb_all.data(), n, gate_all.data(), mode);
    mmb(L.ffn_up, xb_all.data(), n, up_all.data(), mode);
    for (size_t i = 0; i < n * F; i++) gate_all[i] = silu(gate_all[i]) * up_all[i];
    mmb(L.ffn_down, gate_all.data(), n, xb_all.data(), mode);
    for (size_t i = 0; i < n * E; i++) xs[i] += xb_all[i];
    if (c->dump) {
      size_t nd = std::min(n, c->dump_max_tokens);
      std::memcpy(c->dump + l * c->dump_max_tokens * E, xs.data(), nd * E * 4);
    }
  }
  c->len = start_pos + n;
  std::vector<float> xb(E);
  rmsnorm(xb.data(), xs.data() + (n - 1) * E, m->output_norm.data(), E, eps, mode);
  const Weight& w = m->output.present() ? m->output : m->token_embd;
  mm(w, xb.data(), out, mode);
}

// ---------------------------------------------------------------------------
// sampler.rs
// ---------------------------------------------------------------------------
struct orc_sampler {
  uint64_t state;
};

extern "C" {

void orc_forward_into(orc_model* m, orc_cache* c, const uint32_t* tokens, size_t n, size_t start_pos,
                      float* logits, int mode) {
  if (n > 1) {  // model.rs:361-374
    forward_batch(m, tokens, n, start_pos, c, logits, mode);
    return;
  }
  for (size_t i = 0; i < n; i++) forward_one(m, tokens[i], start_pos + i, c, i == n - 1 ? logits : nullptr, mode);
}

orc_sampler* orc_sampler_create(uint64_t seed) { return new orc_sampler{seed | 1}; }
void orc_sampler_destroy(orc_sampler* s) { delete s; }
uint64_t orc_sampler_next_u64(orc_sampler* s) {  // sampler.rs:40-48
  uint64_t x = s->state;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  s->state = x;
  return x * 0x2545F4914F6CDD1DULL;
}
float orc_sampler_next_f32(orc_sampler* s) {  // sampler.rs:51-54
  return (float)(orc_sampler_next_u64(s) >> 40) / (float)(1ULL << 24);
}

// sampler.rs:56-163
uint32_t orc_sampler_sample(orc_sampler* s, const float* logits, size_t n, const orc_sampling_params* p,
                            const uint32_t* recent, size_t n_recent) {
  if (n == 0) return 0;
  if (p->temperature <= 0.0f && p->repetition_penalty == 1.0f) {
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
      if (logits[i] > logits[best]) best = i;
    return (uint32_t)best;
  }
  std::vector<float> probs(logits, logits + n);
  if (p->repetition_penalty != 1.0f) {
    float pen = p->repetition_penalty;
    size_t start = p->repeat_last_n == 0 ? 0 : (n_recent > p->repeat_last_n ? n_recent - p->repeat_last_n : 0);
    std::vector<uint32_t> seen;
    for (size_t k = start; k < n_recent; k++) {
      uint32_t t = recent[k];
      if ((size_t)t >= n || std::find(seen.begin(), seen.end(), t) != seen.end()) continue;
      seen.push_back(t);
      if (probs[t] > 0.0f)
        probs[t] /= pen;
      else
        probs[t] *= pen;
    }
  }
  if (p->temperature <= 0.0f) {
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
      if (probs[i] > probs[best]) best = i;
    return (uint32_t)best;
  }
  float inv_t = 1.0f / p->temperature;
  for (auto& v : probs) v *= inv_t;
  softmax_inplace(probs.data(), n);
  size_t k = (p->top_k == 0 || p->top_k > n) ? n : p->top_k;
  std::vector<size_t> idx(n);
  for (size_t i = 0; i < n; i++) idx[i] = i;
  // select_nth_unstable_by + truncate, then sort_by (sampler.rs:122-132).
  // For distinct probabilities that is the k largest in descending order.
  // Exactly equal probabilities are ordered by token id here; the reference
  // leaves their order to the internals of Rust's selection, which nothing
  // in its tests fixes (tie order is parity-unpinned against the reference).
  auto desc = [&](size_t a, size_t b) { return probs[b] < probs[a] || (probs[b] == probs[a] && a < b); };
  if (k < n) {
    std::nth_element(idx.begin(), idx.begin() + (k - 1), idx.end(), desc);
    idx.resize(k);
  }
  std::stable_sort(idx.begin(), idx.end(), desc);
  size_t cutoff = idx.size();
  if (p->top_p > 0.0f && p->top_p < 1.0f) {
    float cum = 0.f;
    for (size_t pos = 0; pos < idx.size(); pos++) {
      cum += probs[idx[pos]];
      if (cum >= p->top_p) {
        cutoff = pos + 1;
        break;
      }
    }
  }
  idx.resize(cutoff);
  float sum = 0.f;
  for (size_t i : idx) sum += probs[i];
  if (sum <= 0.0f) return (uint32_t)idx[0];
  float r = orc_sampler_next_f32(s) * sum;
  for (size_t i : idx) {
    r -= probs[i];
    if (r <= 0.0f) return (uint32_t)i;
  }
  return (uint32_t)idx.back();
}

uint32_t orc_argmax(const float* x, size_t n) {  // main.rs:453-463
  size_t best = 0;
  float best_v = -INFINITY;
  for (size_t i = 0; i < n; i++)
    if (x[i] > best_v) {
      best_v = x[i];
      best = i;
    }
  return (uint32_t)best;
}

// model.rs:741-776
size_t orc_generate(orc_model* m, orc_cache* c, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                    const orc_sampling_params* p, uint32_t eos, uint32_t* out_tokens, int mode) {
  orc_sampler* s = orc_sampler_create(p->seed);
  c->len = 0;
  std::vector<float> logits(m->cfg.vocab_size);
  orc_forward_into(m, c, prompt, n_prompt, 0, logits.data(), mode);
  std::vector<uint32_t> recent(prompt, prompt + n_prompt);
  size_t produced = 0;
  for (size_t i = 0; i < max_new; i++) {
    uint32_t next = orc_sampler_sample(s, logits.data(), logits.size(), p, recent.data(), recent.size());
    if (next == eos) break;
    out_tokens[produced++] = next;
    recent.push_back(next);
    if (c->len >= c->max_ctx) break;
    orc_forward_into(m, c, &next, 1, c->len, logits.data(), mode);
  }
  orc_sampler_destroy(s);
  return produced;
}

// main.rs:466-530 (EOS ignored so the token count is fixed)
int orc_bench(orc_model* m, orc_cache* c, const uint32_t* prompt, size_t n_prompt, size_t n_gen, int mode,
              int do_warmup, orc_bench_result* out, uint32_t* out_tokens) {
  if (n_prompt == 0) return -1;
  std::vector<float> logits(m->cfg.vocab_size);
  using clk = std::chrono::steady_clock;
  if (do_warmup) {
    c->len = 0;
    orc_forward_into(m, c, prompt, n_prompt, 0, logits.data(), mode);
  }
  c->len = 0;
  auto t0 = clk::now();
  orc_forward_into(m, c, prompt, n_prompt, 0, logits.data(), mode);
  double pt = std::chrono::duration<double>(clk::now() - t0).count();
  size_t generated = 0;
  uint32_t next = orc_argmax(logits.data(), logits.size());
  auto t1 = clk::now();
  for (size_t i = 0; i < n_gen; i++) {
    if (c->len >= c->max_ctx) break;
    if (out_tokens) out_tokens[generated] = next;
    orc_forward_into(m, c, &next, 1, c->len, logits.data(), mode);
    generated++;
    next = orc_argmax(logits.data(), logits.size());
  }
  double gt = std::chrono::duration<double>(clk::now() - t1).count();
  if (out_tokens) out_tokens[generated] = next;
  out->prefill_s = pt;
  out->decode_s = gt;
  out->prompt_len = n_prompt;
  out->generated = generated;
  return 0;
}

}  // extern "C"
