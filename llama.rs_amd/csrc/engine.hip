// engine.hip — host orchestrator of the gfx950 Qwen3 token loop and the C ABI
// declared in include/rlh.h.
//
// Mirrors src/model.rs: a Model (device-resident weights, immutable after
// finalize) and a KvCache (device f32 K/V per layer + workspace + one HIP
// stream). The decode step (Model::forward_one, model.rs:585-738) is captured
// once per cache as a HIP graph whose kernels read the token id and position
// from device memory, so the same graph replays for every position.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/rlh.h"
#include "kernels.h"
#include "attention.h"
#include "matvec.h"
#include "gemm.h"
#include "rlh_format.h"
#include "sampler.h"
#include "sampler_dev.h"

using namespace rlh;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

}  // namespace

int rlh::set_error(int code, const char* msg) { return fail(code, msg); }

namespace {

#define HIPCHK(expr)                                                                              \
  do {                                                                                            \
    hipError_t e_ = (expr);                                                                       \
    if (e_ != hipSuccess) return fail(RLH_EDEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

int block_size(uint32_t ty) {  // quant.rs:44-50
  switch (ty) {
    case RLH_TYPE_F32: case RLH_TYPE_F16: case RLH_TYPE_BF16: return 1;
    case RLH_TYPE_Q4_0: case RLH_TYPE_Q4_1: case RLH_TYPE_Q5_0: case RLH_TYPE_Q5_1: case RLH_TYPE_Q8_0: return 32;
    case RLH_TYPE_Q4_K: case RLH_TYPE_Q5_K: case RLH_TYPE_Q6_K: return 256;
    default: return 0;
  }
}
int type_size(uint32_t ty) {  // quant.rs:53-66
  switch (ty) {
    case RLH_TYPE_F32: return 4;
    case RLH_TYPE_F16: case RLH_TYPE_BF16: return 2;
    case RLH_TYPE_Q4_0: return 18;
    case RLH_TYPE_Q4_1: return 20;
    case RLH_TYPE_Q5_0: return 22;
    case RLH_TYPE_Q5_1: return 24;
    case RLH_TYPE_Q8_0: return 34;
    case RLH_TYPE_Q4_K: return 144;
    case RLH_TYPE_Q5_K: return 176;
    case RLH_TYPE_Q6_K: return 210;
    default: return 0;
  }
}

// Types whose device layout and dequantisation exist (the embedding gather
// and the parity entries); matvec_supported() is the subset with a matvec.
bool layout_supported(uint32_t ty) {
  return is_tiled(ty) || ty == RLH_TYPE_F32 || ty == RLH_TYPE_F16 || ty == RLH_TYPE_BF16;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Largest logits count of rlh_argmax_noalloc (32-bit indices).
constexpr uint64_t kNoAllocMaxN = 0xffffffffull;

// Host-side f16 -> f32 for norm/bias conversion (exact).
float h16(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000) << 16, exp = (h >> 10) & 0x1f, mant = h & 0x3ff, bits;
  if (exp == 0) {
    if (mant == 0) {
      bits = sign;
    } else {
      uint32_t e = 113;
      while (!(mant & 0x400)) {
        mant <<= 1;
        e--;
      }
      bits = sign | (e << 23) | ((mant & 0x3ff) << 13);
    }
  } else if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (mant << 13);
  } else {
    bits = sign | ((exp + 112) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// A weight matrix in device memory (layout: rlh_format.h).
struct DevTensor {
  bool set = false;
  uint32_t ty = 0;
  uint64_t rows = 0, cols = 0;
  uint8_t* mem = nullptr;
  size_t bytes = 0;
  DevMat dm{};
};

struct DevVec {
  float* p = nullptr;
  uint64_t n = 0;
};

struct Layer {
  DevTensor q, k, v, o, gate, up, down;
  DevVec attn_norm, ffn_norm, q_norm, k_norm, bq, bk, bv;
};

// Item bytes (see rlh_format.h) of item j of a ggml row: super-blocks are
// taken as they are; for the 32-value types the quants of 8 blocks come
// first, then their high bits (Q5_0/Q5_1), then their f16 scales (and mins).
void gather_item(uint32_t ty, const uint8_t* row, uint32_t j, uint8_t* item) {
  if (ty == RLH_TYPE_Q4_K || ty == RLH_TYPE_Q5_K || ty == RLH_TYPE_Q6_K) {
    const uint32_t ib = item_bytes(ty);
    std::memcpy(item, row + (size_t)j * ib, ib);
    return;
  }
  if (ty == RLH_TYPE_Q4_1 || ty == RLH_TYPE_Q5_0 || ty == RLH_TYPE_Q5_1) {
    // ggml blocks: Q4_1 (d, m, qs[16]); Q5_0 (d, qh[4], qs[16]); Q5_1 (d, m, qh[4], qs[16])
    const uint32_t bs = (uint32_t)type_size(ty);
    const uint32_t nsc = ty == RLH_TYPE_Q5_0 ? 2 : 4;       // scale bytes per block
    const uint32_t nqh = ty == RLH_TYPE_Q4_1 ? 0 : 4;       // qh bytes per block
    for (uint32_t k = 0; k < 8; k++) {
      const uint8_t* blk = row + ((size_t)j * 8 + k) * bs;
      std::memcpy(item + k * 16, blk + nsc + nqh, 16);                 // quants
      if (nqh) std::memcpy(item + 128 + k * 4, blk + nsc, 4);         // qh
      std::memcpy(item + 128 + 8 * nqh + k * nsc, blk, nsc);          // d (and m)
    }
    return;
  }
  const uint32_t bs = (uint32_t)type_size(ty), qb = bs - 2;  // 34/32 or 18/16
  for (uint32_t k = 0; k < 8; k++) {
    const uint8_t* blk = row + ((size_t)j * 8 + k) * bs;
    std::memcpy(item + k * qb, blk + 2, qb);
    item[8 * qb + 2 * k] = blk[0];
    item[8 * qb + 2 * k + 1] = blk[1];
  }
}

// Fills the DevMat layout fields and returns the device bytes of a rows x
// cols matrix of type ty.
size_t device_layout(DevMat& dm, uint32_t ty, uint64_t rows, uint64_t cols) {
  dm.ty = ty;
  dm.rows = (uint32_t)rows;
  dm.cols = (uint32_t)cols;
  dm.row_bytes = (uint32_t)((size_t)type_size(ty) * (cols / block_size(ty)));
  if (!is_tiled(ty)) {
    dm.tr = dm.tj = dm.ntj = dm.ib = 0;
    return (size_t)rows * dm.row_bytes;
  }
  const uint32_t nitems = (uint32_t)(cols / 256);
  dm.ib = item_bytes(ty);
  dm.tj = tile_width(nitems);
  dm.tr = 64 / dm.tj;
  dm.ntj = nitems / dm.tj;
  const size_t nrt = (rows + dm.tr - 1) / dm.tr;
  return nrt * dm.ntj * 64 * dm.ib;
}

std::vector<uint8_t> to_device_layout(const DevMat& dm, const uint8_t* src, size_t bytes) {
  std::vector<uint8_t> out(bytes, 0);
  if (!is_tiled(dm.ty)) {
    std::memcpy(out.data(), src, bytes);
    return out;
  }
  const uint32_t nitems = dm.cols / 256;
  uint8_t item[272];
  for (uint32_t r = 0; r < dm.rows; r++) {
    const uint8_t* row = src + (size_t)r * dm.row_bytes;
    for (uint32_t j = 0; j < nitems; j++) {
      gather_item(dm.ty, row, j, item);
      const uint32_t ch = dm.ib / 16;
      for (uint32_t k = 0; k < ch; k++) std::memcpy(&out[item_offset(dm, r, j, 16 * k)], item + 16 * k, 16);
      if (dm.ib % 16) std::memcpy(&out[item_offset(dm, r, j, ch * 16)], item + ch * 16, dm.ib % 16);
    }
  }
  return out;
}

int upload_matrix(DevTensor& t, uint32_t ty, const void* bytes, uint64_t cols, uint64_t rows) {
  if (!layout_supported(ty))
    return fail(RLH_EUNSUP, "ggml type " + std::to_string(ty) + " has no device layout on this path");
  if (cols == 0 || rows == 0 || cols % (uint64_t)block_size(ty) != 0)
    return fail(RLH_EINVAL, "row length " + std::to_string(cols) + " is not a multiple of the block size");
  if (is_tiled(ty) && cols % 256 != 0)
    return fail(RLH_EUNSUP, "quantized rows must hold a multiple of 256 values");
  if (rows > 0xffffffffull || cols > 0xffffffffull) return fail(RLH_EINVAL, "matrix too large");
  DevMat dm{};
  const size_t bytes_dev = device_layout(dm, ty, rows, cols);
  std::vector<uint8_t> blob = to_device_layout(dm, (const uint8_t*)bytes, bytes_dev);
  if (t.mem) (void)hipFree(t.mem);
  t.mem = nullptr;
  hipError_t e = hipMalloc((void**)&t.mem, blob.size());
  if (e != hipSuccess) return fail(RLH_ENOMEM, std::string("hipMalloc weights: ") + hipGetErrorString(e));
  HIPCHK(hipMemcpy(t.mem, blob.data(), blob.size(), hipMemcpyHostToDevice));
  t.set = true;
  t.ty = ty;
  t.rows = rows;
  t.cols = cols;
  t.bytes = blob.size();
  t.dm = dm;
  t.dm.a = t.mem;
  return RLH_OK;
}

// Norm / bias vectors: dequantised to f32 on the host (model.rs:156-162).
int upload_vec(DevVec& v, uint32_t ty, const void* bytes, uint64_t n) {
  std::vector<float> f(n);
  const uint8_t* p = (const uint8_t*)bytes;
  if (ty == RLH_TYPE_F32) {
    std::memcpy(f.data(), p, n * 4);
  } else if (ty == RLH_TYPE_F16) {
    for (uint64_t i = 0; i < n; i++) f[i] = h16((uint16_t)(p[2 * i] | (p[2 * i + 1] << 8)));
  } else if (ty == RLH_TYPE_BF16) {
    for (uint64_t i = 0; i < n; i++) {
      uint32_t b = (uint32_t)(p[2 * i] | (p[2 * i + 1] << 8)) << 16;
      std::memcpy(&f[i], &b, 4);
    }
  } else {
    return fail(RLH_EUNSUP, "norm/bias vectors must be F32, F16 or BF16");
  }
  if (v.p) (void)hipFree(v.p);
  v.p = nullptr;
  hipError_t e = hipMalloc((void**)&v.p, n * 4);
  if (e != hipSuccess) return fail(RLH_ENOMEM, "hipMalloc vector");
  HIPCHK(hipMemcpy(v.p, f.data(), n * 4, hipMemcpyHostToDevice));
  v.n = n;
  return RLH_OK;
}

void free_tensor(DevTensor& t) {
  if (t.mem) (void)hipFree(t.mem);
  t = DevTensor();
}
void free_vec(DevVec& v) {
  if (v.p) (void)hipFree(v.p);
  v = DevVec();
}

int ensure_device() {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return fail(RLH_EDEVICE, "no HIP device available (librlh needs an MI355X / gfx950 GPU)");
  static bool lds_set = false;
  if (!lds_set) {
    if (!mv_set_max_lds(150 * 1024)) return fail(RLH_EDEVICE, "matvec LDS attribute");
    lds_set = true;
  }
  return RLH_OK;
}

}  // namespace

struct rlh_model {
  rlh_config cfg{};
  DevTensor token_embd, output;
  DevVec output_norm;
  std::vector<Layer> layers;
  float* rope_cs = nullptr;  // [n_ctx][head_dim]: (cos, sin) of pair i at 2i, 2i+1
  bool finalized = false;
  bool f32_route = false;  // some layer matrix multiplies f32 activations in prefill (Q5_K)
  bool o_quant_ok = false; // attn_output fits the matvec with its quantize prologue
};

struct rlh_cache {
  rlh_model* m = nullptr;
  hipStream_t st = nullptr;
  uint64_t max_ctx = 0, len = 0;
  float* kc = nullptr;  // [L][max_ctx][kvd]
  float* vc = nullptr;
  // workspace for one token
  float *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *g = nullptr, *u = nullptr,
        *logits = nullptr, *scratch = nullptr;
  float* scores = nullptr;  // attention scores [H][max_ctx]
  Q8Buf act_e{}, act_q{}, act_f{};
  // step state (device): tok, pos, step, argmax out
  uint32_t* st_dev = nullptr;  // [0]=tok [1]=pos [2]=step [3]=argmax [4]=wait error flags (kErr*)
  uint32_t* hist = nullptr;    // greedy history [max_ctx + 1]
  float* pv = nullptr;
  uint32_t* pi = nullptr;
  uint32_t nparts = 256;        // partials of the standalone argmax (rlh_greedy_next)
  uint32_t* host_st = nullptr;  // pinned staging for tok/pos
  rlh_dsampler* ds = nullptr;   // device sampler (rlh_sample_next), made on first use
  hipGraphExec_t g_logits = nullptr, g_nologits = nullptr, g_greedy = nullptr;
  // kGreedyBatch greedy steps in one graph (each step reads the token and
  // position its predecessor's argmax left on the device): one graph launch
  // per kGreedyBatch tokens of rlh_generate_greedy
  hipGraphExec_t g_greedy_n = nullptr;
  bool debug = false;
  bool use_graphs = true;  // RLH_GRAPHS=0 launches the same kernels eagerly
  int walk_shift = 0;      // RLH_SOFTMAX_WALK_SHIFT=1|2|3: a test knob of the decode softmax sum (AttnArgs::walk_shift)
  // prefill: the attn_k and attn_v products run on two more streams beside
  // attn_q's (their 1024-row grids fill a quarter of the GPU on their own);
  // side_ok false when RLH_PREFILL_STREAMS=0 or their creation failed (one
  // stream then; what was created is released with the cache)
  hipStream_t side[2] = {nullptr, nullptr};
  bool side_ok = false;
  hipEvent_t ev_fork = nullptr, ev_join[2] = {nullptr, nullptr};
  float* dbg = nullptr;  // [L][kDbgTokens][E]
  uint64_t dbg_tokens = 0;
  bool logits_valid = false;
  // batched prefill workspace (allocated on the first forward_batch): up to
  // kBatch tokens per chunk, token-major
  uint32_t bcap = 0;
  float *xb = nullptr, *qb = nullptr, *kb = nullptr, *vb = nullptr, *attnb = nullptr, *gb = nullptr, *ub = nullptr,
        *scoresb = nullptr, *xnb = nullptr;  // xnb: f32 rmsnorm rows (inputs of f32-route products)
  Q8Buf act_eb{}, act_qb{}, act_fb{};
  uint32_t* tokb = nullptr;   // token ids of the whole call
  uint32_t* posb = nullptr;   // first position of every chunk
  uint64_t tokb_cap = 0, posb_cap = 0;
  // kernel probe (rlh_profile_decode_kernel): event pairs taking the start
  // and end of each eager launch of one weight kind's decode matvec
  int probe_kind = -1;
  std::vector<hipEvent_t> probe_ev;
  uint32_t probe_used = 0;
};

namespace {

constexpr uint64_t kDbgTokens = 64;

float* layer_k(rlh_cache* c, uint32_t l) {
  const rlh_config& cfg = c->m->cfg;
  return c->kc + (size_t)l * c->max_ctx * cfg.n_head_kv * cfg.head_dim;
}
float* layer_v(rlh_cache* c, uint32_t l) {
  const rlh_config& cfg = c->m->cfg;
  return c->vc + (size_t)l * c->max_ctx * cfg.n_head_kv * cfg.head_dim;
}

enum StepKind { STEP_NOLOGITS = 0, STEP_LOGITS = 1, STEP_GREEDY = 2 };

// The cache's device error word: the kernels' bounded intra-block waits set
// a bit here when one expires (kErrMvRing, kErrMvSplit, kErrAttnExp).
uint32_t* err_word(rlh_cache* c) { return c->st_dev + 4; }

// Waits for the cache's stream and reports an expired device wait of any
// kernel enqueued since the last reset. The flags stay set (every later
// step fails too) until rlh_cache_reset: the K/V rows and logits of such a
// step are not the reference's values.
int sync_checked(rlh_cache* c) {
  HIPCHK(hipMemcpyAsync(c->host_st + 4, err_word(c), 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  if (c->host_st[4] != 0) {
    char buf[16];
    std::snprintf(buf, sizeof buf, "0x%08x", c->host_st[4]);
    return fail(RLH_EDEVICE, std::string("a bounded device wait expired (flags ") + buf +
                                 "); the cache holds undefined values until rlh_cache_reset");
  }
  return RLH_OK;
}

// The matvec launch of weight kind `kind` (the kind that names its launch:
// RLH_T_ATTN_Q for q/k/v, RLH_T_FFN_GATE for gate/up, RLH_T_OUTPUT for the
// logits) with the probe's next event pair when a probe of that kind runs.
void mv_launch_probed(rlh_cache* c, int kind, const MvPlan& p) {
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (c->probe_kind == kind && 2 * (c->probe_used + 1) <= c->probe_ev.size()) {
    e0 = c->probe_ev[2 * c->probe_used];
    e1 = c->probe_ev[2 * c->probe_used + 1];
    c->probe_used++;
  }
  mv_launch(c->st, p, err_word(c), e0, e1);
}

// Decode attention writes only f32 (its kernels split the head dimension in
// 16-wide slices) when attn_output can quantize that row in its prologue.
bool attn_f32_out(const rlh_cache* c) { return c->m->o_quant_ok; }

// The attn_output plan of a decode step: its Q8 activation from the f32
// attention output (resident attention) or the attention kernel's Q8 blocks.
void plan_attn_output(MvPlan& p, rlh_cache* c, uint32_t qd) {
  if (attn_f32_out(c)) {
    mv_plan_init_quant(p, qd, c->attn);
  } else {
    mv_plan_init(p, qd, c->act_q);
    mv_plan_set_f32(p, c->attn);
  }
}

// Enqueues one decode step (model.rs:585-738) reading tok = st_dev[0] and
// pos = st_dev[1]. dbg_slot >= 0 copies the residual after each layer.
void enqueue_step(rlh_cache* c, StepKind kind, int64_t dbg_slot) {
  rlh_model* m = c->m;
  const rlh_config& cfg = m->cfg;
  hipStream_t st = c->st;
  const uint32_t E = cfg.n_embd, H = cfg.n_head, KVH = cfg.n_head_kv, hd = cfg.head_dim;
  const float eps = cfg.rms_eps;
  const float scale = 1.0f / std::sqrt((float)hd);  // model.rs:616
  uint32_t* tok = c->st_dev;
  uint32_t* pos = c->st_dev + 1;
  // x = embedding row (model.rs:612); every rmsnorm(x) of the step runs in
  // the prologue of the matvec that consumes it
  launch_embed(st, m->token_embd.dm, tok, 1, c->x);
  const uint32_t qd = H * hd, F = cfg.n_ff;
  for (uint32_t l = 0; l < cfg.n_layer; l++) {
    Layer& L = m->layers[l];
    {  // rmsnorm(x, attn_norm); q, k, v (model.rs:621-624)
      MvPlan p;
      mv_plan_init_norm(p, E, c->x, L.attn_norm.p, eps);
      // attn_v first: its blocks (Q6_K in the Q4_K_M mix: larger items, 16
      // terms per super-block) take longest, so they are dispatched first
      mv_plan_add(p, L.v.dm, c->v, nullptr);
      mv_plan_add(p, L.q.dm, c->q, nullptr);
      mv_plan_add(p, L.k.dm, c->k, nullptr);
      mv_plan_finish(p);
      mv_launch_probed(c, RLH_T_ATTN_Q, p);
    }
    {
      AttnArgs a{};
      a.q = c->q;
      a.k = c->k;
      a.v = c->v;
      a.bq = L.bq.p;
      a.bk = L.bk.p;
      a.bv = L.bv.p;
      a.qn = cfg.has_qk_norm ? L.q_norm.p : nullptr;
      a.kn = cfg.has_qk_norm ? L.k_norm.p : nullptr;
      a.rope_cs = m->rope_cs;
      a.pos0 = pos;
      a.kcache = layer_k(c, l);
      a.vcache = layer_v(c, l);
      a.scores = c->scores;
      a.t_stride = (uint32_t)c->max_ctx;
      a.t_max = (uint32_t)c->max_ctx;
      a.max_ctx = (uint32_t)c->max_ctx;
      a.n_tok = 1;
      a.err = err_word(c);
      a.walk_shift = c->walk_shift;
      a.H = (int)H;
      a.KVH = (int)KVH;
      a.eps = eps;
      a.scale = scale;
      a.out = c->attn;
      a.out_q8 = c->act_q;
      launch_attn_scores(st, a, true);
      launch_attn_decode(st, a, attn_f32_out(c));
    }
    {  // attn_output, x += (model.rs:713-716)
      MvPlan p;
      plan_attn_output(p, c, qd);
      mv_plan_add(p, L.o.dm, nullptr, c->x);
      mv_plan_finish(p);
      mv_launch_probed(c, RLH_T_ATTN_OUTPUT, p);
    }
    if (L.gate.ty == L.up.ty) {  // rmsnorm(x, ffn_norm); gate, up, silu(g)*u and its Q8 blocks (model.rs:719-724)
      MvPlan p;
      mv_plan_init_norm(p, E, c->x, L.ffn_norm.p, eps);
      mv_plan_add_pair(p, L.gate.dm, L.up.dm, c->act_f, c->g);
      mv_plan_finish(p);
      mv_launch_probed(c, RLH_T_FFN_GATE, p);
    } else {  // gate and up of different types: one launch each, then silu(g)*u and its Q8 blocks
      for (int up = 0; up < 2; up++) {
        MvPlan p;
        mv_plan_init_norm(p, E, c->x, L.ffn_norm.p, eps);
        mv_plan_add(p, up ? L.up.dm : L.gate.dm, up ? c->u : c->g, nullptr);
        mv_plan_finish(p);
        mv_launch_probed(c, RLH_T_FFN_GATE, p);
      }
      launch_swiglu_q8(st, c->g, c->u, F, c->act_f, c->g);
    }
    {  // ffn_down, x += (model.rs:725-728)
      MvPlan p;
      mv_plan_init(p, F, c->act_f);
      mv_plan_set_f32(p, c->g);
      mv_plan_add(p, L.down.dm, nullptr, c->x);
      mv_plan_finish(p);
      mv_launch_probed(c, RLH_T_FFN_DOWN, p);
    }
    if (dbg_slot >= 0 && c->dbg && (uint64_t)dbg_slot < c->dbg_tokens)
      (void)hipMemcpyAsync(c->dbg + ((size_t)l * c->dbg_tokens + dbg_slot) * E, c->x, E * 4, hipMemcpyDeviceToDevice,
                           st);
  }
  if (kind == STEP_NOLOGITS) return;
  const DevTensor& ow = m->output.set ? m->output : m->token_embd;
  {  // logits of rmsnorm(x, output_norm) (model.rs:733-737), greedy argmax fused;
     // the norm runs once here rather than in each of the many logits blocks
    launch_rmsnorm_q8(st, c->x, m->output_norm.p, E, 1, eps, c->act_e, c->scratch);
    MvPlan p;
    mv_plan_init(p, E, c->act_e);
    mv_plan_set_f32(p, c->scratch);
    mv_plan_add(p, ow.dm, c->logits, nullptr);
    if (kind == STEP_GREEDY) mv_plan_argmax(p, MvArgmax{c->pv, c->pi});
    mv_plan_finish(p);
    mv_launch_probed(c, RLH_T_OUTPUT, p);
    if (kind == STEP_GREEDY) launch_argmax_final(st, c->pv, c->pi, p.blocks, tok, pos, c->st_dev + 2, c->hist);
  }
}

constexpr uint64_t kGreedyBatch = 8;

int capture(rlh_cache* c, StepKind kind, hipGraphExec_t* out, uint64_t steps = 1) {
  hipGraph_t g = nullptr;
  HIPCHK(hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal));
  for (uint64_t i = 0; i < steps; i++) enqueue_step(c, kind, -1);
  HIPCHK(hipStreamEndCapture(c->st, &g));
  hipError_t e = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return fail(RLH_EDEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
  return RLH_OK;
}

int run_step(rlh_cache* c, StepKind kind, int64_t dbg_slot) {
  if (c->debug || !c->use_graphs) {
    enqueue_step(c, kind, dbg_slot);
    HIPCHK(hipGetLastError());
    return RLH_OK;
  }
  hipGraphExec_t g = kind == STEP_LOGITS ? c->g_logits : (kind == STEP_GREEDY ? c->g_greedy : c->g_nologits);
  HIPCHK(hipGraphLaunch(g, c->st));
  return RLH_OK;
}

int set_tok_pos(rlh_cache* c, uint32_t tok, uint32_t pos) {
  // The previous step may still read the staging words; wait for the stream
  // before overwriting them.
  HIPCHK(hipStreamSynchronize(c->st));
  c->host_st[0] = tok;
  c->host_st[1] = pos;
  HIPCHK(hipMemcpyAsync(c->st_dev, c->host_st, 8, hipMemcpyHostToDevice, c->st));
  return RLH_OK;
}

// Default stream/context for the op-level entries.
hipStream_t op_stream() {
  static hipStream_t s = nullptr;
  if (!s) (void)hipStreamCreate(&s);
  return s;
}

template <typename T>
struct DevBuf {
  T* p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  hipError_t alloc(size_t n) { return hipMalloc((void**)&p, std::max<size_t>(n, 1) * sizeof(T)); }
};

}  // namespace

extern "C" {

const char* rlh_last_error(void) { return g_err.c_str(); }
const char* rlh_version(void) { return "rlh 0.1 (gfx950)"; }

uint64_t rlh_row_bytes(uint32_t ty, uint64_t cols) {
  int bs = block_size(ty);
  if (bs == 0 || cols % (uint64_t)bs != 0) return 0;
  return (uint64_t)type_size(ty) * (cols / (uint64_t)bs);
}

int rlh_config_check(const rlh_config* cfg) {
  if (!cfg) return fail(RLH_EINVAL, "null argument");
  if (cfg->n_layer == 0 || cfg->n_embd == 0 || cfg->n_head == 0 || cfg->n_head_kv == 0 || cfg->n_ff == 0 ||
      cfg->vocab_size == 0)
    return fail(RLH_EINVAL, "config has a zero dimension");
  if (cfg->n_head % cfg->n_head_kv != 0) return fail(RLH_EINVAL, "n_head must be a multiple of n_head_kv");
  // Shapes the reference runs (model.rs:249-268 reads any head_dim; rows of
  // any whole number of blocks, tensor.rs:28-30) that this path refuses up
  // front, before any tensor is read or uploaded:
  if (cfg->head_dim != 128)
    return fail(RLH_EUNSUP, "head_dim " + std::to_string(cfg->head_dim) +
                                ": the attention kernels are built for 128-value heads (one K/V row per lane pair "
                                "of 64, the NeoX RoPE table of 64 pairs), as Qwen3 and Qwen2.5 from 1.5B up use; "
                                "Qwen2.5-0.5B-shaped models (head_dim 64) are not supported on this path");
  if (cfg->n_embd % 256 != 0 || cfg->n_ff % 256 != 0)
    return fail(RLH_EUNSUP, "n_embd " + std::to_string(cfg->n_embd) + " / n_ff " + std::to_string(cfg->n_ff) +
                                ": the device weight layout tiles rows in 256-value items, so n_embd and n_ff "
                                "must be multiples of 256");
  if (cfg->n_head / cfg->n_head_kv > (uint32_t)kAttnMaxGroup)
    return fail(RLH_EUNSUP, "more than 8 query heads per KV head");
  return RLH_OK;
}

int rlh_model_create(const rlh_config* cfg, rlh_model** out) {
  if (!cfg || !out) return fail(RLH_EINVAL, "null argument");
  *out = nullptr;
  int rc = rlh_config_check(cfg);
  if (rc) return rc;
  if ((rc = ensure_device())) return rc;
  rlh_model* m = new rlh_model();
  m->cfg = *cfg;
  m->layers.resize(cfg->n_layer);
  *out = m;
  return RLH_OK;
}

int rlh_model_set_tensor(rlh_model* m, int kind, int layer, uint32_t ty, const void* bytes, uint64_t n_cols,
                         uint64_t n_rows) {
  if (!m || !bytes) return fail(RLH_EINVAL, "null argument");
  if (m->finalized) return fail(RLH_ESTATE, "model is finalized");
  if (block_size(ty) == 0) return fail(RLH_EINVAL, "unknown ggml type " + std::to_string(ty));
  Layer* L = nullptr;
  if (kind >= RLH_T_ATTN_NORM) {
    if (layer < 0 || (uint32_t)layer >= m->cfg.n_layer) return fail(RLH_EINVAL, "layer out of range");
    L = &m->layers[layer];
  }
  uint64_t n = n_cols * n_rows;
  switch (kind) {
    case RLH_T_TOKEN_EMBD: return upload_matrix(m->token_embd, ty, bytes, n_cols, n_rows);
    case RLH_T_OUTPUT_NORM: return upload_vec(m->output_norm, ty, bytes, n);
    case RLH_T_OUTPUT: return upload_matrix(m->output, ty, bytes, n_cols, n_rows);
    case RLH_T_ATTN_NORM: return upload_vec(L->attn_norm, ty, bytes, n);
    case RLH_T_ATTN_Q: return upload_matrix(L->q, ty, bytes, n_cols, n_rows);
    case RLH_T_ATTN_K: return upload_matrix(L->k, ty, bytes, n_cols, n_rows);
    case RLH_T_ATTN_V: return upload_matrix(L->v, ty, bytes, n_cols, n_rows);
    case RLH_T_ATTN_OUTPUT: return upload_matrix(L->o, ty, bytes, n_cols, n_rows);
    case RLH_T_ATTN_Q_NORM: return upload_vec(L->q_norm, ty, bytes, n);
    case RLH_T_ATTN_K_NORM: return upload_vec(L->k_norm, ty, bytes, n);
    case RLH_T_FFN_NORM: return upload_vec(L->ffn_norm, ty, bytes, n);
    case RLH_T_FFN_GATE: return upload_matrix(L->gate, ty, bytes, n_cols, n_rows);
    case RLH_T_FFN_UP: return upload_matrix(L->up, ty, bytes, n_cols, n_rows);
    case RLH_T_FFN_DOWN: return upload_matrix(L->down, ty, bytes, n_cols, n_rows);
    case RLH_T_ATTN_Q_BIAS: return upload_vec(L->bq, ty, bytes, n);
    case RLH_T_ATTN_K_BIAS: return upload_vec(L->bk, ty, bytes, n);
    case RLH_T_ATTN_V_BIAS: return upload_vec(L->bv, ty, bytes, n);
    default: return fail(RLH_EINVAL, "unknown tensor kind " + std::to_string(kind));
  }
}

static int check_matrix(const DevTensor& t, const char* name, int layer, uint64_t rows, uint64_t cols) {
  std::string nm = layer >= 0 ? "blk." + std::to_string(layer) + "." + name : std::string(name);
  if (!t.set) return fail(RLH_ESTATE, "model is missing required tensor '" + nm + ".weight'");
  if (t.rows != rows || t.cols != cols)
    return fail(RLH_EINVAL, "tensor '" + nm + "' has shape " + std::to_string(t.rows) + "x" + std::to_string(t.cols) +
                                ", expected " + std::to_string(rows) + "x" + std::to_string(cols));
  if (!matvec_supported(t.ty) || (layer >= 0 && !gemm_supported(t.ty) && !gemm_f32_supported(t.ty)))
    return fail(RLH_EUNSUP, "tensor '" + nm + "' has ggml type " + std::to_string(t.ty) + " with no kernel");
  return RLH_OK;
}
static int check_vec(const DevVec& v, const char* name, int layer, uint64_t n, bool required) {
  std::string nm = layer >= 0 ? "blk." + std::to_string(layer) + "." + name : std::string(name);
  if (!v.p) return required ? fail(RLH_ESTATE, "model is missing required tensor '" + nm + "'") : RLH_OK;
  if (v.n != n) return fail(RLH_EINVAL, "tensor '" + nm + "' has " + std::to_string(v.n) + " elements");
  return RLH_OK;
}

int rlh_model_finalize(rlh_model* m) {
  if (!m) return fail(RLH_EINVAL, "null model");
  if (m->finalized) return RLH_OK;
  const rlh_config& c = m->cfg;
  uint64_t E = c.n_embd, F = c.n_ff, qd = (uint64_t)c.n_head * c.head_dim, kvd = (uint64_t)c.n_head_kv * c.head_dim;
  if (!m->token_embd.set) return fail(RLH_ESTATE, "model is missing required tensor 'token_embd.weight'");
  if (m->token_embd.cols != E || m->token_embd.rows != c.vocab_size)
    return fail(RLH_EINVAL, "token_embd shape does not match n_embd x vocab_size");
  int rc;
  if ((rc = check_vec(m->output_norm, "output_norm.weight", -1, E, true))) return rc;
  if (m->output.set) {
    if ((rc = check_matrix(m->output, "output", -1, c.vocab_size, E))) return rc;
  } else if (!matvec_supported(m->token_embd.ty)) {
    return fail(RLH_EUNSUP, "tied token_embd type has no matvec kernel for the logits");
  }
  for (uint32_t l = 0; l < c.n_layer; l++) {
    Layer& L = m->layers[l];
    int li = (int)l;
    if ((rc = check_vec(L.attn_norm, "attn_norm.weight", li, E, true))) return rc;
    if ((rc = check_vec(L.ffn_norm, "ffn_norm.weight", li, E, true))) return rc;
    if ((rc = check_matrix(L.q, "attn_q", li, qd, E))) return rc;
    if ((rc = check_matrix(L.k, "attn_k", li, kvd, E))) return rc;
    if ((rc = check_matrix(L.v, "attn_v", li, kvd, E))) return rc;
    if ((rc = check_matrix(L.o, "attn_output", li, E, qd))) return rc;
    if ((rc = check_matrix(L.gate, "ffn_gate", li, F, E))) return rc;
    if ((rc = check_matrix(L.up, "ffn_up", li, F, E))) return rc;
    if ((rc = check_matrix(L.down, "ffn_down", li, E, F))) return rc;
    if ((rc = check_vec(L.q_norm, "attn_q_norm.weight", li, c.head_dim, c.has_qk_norm != 0))) return rc;
    if ((rc = check_vec(L.k_norm, "attn_k_norm.weight", li, c.head_dim, c.has_qk_norm != 0))) return rc;
    if ((rc = check_vec(L.bq, "attn_q.bias", li, qd, false))) return rc;
    if ((rc = check_vec(L.bk, "attn_k.bias", li, kvd, false))) return rc;
    if ((rc = check_vec(L.bv, "attn_v.bias", li, kvd, false))) return rc;
  }
  m->f32_route = false;
  for (const Layer& L : m->layers)
    for (const DevTensor* t : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down})
      if (!gemm_supported(t->ty)) m->f32_route = true;
  // every decode matvec launch must fit the kernel's LDS budget
  for (uint32_t l = 0; l < c.n_layer; l++) {
    Layer& L = m->layers[l];
    const Q8Mut none{};
    static const float kShapeOnly = 0.0f;  // plans below are built for their shape only
    MvPlan p;
    mv_plan_init_norm(p, (uint32_t)E, nullptr, nullptr, 0.0f);
    mv_plan_add(p, L.q.dm, nullptr, nullptr);
    mv_plan_add(p, L.k.dm, nullptr, nullptr);
    mv_plan_add(p, L.v.dm, nullptr, nullptr);
    bool ok = mv_plan_finish(p);
    mv_plan_init(p, (uint32_t)qd, none);
    mv_plan_set_f32(p, &kShapeOnly);
    mv_plan_add(p, L.o.dm, nullptr, nullptr);
    ok = ok && mv_plan_finish(p);
    if (L.gate.ty == L.up.ty) {
      mv_plan_init_norm(p, (uint32_t)E, nullptr, nullptr, 0.0f);
      mv_plan_add_pair(p, L.gate.dm, L.up.dm, none, nullptr);
      ok = ok && mv_plan_finish(p);
    } else {  // separate launches (the decode step's fallback)
      for (const DevTensor* t : {&L.gate, &L.up}) {
        mv_plan_init_norm(p, (uint32_t)E, nullptr, nullptr, 0.0f);
        mv_plan_add(p, t->dm, nullptr, nullptr);
        ok = ok && mv_plan_finish(p);
      }
    }
    mv_plan_init(p, (uint32_t)F, none);
    mv_plan_set_f32(p, &kShapeOnly);
    mv_plan_add(p, L.down.dm, nullptr, nullptr);
    ok = ok && mv_plan_finish(p);
    if (l == 0) m->o_quant_ok = true;
    if (qd <= kMvMaxQuantCols) {  // the attn_output launch after the f32-output attention kernels
      mv_plan_init_quant(p, (uint32_t)qd, &kShapeOnly);
      mv_plan_add(p, L.o.dm, nullptr, nullptr);
      m->o_quant_ok = m->o_quant_ok && mv_plan_finish(p);
    } else {
      m->o_quant_ok = false;
    }
    if (!ok) return fail(RLH_EUNSUP, "blk." + std::to_string(l) + ": matrix shapes or types are not supported by the matvec");
  }
  {
    const DevTensor& ow = m->output.set ? m->output : m->token_embd;
    static const float kShapeOnly = 0.0f;  // built for its shape only
    MvPlan p;
    mv_plan_init(p, (uint32_t)E, Q8Mut{});
    mv_plan_set_f32(p, &kShapeOnly);
    mv_plan_add(p, ow.dm, nullptr, nullptr);
    if (!mv_plan_finish(p)) return fail(RLH_EUNSUP, "logits matrix shape or type is not supported by the matvec");
  }
  // RoPE table with the host libm, as the reference computes it:
  // inv_freq = theta^(-2i/hd) (model.rs:221-227), angle = pos * inv_freq,
  // (sin, cos) = f32::sin_cos (ops.rs:439).
  uint32_t half = c.head_dim / 2;
  std::vector<float> inv(half);
  for (uint32_t i = 0; i < half; i++) {
    float e = -2.0f * (float)i / (float)c.head_dim;
    inv[i] = std::pow(c.rope_theta, e);
  }
  uint64_t nctx = std::max<uint32_t>(c.n_ctx, 1);
  std::vector<float> cs((size_t)nctx * c.head_dim);
  for (uint64_t p = 0; p < nctx; p++) {
    float pf = (float)p;
    for (uint32_t i = 0; i < half; i++) {
      float a = pf * inv[i];
      cs[p * c.head_dim + 2 * i] = std::cos(a);
      cs[p * c.head_dim + 2 * i + 1] = std::sin(a);
    }
  }
  hipError_t e = hipMalloc((void**)&m->rope_cs, cs.size() * 4);
  if (e != hipSuccess) return fail(RLH_ENOMEM, "hipMalloc rope table");
  HIPCHK(hipMemcpy(m->rope_cs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  m->finalized = true;
  return RLH_OK;
}

void rlh_model_destroy(rlh_model* m) {
  if (!m) return;
  free_tensor(m->token_embd);
  free_tensor(m->output);
  free_vec(m->output_norm);
  for (auto& L : m->layers) {
    free_tensor(L.q); free_tensor(L.k); free_tensor(L.v); free_tensor(L.o);
    free_tensor(L.gate); free_tensor(L.up); free_tensor(L.down);
    free_vec(L.attn_norm); free_vec(L.ffn_norm); free_vec(L.q_norm); free_vec(L.k_norm);
    free_vec(L.bq); free_vec(L.bk); free_vec(L.bv);
  }
  if (m->rope_cs) (void)hipFree(m->rope_cs);
  delete m;
}

uint64_t rlh_model_weight_bytes(const rlh_model* m) {
  if (!m) return 0;
  uint64_t s = m->token_embd.bytes + m->output.bytes;
  for (auto& L : m->layers) s += L.q.bytes + L.k.bytes + L.v.bytes + L.o.bytes + L.gate.bytes + L.up.bytes + L.down.bytes;
  return s;
}

static void cache_free(rlh_cache* c) {
  if (c->g_logits) (void)hipGraphExecDestroy(c->g_logits);
  if (c->g_nologits) (void)hipGraphExecDestroy(c->g_nologits);
  if (c->g_greedy) (void)hipGraphExecDestroy(c->g_greedy);
  if (c->g_greedy_n) (void)hipGraphExecDestroy(c->g_greedy_n);
  void* ptrs[] = {c->kc, c->vc, c->scores, c->x, c->q, c->k, c->v, c->attn, c->g, c->u, c->logits, c->scratch,
                  c->act_e.qs, c->act_e.d, c->act_e.s, c->act_e.s16, c->act_q.qs, c->act_q.d, c->act_q.s,
                  c->act_q.s16, c->act_f.qs, c->act_f.d, c->act_f.s, c->act_f.s16, c->st_dev, c->hist, c->pv,
                  c->pi, c->dbg};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  void* bptrs[] = {c->xb, c->qb, c->kb, c->vb, c->attnb, c->gb, c->ub, c->scoresb, c->xnb, c->act_eb.qs, c->act_eb.d,
                   c->act_eb.s, c->act_eb.s16, c->act_qb.qs, c->act_qb.d, c->act_qb.s, c->act_qb.s16, c->act_fb.qs,
                   c->act_fb.d, c->act_fb.s, c->act_fb.s16, c->tokb, c->posb};
  for (void* p : bptrs)
    if (p) (void)hipFree(p);
  if (c->host_st) (void)hipHostFree(c->host_st);
  if (c->ds) rlh_dsampler_destroy(c->ds);
  for (int i = 0; i < 2; i++) {
    if (c->side[i]) (void)hipStreamDestroy(c->side[i]);
    if (c->ev_join[i]) (void)hipEventDestroy(c->ev_join[i]);
  }
  if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
  if (c->st) (void)hipStreamDestroy(c->st);
  delete c;
}

static int alloc_q8(Q8Buf& b, uint64_t n) {
  if (hipMalloc((void**)&b.qs, n) != hipSuccess || hipMalloc((void**)&b.d, n / 32 * 4) != hipSuccess ||
      hipMalloc((void**)&b.s, n / 32 * 4) != hipSuccess || hipMalloc((void**)&b.s16, n / 16 * 4) != hipSuccess)
    return fail(RLH_ENOMEM, "hipMalloc Q8 activation");
  return RLH_OK;
}

int rlh_cache_create(rlh_model* m, uint64_t max_ctx, rlh_cache** out) {
  if (!m || !out) return fail(RLH_EINVAL, "null argument");
  *out = nullptr;
  if (!m->finalized) return fail(RLH_ESTATE, "model is not finalized");
  const rlh_config& cfg = m->cfg;
  max_ctx = std::min<uint64_t>(max_ctx, cfg.n_ctx);  // model.rs:340
  if (max_ctx == 0) return fail(RLH_EINVAL, "max_ctx is 0");
  if (max_ctx > kAttnMaxCtx) return fail(RLH_EUNSUP, "max_ctx above 32768 is not supported by the attention kernels");
  if (cfg.n_head / cfg.n_head_kv > (uint32_t)kAttnMaxGroup) return fail(RLH_EUNSUP, "more than 8 query heads per KV head");
  if (!attn_init((uint32_t)max_ctx)) return fail(RLH_EDEVICE, "attention LDS attribute");
  rlh_cache* c = new rlh_cache();
  c->m = m;
  c->max_ctx = max_ctx;
  const DevTensor& ow = m->output.set ? m->output : m->token_embd;
  const uint32_t npv = std::max(c->nparts, mv_blocks_for(ow.ty, cfg.vocab_size, cfg.n_embd));
  uint64_t E = cfg.n_embd, F = cfg.n_ff, qd = (uint64_t)cfg.n_head * cfg.head_dim,
           kvd = (uint64_t)cfg.n_head_kv * cfg.head_dim;
  size_t kvbytes = (size_t)cfg.n_layer * max_ctx * kvd * 4;
  // scratch holds the f32 rmsnorm row of the logits launch (E floats) and
  // vocabulary- or F-sized temporaries: E can exceed both (a small or pruned
  // vocabulary)
  const size_t scratch_bytes = (size_t)std::max<uint64_t>(std::max<uint64_t>(cfg.vocab_size, F), E) * 4;
  bool ok = hipStreamCreate(&c->st) == hipSuccess && hipMalloc((void**)&c->kc, kvbytes) == hipSuccess &&
            hipMalloc((void**)&c->scores, (size_t)cfg.n_head * max_ctx * 4) == hipSuccess &&
            hipMalloc((void**)&c->vc, kvbytes) == hipSuccess && hipMalloc((void**)&c->x, E * 4) == hipSuccess &&
            hipMalloc((void**)&c->q, qd * 4) == hipSuccess && hipMalloc((void**)&c->k, kvd * 4) == hipSuccess &&
            hipMalloc((void**)&c->v, kvd * 4) == hipSuccess && hipMalloc((void**)&c->attn, qd * 4) == hipSuccess &&
            hipMalloc((void**)&c->g, F * 4) == hipSuccess && hipMalloc((void**)&c->u, F * 4) == hipSuccess &&
            hipMalloc((void**)&c->logits, (size_t)cfg.vocab_size * 4) == hipSuccess &&
            hipMalloc((void**)&c->scratch, scratch_bytes) == hipSuccess &&
            hipMalloc((void**)&c->st_dev, 64) == hipSuccess &&
            hipMalloc((void**)&c->hist, (max_ctx + 2) * 4) == hipSuccess &&
            hipMalloc((void**)&c->pv, (size_t)npv * 4) == hipSuccess &&
            hipMalloc((void**)&c->pi, (size_t)npv * 4) == hipSuccess &&
            hipHostMalloc((void**)&c->host_st, 64) == hipSuccess;
  if (!ok) {
    cache_free(c);
    return fail(RLH_ENOMEM, "cache allocation failed");
  }
  int rc = alloc_q8(c->act_e, E);
  if (!rc) rc = alloc_q8(c->act_q, qd);
  if (!rc) rc = alloc_q8(c->act_f, F);
  if (rc) {
    cache_free(c);
    return rc;
  }
  if (hipMemset(c->st_dev, 0, 64) != hipSuccess || hipMemset(c->kc, 0, kvbytes) != hipSuccess ||
      hipMemset(c->vc, 0, kvbytes) != hipSuccess || hipMemset(c->scratch, 0, scratch_bytes) != hipSuccess ||
      hipMemset(c->act_e.qs, 0, E) != hipSuccess || hipMemset(c->act_e.d, 0, E / 32 * 4) != hipSuccess ||
      hipMemset(c->act_e.s, 0, E / 32 * 4) != hipSuccess || hipMemset(c->act_e.s16, 0, E / 16 * 4) != hipSuccess) {
    cache_free(c);
    return fail(RLH_EDEVICE, "cache init");
  }
  const char* env = std::getenv("RLH_GRAPHS");
  c->use_graphs = !(env && std::strcmp(env, "0") == 0);
  const char* senv = std::getenv("RLH_PREFILL_STREAMS");
  if (!(senv && std::strcmp(senv, "0") == 0)) {
    bool sok = hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming) == hipSuccess;
    for (int i = 0; i < 2 && sok; i++)
      sok = hipStreamCreate(&c->side[i]) == hipSuccess &&
            hipEventCreateWithFlags(&c->ev_join[i], hipEventDisableTiming) == hipSuccess;
    c->side_ok = sok;
    if (!sok) (void)hipGetLastError();
  }
  const char* wenv = std::getenv("RLH_SOFTMAX_WALK_SHIFT");
  if (wenv && wenv[0] >= '1' && wenv[0] <= '3' && wenv[1] == 0) c->walk_shift = wenv[0] - '0';
  if (c->use_graphs &&
      ((rc = capture(c, STEP_LOGITS, &c->g_logits)) || (rc = capture(c, STEP_NOLOGITS, &c->g_nologits)) ||
       (rc = capture(c, STEP_GREEDY, &c->g_greedy)) ||
       (rc = capture(c, STEP_GREEDY, &c->g_greedy_n, kGreedyBatch)))) {
    std::string msg = g_err;
    cache_free(c);
    return fail(rc, msg);
  }
  *out = c;
  return RLH_OK;
}

int rlh_cache_reset(rlh_cache* c) {
  if (!c) return fail(RLH_EINVAL, "null cache");
  HIPCHK(hipStreamSynchronize(c->st));
  c->host_st[4] = 0;  // clear the wait error flags
  HIPCHK(hipMemcpyAsync(err_word(c), c->host_st + 4, 4, hipMemcpyHostToDevice, c->st));
  c->len = 0;
  c->logits_valid = false;
  return RLH_OK;
}
uint64_t rlh_cache_len(const rlh_cache* c) { return c ? c->len : 0; }
uint64_t rlh_cache_max_ctx(const rlh_cache* c) { return c ? c->max_ctx : 0; }
void rlh_cache_destroy(rlh_cache* c) {
  if (!c) return;
  (void)hipStreamSynchronize(c->st);
  cache_free(c);
}

int rlh_cache_set_debug(rlh_cache* c, int enable) {
  if (!c) return fail(RLH_EINVAL, "null cache");
  c->debug = enable != 0;
  if (c->debug && !c->dbg) {
    size_t n = (size_t)c->m->cfg.n_layer * kDbgTokens * c->m->cfg.n_embd;
    if (hipMalloc((void**)&c->dbg, n * 4) != hipSuccess) return fail(RLH_ENOMEM, "hipMalloc debug buffer");
    c->dbg_tokens = kDbgTokens;
  }
  return RLH_OK;
}

static int check_forward_args(rlh_model* m, rlh_cache* c) {
  if (!m || !c) return fail(RLH_EINVAL, "null argument");
  if (c->m != m) return fail(RLH_EINVAL, "cache belongs to another model");
  return RLH_OK;
}

static int copy_logits(rlh_cache* c, float* logits) {
  if (logits)
    HIPCHK(hipMemcpyAsync(logits, c->logits, (size_t)c->m->cfg.vocab_size * 4, hipMemcpyDeviceToHost, c->st));
  return sync_checked(c);
}

int rlh_forward_one(rlh_model* m, rlh_cache* c, uint32_t token, uint64_t pos, float* logits) {
  int rc = check_forward_args(m, c);
  if (rc) return rc;
  if (token >= m->cfg.vocab_size) return fail(RLH_EINVAL, "token id out of range");
  if (pos >= c->max_ctx) return fail(RLH_ECTX, "position " + std::to_string(pos) + " >= max_ctx");
  if ((rc = set_tok_pos(c, token, (uint32_t)pos))) return rc;
  if ((rc = run_step(c, STEP_LOGITS, 0))) return rc;
  c->len = pos + 1;
  c->logits_valid = true;
  return copy_logits(c, logits);
}

// Tokens per prefill chunk: the batched workspace holds this many rows.
static constexpr uint32_t kBatch = 512;

static int ensure_batch(rlh_cache* c) {
  if (c->bcap) return RLH_OK;
  const rlh_config& cfg = c->m->cfg;
  const uint32_t B = (uint32_t)std::min<uint64_t>(kBatch, c->max_ctx);
  const size_t E = cfg.n_embd, F = cfg.n_ff, qd = (size_t)cfg.n_head * cfg.head_dim,
               kvd = (size_t)cfg.n_head_kv * cfg.head_dim;
  bool ok = hipMalloc((void**)&c->xb, B * E * 4) == hipSuccess && hipMalloc((void**)&c->qb, B * qd * 4) == hipSuccess &&
            hipMalloc((void**)&c->kb, B * kvd * 4) == hipSuccess && hipMalloc((void**)&c->vb, B * kvd * 4) == hipSuccess &&
            hipMalloc((void**)&c->attnb, B * qd * 4) == hipSuccess && hipMalloc((void**)&c->gb, B * F * 4) == hipSuccess &&
            hipMalloc((void**)&c->ub, B * F * 4) == hipSuccess && hipMalloc((void**)&c->xnb, B * E * 4) == hipSuccess &&
            hipMalloc((void**)&c->scoresb, (size_t)B * cfg.n_head * c->max_ctx * 4) == hipSuccess;
  if (!ok) return fail(RLH_ENOMEM, "prefill workspace allocation failed");
  int rc = alloc_q8(c->act_eb, B * E);
  if (!rc) rc = alloc_q8(c->act_qb, B * qd);
  if (!rc) rc = alloc_q8(c->act_fb, B * F);
  if (rc) return rc;
  c->bcap = B;
  return RLH_OK;
}

// Model::forward_batch (model.rs:384-583) with the integer batch products of
// RUST_LLAMA_BATCH_INT=1: the prompt runs through every layer in chunks of
// up to kBatch tokens (a chunk's attention reads the K/V rows the earlier
// chunks wrote, so chunking changes no value). Per layer: rmsnorm + Q8 of
// every token, q/k/v products, QK-norm + RoPE + K/V write, causal attention
// (query rows in parallel), attn_output product added to the residual,
// rmsnorm + Q8, gate/up products, SwiGLU + Q8, ffn_down product added to the
// residual. Logits for the last token only (model.rs:578-582).
static int forward_batch_impl(rlh_model* m, rlh_cache* c, const uint32_t* tokens, uint64_t n, uint64_t start_pos) {
  int rc = ensure_batch(c);
  if (rc) return rc;
  const rlh_config& cfg = m->cfg;
  hipStream_t st = c->st;
  const uint32_t E = cfg.n_embd, H = cfg.n_head, KVH = cfg.n_head_kv, hd = cfg.head_dim;
  const float eps = cfg.rms_eps, scale = 1.0f / std::sqrt((float)hd);
  const uint32_t B = c->bcap;
  const uint64_t nchunks = (n + B - 1) / B;
  HIPCHK(hipStreamSynchronize(st));
  if (n > c->tokb_cap) {
    if (c->tokb) (void)hipFree(c->tokb);
    c->tokb = nullptr;
    if (hipMalloc((void**)&c->tokb, n * 4) != hipSuccess) return fail(RLH_ENOMEM, "hipMalloc prompt ids");
    c->tokb_cap = n;
  }
  if (nchunks > c->posb_cap) {
    if (c->posb) (void)hipFree(c->posb);
    c->posb = nullptr;
    if (hipMalloc((void**)&c->posb, nchunks * 4) != hipSuccess) return fail(RLH_ENOMEM, "hipMalloc chunk positions");
    c->posb_cap = nchunks;
  }
  std::vector<uint32_t> p0s(nchunks);
  for (uint64_t i = 0; i < nchunks; i++) p0s[i] = (uint32_t)(start_pos + i * B);
  HIPCHK(hipMemcpy(c->tokb, tokens, n * 4, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(c->posb, p0s.data(), nchunks * 4, hipMemcpyHostToDevice));
  uint32_t last_m = 0;
  for (uint64_t ci = 0; ci < nchunks; ci++) {
    const uint64_t c0 = ci * B;
    const uint32_t mtok = (uint32_t)std::min<uint64_t>(B, n - c0);
    const uint32_t p0 = p0s[ci];
    const uint32_t* pos = c->posb + ci;
    last_m = mtok;
    // tokens of this chunk that are in the call's groups of 4 (f32-route
    // products give the last n % 4 tokens of the call the single-token order)
    const uint64_t n4_all = n - n % 4;
    const uint32_t n4 = (uint32_t)std::min<uint64_t>(mtok, n4_all > c0 ? n4_all - c0 : 0);
    auto product_on = [&](hipStream_t s, const DevMat& w, const Q8Buf& q8, const float* xf, float* y,
                          float* resid) {
      if (gemm_supported(w.ty))
        launch_gemm(s, w, q8, mtok, y, resid);
      else
        launch_gemm_f32(s, w, xf, mtok, n4, y, resid);
    };
    auto product = [&](const DevMat& w, const Q8Buf& q8, const float* xf, float* y, float* resid) {
      product_on(st, w, q8, xf, y, resid);
    };
    float* xn = m->f32_route ? c->xnb : nullptr;  // f32 rmsnorm rows, when a product needs them
    launch_embed(st, m->token_embd.dm, c->tokb + c0, mtok, c->xb);
    for (uint32_t l = 0; l < cfg.n_layer; l++) {
      Layer& L = m->layers[l];
      launch_rmsnorm_q8(st, c->xb, L.attn_norm.p, E, mtok, eps, c->act_eb, xn);
      // Without a v bias the v product writes the chunk's V cache rows
      // itself ([position][KVH * hd], the product's own [token][rows]
      // layout from row p0), and nothing reads them before the PV kernel.
      const bool v_direct = L.bv.p == nullptr;
      float* vdst = v_direct ? layer_v(c, l) + (size_t)p0 * KVH * hd : c->vb;
      bool v_pending = false;  // the main stream has yet to wait for the v stream
      // q and k of one type and width: one launch of both (no stream join
      // for k on the way to the next kernel)
      const bool qk_pair = gemm_pair_supported(L.q.dm, L.k.dm);
      auto q_and_k = [&](hipStream_t s) {
        if (qk_pair) {
          launch_gemm_pair(s, L.q.dm, L.k.dm, c->act_eb, mtok, c->qb, c->kb);
        } else {
          product_on(s, L.q.dm, c->act_eb, xn, c->qb, nullptr);
          product_on(s, L.k.dm, c->act_eb, xn, c->kb, nullptr);
        }
      };
      if (c->side_ok) {
        // v (and k, when q and k cannot share a launch) beside q: the side
        // streams start after the norm; the main stream waits for k before
        // the next kernel reads it, and for v there too when v goes
        // through vb, else just before the PV kernel (nothing writes the
        // norm's outputs before either join)
        HIPCHK(hipEventRecord(c->ev_fork, st));
        HIPCHK(hipStreamWaitEvent(c->side[1], c->ev_fork, 0));
        if (!qk_pair) {
          HIPCHK(hipStreamWaitEvent(c->side[0], c->ev_fork, 0));
          product_on(c->side[0], L.k.dm, c->act_eb, xn, c->kb, nullptr);
          HIPCHK(hipEventRecord(c->ev_join[0], c->side[0]));
        }
        product_on(c->side[1], L.v.dm, c->act_eb, xn, vdst, nullptr);
        HIPCHK(hipEventRecord(c->ev_join[1], c->side[1]));
        if (qk_pair)
          q_and_k(st);
        else
          product(L.q.dm, c->act_eb, xn, c->qb, nullptr);
        if (!qk_pair) HIPCHK(hipStreamWaitEvent(st, c->ev_join[0], 0));
        if (v_direct)
          v_pending = true;
        else
          HIPCHK(hipStreamWaitEvent(st, c->ev_join[1], 0));
      } else {
        q_and_k(st);
        product(L.v.dm, c->act_eb, xn, vdst, nullptr);
      }
      launch_qk_norm_rope_kv(st, c->qb, c->kb, v_direct ? nullptr : c->vb, L.bq.p, L.bk.p, L.bv.p,
                             cfg.has_qk_norm ? L.q_norm.p : nullptr, cfg.has_qk_norm ? L.k_norm.p : nullptr,
                             m->rope_cs, pos, layer_k(c, l), layer_v(c, l), (int)H, (int)KVH, mtok, eps);
      AttnArgs a{};
      a.q = c->qb;
      a.rope_cs = m->rope_cs;
      a.pos0 = pos;
      a.kcache = layer_k(c, l);
      a.vcache = layer_v(c, l);
      a.scores = c->scoresb;
      a.t_stride = (uint32_t)c->max_ctx;
      a.t_max = p0 + mtok;
      a.max_ctx = (uint32_t)c->max_ctx;
      a.n_tok = mtok;
      a.H = (int)H;
      a.KVH = (int)KVH;
      a.eps = eps;
      a.scale = scale;
      a.out = c->attnb;
      a.out_q8 = c->act_qb;
      a.err = err_word(c);
      launch_attn_scores(st, a, false);
      launch_attn_softmax(st, a);
      if (v_pending) HIPCHK(hipStreamWaitEvent(st, c->ev_join[1], 0));
      launch_attn_pv(st, a, false);
      product(L.o.dm, c->act_qb, c->attnb, nullptr, c->xb);
      launch_rmsnorm_q8(st, c->xb, L.ffn_norm.p, E, mtok, eps, c->act_eb, xn);
      if (gemm_pair_supported(L.gate.dm, L.up.dm)) {  // one launch of both (one boundary less)
        launch_gemm_pair(st, L.gate.dm, L.up.dm, c->act_eb, mtok, c->gb, c->ub);
      } else {
        product(L.gate.dm, c->act_eb, xn, c->gb, nullptr);
        product(L.up.dm, c->act_eb, xn, c->ub, nullptr);
      }
      // h over the gate rows in place when ffn_down takes the f32 route
      const bool hf = !gemm_supported(L.down.ty);
      launch_swiglu_q8(st, c->gb, c->ub, mtok * cfg.n_ff, c->act_fb, hf ? c->gb : nullptr);
      product(L.down.dm, c->act_fb, c->gb, nullptr, c->xb);
      if (c->debug && c->dbg && c0 < c->dbg_tokens) {
        const uint64_t nd = std::min<uint64_t>(mtok, c->dbg_tokens - c0);
        HIPCHK(hipMemcpyAsync(c->dbg + ((size_t)l * c->dbg_tokens + c0) * E, c->xb, nd * E * 4,
                              hipMemcpyDeviceToDevice, st));
      }
    }
    HIPCHK(hipGetLastError());
  }
  // logits of the last token: rmsnorm(x, output_norm), then the decode matvec
  HIPCHK(hipMemcpyAsync(c->x, c->xb + (size_t)(last_m - 1) * E, (size_t)E * 4, hipMemcpyDeviceToDevice, st));
  launch_rmsnorm_q8(st, c->x, m->output_norm.p, E, 1, eps, c->act_e, c->scratch);
  const DevTensor& ow = m->output.set ? m->output : m->token_embd;
  MvPlan p;
  mv_plan_init(p, E, c->act_e);
  mv_plan_set_f32(p, c->scratch);
  mv_plan_add(p, ow.dm, c->logits, nullptr);
  mv_plan_finish(p);
  mv_launch(st, p, err_word(c));
  HIPCHK(hipGetLastError());
  return RLH_OK;
}

int rlh_forward_batch(rlh_model* m, rlh_cache* c, const uint32_t* tokens, uint64_t n, uint64_t start_pos,
                      float* logits) {
  int rc = check_forward_args(m, c);
  if (rc) return rc;
  if (!tokens && n) return fail(RLH_EINVAL, "null tokens");
  n = std::min<uint64_t>(n, c->max_ctx > start_pos ? c->max_ctx - start_pos : 0);  // model.rs:392
  if (n == 0) return RLH_OK;
  for (uint64_t i = 0; i < n; i++)
    if (tokens[i] >= m->cfg.vocab_size) return fail(RLH_EINVAL, "token id out of range");
  if ((rc = forward_batch_impl(m, c, tokens, n, start_pos))) return rc;
  c->len = start_pos + n;
  c->logits_valid = true;
  return copy_logits(c, logits);
}

int rlh_forward_into(rlh_model* m, rlh_cache* c, const uint32_t* tokens, uint64_t n, uint64_t start_pos,
                     float* logits) {
  if (n > 1) return rlh_forward_batch(m, c, tokens, n, start_pos, logits);  // model.rs:362-366
  if (n == 0) return check_forward_args(m, c);
  if (!tokens) return fail(RLH_EINVAL, "null tokens");
  return rlh_forward_one(m, c, tokens[0], start_pos, logits);
}

int rlh_greedy_next(rlh_model* m, rlh_cache* c, uint32_t* token) {
  int rc = check_forward_args(m, c);
  if (rc) return rc;
  if (!token) return fail(RLH_EINVAL, "null token");
  if (!c->logits_valid) return fail(RLH_ESTATE, "no logits computed on this cache yet");
  launch_argmax(c->st, c->logits, m->cfg.vocab_size, c->pv, c->pi, c->nparts, c->st_dev + 3, nullptr, nullptr,
                nullptr);
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(c->host_st + 3, c->st_dev + 3, 4, hipMemcpyDeviceToHost, c->st));
  HIPCHK(hipStreamSynchronize(c->st));
  *token = c->host_st[3];
  return RLH_OK;
}

int rlh_sample_next(rlh_model* m, rlh_cache* c, const rlh_sampling_params* p, const uint32_t* recent,
                    uint64_t n_recent, uint64_t* rng_state, uint32_t* token) {
  int rc = check_forward_args(m, c);
  if (rc) return rc;
  if (!p || !rng_state || !token || (n_recent && !recent)) return fail(RLH_EINVAL, "null argument");
  if (!c->logits_valid) return fail(RLH_ESTATE, "no logits computed on this cache yet");
  if (!c->ds && (rc = rlh_dsampler_create(m->cfg.vocab_size, &c->ds))) return rc;
  return dsampler_sample(c->ds, c->logits, m->cfg.vocab_size, *p, recent, n_recent, rng_state, token, c->st);
}

int rlh_generate(rlh_model* m, rlh_cache* c, const uint32_t* prompt, uint64_t n_prompt, uint64_t max_new,
                 const rlh_sampling_params* p, uint32_t eos, uint32_t* out_tokens, uint64_t* n_out) {
  int rc = check_forward_args(m, c);
  if (rc) return rc;
  if (!prompt || !p || !n_out || (max_new && !out_tokens)) return fail(RLH_EINVAL, "null argument");
  if (n_prompt == 0) return fail(RLH_EINVAL, "empty prompt");
  *n_out = 0;
  uint64_t state = rlh_sampler_init(p->seed);
  if ((rc = rlh_cache_reset(c))) return rc;
  if ((rc = rlh_forward_into(m, c, prompt, n_prompt, 0, nullptr))) return rc;
  std::vector<uint32_t> recent(prompt, prompt + n_prompt);
  for (uint64_t i = 0; i < max_new; i++) {
    uint32_t next = 0;
    if ((rc = rlh_sample_next(m, c, p, recent.data(), recent.size(), &state, &next))) return rc;
    if (next == eos) break;
    out_tokens[(*n_out)++] = next;
    recent.push_back(next);
    if (c->len >= c->max_ctx) break;
    if ((rc = rlh_forward_into(m, c, &next, 1, c->len, nullptr))) return rc;
  }
  return RLH_OK;
}

int rlh_generate_greedy(rlh_model* m, rlh_cache* c, uint32_t first, uint64_t n_steps, uint32_t* out_tokens) {
  int rc = check_forward_args(m, c);
  if (rc) return rc;
  if (!out_tokens) return fail(RLH_EINVAL, "null out_tokens");
  if (first >= m->cfg.vocab_size) return fail(RLH_EINVAL, "token id out of range");
  uint64_t room = c->max_ctx > c->len ? c->max_ctx - c->len : 0;
  uint64_t n = std::min(n_steps, room);
  HIPCHK(hipStreamSynchronize(c->st));
  c->host_st[0] = first;
  c->host_st[1] = (uint32_t)c->len;
  c->host_st[2] = 0;
  HIPCHK(hipMemcpyAsync(c->st_dev, c->host_st, 12, hipMemcpyHostToDevice, c->st));
  HIPCHK(hipMemcpyAsync(c->hist, c->host_st, 4, hipMemcpyHostToDevice, c->st));
  uint64_t i = 0;
  if (!c->debug && c->use_graphs && c->g_greedy_n)
    for (; i + kGreedyBatch <= n; i += kGreedyBatch) HIPCHK(hipGraphLaunch(c->g_greedy_n, c->st));
  for (; i < n; i++)
    if ((rc = run_step(c, STEP_GREEDY, (int64_t)i))) return rc;
  HIPCHK(hipMemcpyAsync(out_tokens, c->hist, (n + 1) * 4, hipMemcpyDeviceToHost, c->st));
  if ((rc = sync_checked(c))) return rc;
  c->len += n;
  if (n > 0) {
    c->logits_valid = true;
  }
  if (n < n_steps) return fail(RLH_ECTX, "cache full after " + std::to_string(n) + " steps");
  return RLH_OK;
}

int rlh_debug_layer_hidden(rlh_cache* c, int layer, float* out, uint64_t max_tokens) {
  if (!c || !out) return fail(RLH_EINVAL, "null argument");
  if (!c->dbg) return fail(RLH_ESTATE, "debug capture is off (rlh_cache_set_debug)");
  if (layer < 0 || (uint32_t)layer >= c->m->cfg.n_layer) return fail(RLH_EINVAL, "layer out of range");
  uint64_t n = std::min(max_tokens, c->dbg_tokens);
  size_t E = c->m->cfg.n_embd;
  HIPCHK(hipStreamSynchronize(c->st));
  HIPCHK(hipMemcpy(out, c->dbg + (size_t)layer * c->dbg_tokens * E, n * E * 4, hipMemcpyDeviceToHost));
  return RLH_OK;
}

int rlh_cache_read_kv(rlh_cache* c, int layer, int which_v, uint64_t n_pos, float* out) {
  if (!c || !out) return fail(RLH_EINVAL, "null argument");
  if (layer < 0 || (uint32_t)layer >= c->m->cfg.n_layer) return fail(RLH_EINVAL, "layer out of range");
  if (n_pos > c->max_ctx) return fail(RLH_EINVAL, "n_pos > max_ctx");
  size_t kvd = (size_t)c->m->cfg.n_head_kv * c->m->cfg.head_dim;
  HIPCHK(hipStreamSynchronize(c->st));
  HIPCHK(hipMemcpy(out, which_v ? layer_v(c, layer) : layer_k(c, layer), n_pos * kvd * 4, hipMemcpyDeviceToHost));
  return RLH_OK;
}

// ---- op-level entries ----------------------------------------------------
int rlh_quantize_q8(const float* x, uint64_t n, int8_t* qs, float* scales, int32_t* sums, int32_t* sums16) {
  if (!x || !qs || !scales || !sums || !sums16) return fail(RLH_EINVAL, "null argument");
  if (n == 0 || n % 32) return fail(RLH_EINVAL, "n must be a positive multiple of 32");
  int rc = ensure_device();
  if (rc) return rc;
  hipStream_t st = op_stream();
  DevBuf<float> dx;
  DevBuf<int8_t> dq;
  DevBuf<float> dd;
  DevBuf<int32_t> ds, ds16;
  if (dx.alloc(n) || dq.alloc(n) || dd.alloc(n / 32) || ds.alloc(n / 32) || ds16.alloc(n / 16))
    return fail(RLH_ENOMEM, "hipMalloc");
  HIPCHK(hipMemcpyAsync(dx.p, x, n * 4, hipMemcpyHostToDevice, st));
  launch_quantize_q8(st, dx.p, (uint32_t)n, Q8Buf{dq.p, dd.p, ds.p, ds16.p});
  HIPCHK(hipGetLastError());
  HIPCHK(hipMemcpyAsync(qs, dq.p, n, hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemcpyAsync(scales, dd.p, n / 32 * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemcpyAsync(sums, ds.p, n / 32 * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemcpyAsync(sums16, ds16.p, n / 16 * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  return RLH_OK;
}

static int op_upload(DevTensor& t, uint32_t ty, const void* w, uint64_t rows, uint64_t cols) {
  if (!w) return fail(RLH_EINVAL, "null weights");
  int rc = ensure_device();
  if (rc) return rc;
  return upload_matrix(t, ty, w, cols, rows);
}

int rlh_dequant(uint32_t ty, const void* bytes, uint64_t n, float* out) {
  if (!out) return fail(RLH_EINVAL, "null argument");
  if (block_size(ty) == 0) return fail(RLH_EINVAL, "unknown ggml type");
  DevTensor t;
  int rc = op_upload(t, ty, bytes, 1, n);
  if (rc) return rc;
  hipStream_t st = op_stream();
  DevBuf<float> d;
  if (d.alloc(n)) {
    free_tensor(t);
    return fail(RLH_ENOMEM, "hipMalloc");
  }
  launch_dequant(st, t.dm, d.p);
  hipError_t e = hipMemcpyAsync(out, d.p, n * 4, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  free_tensor(t);
  if (e != hipSuccess) return fail(RLH_EDEVICE, hipGetErrorString(e));
  return RLH_OK;
}

int rlh_matvec(uint32_t ty, const void* w, uint64_t rows, uint64_t cols, const float* x, float* y) {
  if (!x || !y) return fail(RLH_EINVAL, "null argument");
  if (!matvec_supported(ty)) return fail(RLH_EUNSUP, "no matvec kernel for ggml type " + std::to_string(ty));
  if (cols == 0 || cols % 256) return fail(RLH_EINVAL, "cols must be a positive multiple of 256");
  if (rows == 0 || rows > 0xffffffffull) return fail(RLH_EINVAL, "rows out of range");
  DevTensor t;
  int rc = op_upload(t, ty, w, rows, cols);
  if (rc) return rc;
  hipStream_t st = op_stream();
  DevBuf<float> dx, dy, dd;
  DevBuf<int8_t> dq;
  DevBuf<int32_t> ds, ds16;
  DevBuf<uint32_t> derr;
  if (dx.alloc(cols) || dy.alloc(rows) || dq.alloc(cols) || dd.alloc(cols / 32) || ds.alloc(cols / 32) ||
      ds16.alloc(cols / 16) || derr.alloc(1) || hipMemset(derr.p, 0, 4)) {
    free_tensor(t);
    return fail(RLH_ENOMEM, "hipMalloc");
  }
  const Q8Buf act{dq.p, dd.p, ds.p, ds16.p};
  MvPlan p;
  mv_plan_init(p, (uint32_t)cols, act);
  mv_plan_set_f32(p, dx.p);
  mv_plan_add(p, t.dm, dy.p, nullptr);
  if (!mv_plan_finish(p)) {
    free_tensor(t);
    return fail(RLH_EUNSUP, "row length " + std::to_string(cols) + " exceeds the matvec LDS budget");
  }
  hipError_t e = hipMemcpyAsync(dx.p, x, cols * 4, hipMemcpyHostToDevice, st);
  launch_quantize_q8(st, dx.p, (uint32_t)cols, act);  // quantize_q8 once (ops.rs:104)
  mv_launch(st, p, derr.p);
  uint32_t werr = 0;
  if (e == hipSuccess) e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(y, dy.p, rows * 4, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipMemcpyAsync(&werr, derr.p, 4, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  free_tensor(t);
  if (e != hipSuccess) return fail(RLH_EDEVICE, hipGetErrorString(e));
  if (werr) return fail(RLH_EDEVICE, "a bounded device wait of the matvec expired (flags " + std::to_string(werr) + ")");
  return RLH_OK;
}

int rlh_matmul_batch(uint32_t ty, const void* w, uint64_t rows, uint64_t cols, const float* xs, uint64_t n,
                     float* ys) {
  if (!xs || !ys) return fail(RLH_EINVAL, "null argument");
  if (n == 0) return RLH_OK;
  if (n == 1) return rlh_matvec(ty, w, rows, cols, xs, ys);  // ops.rs:158-161
  if (!gemm_supported(ty) && !gemm_f32_supported(ty))
    return fail(RLH_EUNSUP, "no batched kernel for ggml type " + std::to_string(ty));
  if (cols == 0 || cols % 256) return fail(RLH_EINVAL, "cols must be a positive multiple of 256");
  if (rows == 0 || rows > 0xffffffffull || n > 0xffffffffull / cols) return fail(RLH_EINVAL, "shape out of range");
  DevTensor t;
  int rc = op_upload(t, ty, w, rows, cols);
  if (rc) return rc;
  hipStream_t st = op_stream();
  const uint64_t nv = n * cols;
  DevBuf<float> dx, dy, dd;
  DevBuf<int8_t> dq;
  DevBuf<int32_t> ds, ds16;
  if (dx.alloc(nv) || dy.alloc(n * rows) || dq.alloc(nv) || dd.alloc(nv / 32) || ds.alloc(nv / 32) ||
      ds16.alloc(nv / 16)) {
    free_tensor(t);
    return fail(RLH_ENOMEM, "hipMalloc");
  }
  // quantize_q8 of every token row (ops.rs:207-209), then the products
  const Q8Buf act{dq.p, dd.p, ds.p, ds16.p};
  hipError_t e = hipMemcpyAsync(dx.p, xs, nv * 4, hipMemcpyHostToDevice, st);
  if (gemm_supported(ty)) {
    launch_quantize_q8(st, dx.p, (uint32_t)nv, act);
    launch_gemm(st, t.dm, act, (uint32_t)n, dy.p, nullptr);
  } else {  // the f32 route (ops.rs:237-312): no activation quantization
    launch_gemm_f32(st, t.dm, dx.p, (uint32_t)n, (uint32_t)(n - n % 4), dy.p, nullptr);
  }
  if (e == hipSuccess) e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(ys, dy.p, n * rows * 4, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  free_tensor(t);
  if (e != hipSuccess) return fail(RLH_EDEVICE, hipGetErrorString(e));
  return RLH_OK;
}

int rlh_block_dots(uint32_t ty, const void* w, uint64_t rows, uint64_t cols, const int8_t* q8, int32_t* out) {
  if (!q8 || !out) return fail(RLH_EINVAL, "null argument");
  if (!gemm_supported(ty)) return fail(RLH_EUNSUP, "no integer dot for ggml type " + std::to_string(ty));
  uint32_t per_row = ty == RLH_TYPE_Q6_K ? (uint32_t)(cols / 16) : (uint32_t)(cols / 32);
  DevTensor t;
  int rc = op_upload(t, ty, w, rows, cols);
  if (rc) return rc;
  hipStream_t st = op_stream();
  DevBuf<int8_t> dq;
  DevBuf<int32_t> dout;
  if (dq.alloc(cols) || dout.alloc(rows * per_row)) {
    free_tensor(t);
    return fail(RLH_ENOMEM, "hipMalloc");
  }
  hipError_t e = hipMemcpyAsync(dq.p, q8, cols, hipMemcpyHostToDevice, st);
  launch_block_dots(st, t.dm, dq.p, dout.p, per_row);
  if (e == hipSuccess) e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(out, dout.p, rows * per_row * 4, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  free_tensor(t);
  if (e != hipSuccess) return fail(RLH_EDEVICE, hipGetErrorString(e));
  return RLH_OK;
}

// ---- measurement -----------------------------------------------------------
static const DevTensor* find_matrix(rlh_model* m, int kind, int layer) {
  if (kind == RLH_T_TOKEN_EMBD) return &m->token_embd;
  if (kind == RLH_T_OUTPUT) return m->output.set ? &m->output : &m->token_embd;
  if (layer < 0 || (uint32_t)layer >= m->cfg.n_layer) return nullptr;
  Layer& L = m->layers[layer];
  switch (kind) {
    case RLH_T_ATTN_Q: return &L.q;
    case RLH_T_ATTN_K: return &L.k;
    case RLH_T_ATTN_V: return &L.v;
    case RLH_T_ATTN_OUTPUT: return &L.o;
    case RLH_T_FFN_GATE: return &L.gate;
    case RLH_T_FFN_UP: return &L.up;
    case RLH_T_FFN_DOWN: return &L.down;
    default: return nullptr;
  }
}

int rlh_profile_matvec(rlh_model* m, rlh_cache* c, int kind, int iters, double* avg_us) {
  int rc = check_forward_args(m, c);
  if (rc) return rc;
  if (!avg_us || iters <= 0 || iters > 4096) return fail(RLH_EINVAL, "bad argument");
  const rlh_config& cfg = m->cfg;
  const bool global = kind == RLH_T_OUTPUT || kind == RLH_T_TOKEN_EMBD;
  const bool pair = kind == RLH_T_FFN_GATE || kind == RLH_T_FFN_UP;
  const bool qkv = kind == RLH_T_ATTN_Q;
  // One plan per layer, built as the decode step builds that launch, so the
  // launches rotate over every layer's weights and stream them from HBM
  // rather than from the 256 MB last-level cache a re-launched matrix would
  // sit in.
  std::vector<MvPlan> plans;
  for (uint32_t l = 0; l < (global ? 1u : cfg.n_layer); l++) {
    MvPlan p;
    if (global) {
      const DevTensor* t = find_matrix(m, kind, 0);
      if (!t || !t->set) return fail(RLH_EINVAL, "no such matrix");
      mv_plan_init(p, (uint32_t)t->cols, c->act_e);
      mv_plan_set_f32(p, c->scratch);
      mv_plan_add(p, t->dm, c->logits, nullptr);
    } else {
      const Layer& L = m->layers[l];
      if (pair) {
        mv_plan_init_norm(p, cfg.n_embd, c->x, L.ffn_norm.p, cfg.rms_eps);
        mv_plan_add_pair(p, L.gate.dm, L.up.dm, c->act_f, c->g);
      } else if (qkv) {
        mv_plan_init_norm(p, cfg.n_embd, c->x, L.attn_norm.p, cfg.rms_eps);
        mv_plan_add(p, L.v.dm, c->v, nullptr);  // as the decode step orders them
        mv_plan_add(p, L.q.dm, c->q, nullptr);
        mv_plan_add(p, L.k.dm, c->k, nullptr);
      } else {
        const DevTensor* t = find_matrix(m, kind, (int)l);
        if (!t || !t->set) return fail(RLH_EINVAL, "no such matrix");
        const uint32_t cols = (uint32_t)t->cols;
        if (kind == RLH_T_ATTN_OUTPUT) {  // attention output in, as in decode
          plan_attn_output(p, c, cols);
        } else if (kind == RLH_T_FFN_DOWN) {  // silu(g)*u in
          mv_plan_init(p, cols, c->act_f);
          mv_plan_set_f32(p, c->g);
        } else {  // rmsnorm(x) in (attn_k / attn_v alone)
          mv_plan_init_norm(p, cols, c->x, L.attn_norm.p, cfg.rms_eps);
        }
        mv_plan_add(p, t->dm, c->logits, nullptr);
      }
    }
    if (!mv_plan_finish(p)) return fail(RLH_EUNSUP, "matvec shape");
    plans.push_back(p);
  }
  // back-to-back launches between one event pair on the cache's stream, as
  // the kernels follow each other inside a captured step (an event pair
  // around each launch would add the events' own cost to every launch)
  hipEvent_t e0, e1;
  HIPCHK(hipEventCreate(&e0));
  HIPCHK(hipEventCreate(&e1));
  mv_launch(c->st, plans[0], err_word(c));  // warm-up
  (void)hipEventRecord(e0, c->st);
  for (int i = 0; i < iters; i++) mv_launch(c->st, plans[i % plans.size()], err_word(c));
  (void)hipEventRecord(e1, c->st);
  hipError_t e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (e != hipSuccess) return fail(RLH_EDEVICE, std::string("profile events: ") + hipGetErrorString(e));
  if ((rc = sync_checked(c))) return rc;
  const double total_ms = ms;
  *avg_us = total_ms * 1000.0 / iters;
  return RLH_OK;
}

// ---- greedy argmax without allocation ------------------------------------
}  // extern "C"

namespace {

// Partial (value, index) pairs of one rlh_argmax_noalloc call: one per block
// of the partial launch, values first, then indices. Every call writes all
// of them before the final reduction reads them, so nothing is cleared
// between calls.
constexpr uint32_t kNoAllocParts = 256;
static __device__ __align__(256) uint32_t scratch[2 * kNoAllocParts];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// The current device's address of `scratch` (looked up once per device
// with that device current; host code uses only this address).
int noalloc_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail(RLH_EDEVICE, "no HIP device available (librlh needs an MI355X / gfx950 GPU)");
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(RLH_EDEVICE, "device ordinal out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(RLH_EDEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return RLH_OK;
}

// True when p is memory the current device can read or write.
bool device_accessible(const void* p) {
  hipPointerAttribute_t a{};
  if (hipPointerGetAttributes(&a, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return a.devicePointer != nullptr;
}

}  // namespace

extern "C" {

int rlh_argmax_noalloc(const float* logits, uint64_t n, uint32_t* token, void* stream) {
  if (!logits || !token) return fail(RLH_EINVAL, "null argument");
  if (n == 0 || n > kNoAllocMaxN)
    return fail(RLH_EINVAL, "n = " + std::to_string(n) + " is outside [1, " + std::to_string(kNoAllocMaxN) + "]");
  // only calls that are legal under stream capture: the current device, the
  // pointers' attributes and (once per device) the scratch array's address
  void* sp = nullptr;
  int rc = noalloc_scratch(&sp);
  if (rc) return rc;
  if (!device_accessible(logits) || !device_accessible(token))
    return fail(RLH_EINVAL, "logits and token must be device-accessible memory");
  float* pv = (float*)sp;
  uint32_t* pi = (uint32_t*)sp + kNoAllocParts;
  launch_argmax((hipStream_t)stream, logits, (uint32_t)n, pv, pi, kNoAllocParts, token, nullptr, nullptr, nullptr);
  HIPCHK(hipGetLastError());
  return RLH_OK;
}

int rlh_profile_decode_kernel(rlh_model* m, rlh_cache* c, int kind, uint32_t first, int steps, double* avg_us,
                              uint64_t* launches) {
  int rc = check_forward_args(m, c);
  if (rc) return rc;
  if (!avg_us || steps <= 0 || steps > 4096) return fail(RLH_EINVAL, "bad argument");
  if (kind != RLH_T_ATTN_Q && kind != RLH_T_ATTN_OUTPUT && kind != RLH_T_FFN_GATE && kind != RLH_T_FFN_DOWN &&
      kind != RLH_T_OUTPUT)
    return fail(RLH_EINVAL, "kind names no decode matvec launch");
  if (first >= m->cfg.vocab_size) return fail(RLH_EINVAL, "token id out of range");
  if (c->len + (uint64_t)steps > c->max_ctx) return fail(RLH_ECTX, "not enough room in the cache");
  if (c->debug) return fail(RLH_ESTATE, "profiling needs debug capture off");
  const uint32_t per_step = kind == RLH_T_OUTPUT ? 1u : m->cfg.n_layer;
  const size_t n = (size_t)per_step * steps;
  HIPCHK(hipStreamSynchronize(c->st));
  c->probe_ev.assign(2 * n, nullptr);
  auto release = [c] {
    for (hipEvent_t e : c->probe_ev)
      if (e) (void)hipEventDestroy(e);
    c->probe_ev.clear();
    c->probe_kind = -1;
    c->probe_used = 0;
  };
  for (auto& e : c->probe_ev)
    if (hipEventCreate(&e) != hipSuccess) {
      release();
      return fail(RLH_EDEVICE, "hipEventCreate");
    }
  c->host_st[0] = first;
  c->host_st[1] = (uint32_t)c->len;
  c->host_st[2] = 0;
  if (hipMemcpyAsync(c->st_dev, c->host_st, 12, hipMemcpyHostToDevice, c->st) != hipSuccess) {
    release();
    return fail(RLH_EDEVICE, "hipMemcpyAsync");
  }
  c->probe_kind = kind;
  c->probe_used = 0;
  for (int i = 0; i < steps; i++) enqueue_step(c, STEP_GREEDY, -1);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(c->st);
  double total_ms = 0.0;
  for (uint32_t i = 0; e == hipSuccess && i < c->probe_used; i++) {
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, c->probe_ev[2 * i], c->probe_ev[2 * i + 1]);
    total_ms += ms;
  }
  const uint32_t used = c->probe_used;
  release();
  if (e != hipSuccess) return fail(RLH_EDEVICE, std::string("kernel probe: ") + hipGetErrorString(e));
  if ((rc = sync_checked(c))) return rc;
  c->len += (uint64_t)steps;
  c->logits_valid = true;
  *avg_us = used ? total_ms * 1000.0 / used : 0.0;
  if (launches) *launches = used;
  return RLH_OK;
}

int rlh_profile_decode(rlh_model* m, rlh_cache* c, int iters, double* avg_us) {
  int rc = check_forward_args(m, c);
  if (rc) return rc;
  if (!avg_us || iters <= 0) return fail(RLH_EINVAL, "bad argument");
  if (c->len + (uint64_t)iters > c->max_ctx) return fail(RLH_ECTX, "not enough room in the cache");
  if (c->debug) return fail(RLH_ESTATE, "profiling needs debug capture off");
  HIPCHK(hipStreamSynchronize(c->st));
  c->host_st[0] = 0;
  c->host_st[1] = (uint32_t)c->len;
  c->host_st[2] = 0;
  HIPCHK(hipMemcpyAsync(c->st_dev, c->host_st, 12, hipMemcpyHostToDevice, c->st));
  hipEvent_t e0, e1;
  HIPCHK(hipEventCreate(&e0));
  HIPCHK(hipEventCreate(&e1));
  HIPCHK(hipEventRecord(e0, c->st));
  for (int i = 0; i < iters; i++)
    if ((rc = run_step(c, STEP_GREEDY, -1))) return rc;
  HIPCHK(hipEventRecord(e1, c->st));
  HIPCHK(hipEventSynchronize(e1));
  float ms = 0.f;
  HIPCHK(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if ((rc = sync_checked(c))) return rc;
  c->len += (uint64_t)iters;
  c->logits_valid = true;
  *avg_us = (double)ms * 1000.0 / iters;
  return RLH_OK;
}

}  // extern "C"
