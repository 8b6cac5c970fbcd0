// C ABI of the decode-step operations around attention (include/qdiy/decode.h)
// and of the .bin model format and greedy decode engine (include/qdiy/engine.h).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <thread>
#include <vector>

#include "qd_internal.h"
#include "qdiy/decode.h"
#include "qdiy/engine.h"

using qd::aligned16;
using qd::aligned2;
using qd::aligned8;
using qd::fail;
using qd::overlaps;
using qd::hip_fail;

namespace {


// ---------------------------------------------------------------------------
// .bin layout (model_weights/convert_weights.py:105-185): element offsets of
// every tensor from the start of the tensor data (byte 28 of the file).

struct LayerOff {
  long long ln_1, qkv_w, qkv_b, proj_w, ln_2, w1, w2, w_down;
};

struct ModelLayout {
  long long wte = 0;
  std::vector<LayerOff> layers;
  long long ln_f = 0, lm_head = 0, total = 0;   // total fp16 elements
};

bool cfg_valid(const qd_model_cfg* c) {
  return c && c->vocab_size >= 1 && c->num_layers >= 1 && c->num_heads >= 1 &&
         c->hidden_size == c->num_heads * (uint32_t)QD_HEAD_DIM && c->hidden_size % 512 == 0 &&
         c->hidden_size <= 4096 && c->intermediate_size >= 8 && c->intermediate_size % 8 == 0 &&
         c->max_seqlen >= 1 && c->vocab_size < (1u << 30) && c->num_layers <= 4096 &&
         c->intermediate_size <= 8192;
}

ModelLayout layout_of(const qd_model_cfg& c) {
  ModelLayout L;
  const long long V = c.vocab_size, H = c.hidden_size, I = c.intermediate_size;
  long long o = 0;
  L.wte = o;
  o += V * H;
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    LayerOff f;
    f.ln_1 = o;   o += H;
    f.qkv_w = o;  o += 3 * H * H;
    f.qkv_b = o;  o += 3 * H;
    f.proj_w = o; o += H * H;
    f.ln_2 = o;   o += H;
    f.w1 = o;     o += I * H;
    f.w2 = o;     o += I * H;
    f.w_down = o; o += H * I;
    L.layers.push_back(f);
  }
  L.ln_f = o;    o += H;
  L.lm_head = o; o += V * H;
  L.total = o;
  return L;
}

uint64_t splitmix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// float -> binary16, round to nearest even (finite inputs of modest size).
uint16_t to_half(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  x &= 0x7FFFFFFFu;
  if (x >= 0x47800000u) return (uint16_t)(sign | (x > 0x7F800000u ? 0x7E00u : 0x7C00u));
  if (x < 0x38800000u) {                              // subnormal or zero in fp16
    if (x < 0x33000000u) return (uint16_t)sign;       // below half the smallest subnormal
    const uint32_t m = (x & 0x7FFFFFu) | 0x800000u;
    const int shift = 126 - (int)(x >> 23);           // 14..24
    uint32_t r = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ((x >> 13) - (112u << 10));
  const uint32_t rem = x & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}

void fill_range(uint16_t* t, long long begin, long long end, uint64_t seed, float scale,
                const std::vector<std::pair<long long, long long>>& ones) {
  for (long long i = begin; i < end; ++i) {
    const uint64_t z = splitmix64(seed + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull);
    const int s = (int)(z & 0xFFFF) + (int)((z >> 16) & 0xFFFF) + (int)((z >> 32) & 0xFFFF) +
                  (int)(z >> 48) - 2 * 65535;
    t[i] = to_half((float)s * scale);
  }
  for (const auto& r : ones) {
    const long long b = std::max(begin, r.first), e = std::min(end, r.second);
    for (long long i = b; i < e; ++i) t[i] = 0x3C00;  // 1.0
  }
}

constexpr float kEps = 1e-6f;      // qwen_infer.cu:620
constexpr int kPrefillChunk = 256; // prompt tokens per batched prefill pass (exact mode)
constexpr int kPrefillChunkMfma = 2048;  // ... in the matrix-core mode: M of its GEMMs
constexpr int kEosA = 151645;      // <|im_end|>, qwen_infer.cu:801
constexpr int kEosB = 151643;      // <|endoftext|>

}  // namespace

struct qd_engine {
  qd_model_cfg cfg;
  ModelLayout lay;
  int device = -1;
  hipStream_t stream = nullptr;
  qd_ctx* attn = nullptr;
  uint16_t* weights = nullptr;          // tensor data of the image, file order
  uint16_t* k_cache = nullptr;          // [layers][max_seqlen][hidden]
  uint16_t* v_cache = nullptr;
  uint16_t* x = nullptr;                // residual stream [hidden]
  uint16_t* qkv = nullptr;              // [3*hidden]
  uint16_t* attn_out = nullptr;         // [hidden]
  uint16_t* act = nullptr;              // [inter]
  uint16_t* logits = nullptr;           // [vocab]
  void* lm_ws = nullptr;
  size_t lm_ws_bytes = 0;
  int* h_token = nullptr;               // pinned, mapped: the argmax writes it directly
  int* h_token_dev = nullptr;           // h_token's device address
  long long kv_bytes = 0;
  int prefill_mode = QD_GEMM_EXACT;     // qd_engine_prefill's projections and attention
  // batched prefill scratch for p_cap tokens
  int p_cap = 0;
  int* p_tokens = nullptr;
  uint16_t *p_x = nullptr, *p_xn = nullptr, *p_qkv = nullptr, *p_att = nullptr;
  uint16_t *p_g = nullptr, *p_u = nullptr, *p_act = nullptr;   // p_u lies inside p_g's allocation
  float* p_split = nullptr;             // split-K partials of the MFMA prefill GEMMs

  const uint16_t* w(long long off) const { return weights + off; }
  uint16_t* kc(int l) const { return k_cache + (long long)l * cfg.max_seqlen * cfg.hidden_size; }
  uint16_t* vc(int l) const { return v_cache + (long long)l * cfg.max_seqlen * cfg.hidden_size; }
};

namespace {

void engine_free(qd_engine* e) {
  if (!e) return;
  int prev = -1;
  (void)hipGetDevice(&prev);
  if (e->device >= 0) (void)hipSetDevice(e->device);
  if (e->stream) (void)hipStreamSynchronize(e->stream);
  (void)hipFree(e->weights);
  (void)hipFree(e->k_cache);
  (void)hipFree(e->v_cache);
  (void)hipFree(e->x);
  (void)hipFree(e->qkv);
  (void)hipFree(e->attn_out);
  (void)hipFree(e->act);
  (void)hipFree(e->logits);
  (void)hipFree(e->lm_ws);
  (void)hipFree(e->p_split);
  for (void* q : {(void*)e->p_tokens, (void*)e->p_x, (void*)e->p_xn, (void*)e->p_qkv, (void*)e->p_att,
                  (void*)e->p_g, (void*)e->p_act})
    (void)hipFree(q);
  if (e->h_token) (void)hipHostFree(e->h_token);
  if (e->attn) qd_ctx_destroy(e->attn);
  if (e->stream) (void)hipStreamDestroy(e->stream);
  if (prev >= 0) (void)hipSetDevice(prev);
  delete e;
}

// (Re)allocates the batched prefill scratch for `cap` tokens.  The new buffers
// are allocated before the old ones are freed, so on failure the engine keeps
// its previous scratch.  The caller has synchronised the engine's stream.
int resize_prefill_scratch(qd_engine* e, int cap) {
  const long long H = e->cfg.hidden_size, I = e->cfg.intermediate_size;
  int* tok = nullptr;
  uint16_t *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *g = nullptr, *act = nullptr;
  // g holds 2 * inter columns per token: [g | u] rows of the joint gate/up
  // product, or g then u as two packed blocks
  struct { void** p; long long n; } allocs[] = {
      {(void**)&tok, (long long)cap * 4},    {(void**)&x, cap * H * 2},   {(void**)&xn, cap * H * 2},
      {(void**)&qkv, cap * 3 * H * 2},       {(void**)&att, cap * H * 2}, {(void**)&g, cap * I * 4},
      {(void**)&act, cap * I * 2}};
  for (auto& a : allocs) {
    const hipError_t he = hipMalloc(a.p, (size_t)a.n);
    if (he != hipSuccess) {
      for (auto& b : allocs) (void)hipFree(*b.p);
      return fail(QD_ENOMEM, "hipMalloc of %lld bytes of prefill scratch failed: %s", a.n,
                  hipGetErrorString(he));
    }
  }
  for (void* q : {(void*)e->p_tokens, (void*)e->p_x, (void*)e->p_xn, (void*)e->p_qkv, (void*)e->p_att,
                  (void*)e->p_g, (void*)e->p_act})
    (void)hipFree(q);
  e->p_tokens = tok;
  e->p_x = x;
  e->p_xn = xn;
  e->p_qkv = qkv;
  e->p_att = att;
  e->p_g = g;
  e->p_u = g + cap * I;
  e->p_act = act;
  e->p_cap = cap;
  return QD_OK;
}

// Per-layer path of one token at `pos` (qwen_infer.cu:622-722).
int run_layers(qd_engine* e, int token, int pos) {
  const qd_model_cfg& c = e->cfg;
  const int H = (int)c.hidden_size, I = (int)c.intermediate_size, NH = (int)c.num_heads;
  const uint16_t* xin = e->w(e->lay.wte) + (long long)token * H;   // embedding row (:617)
  for (uint32_t l = 0; l < c.num_layers; ++l) {
    const LayerOff& f = e->lay.layers[l];
    // attention front end and attention (one launch where the plan allows)
    int rc = qd_qkv_proj_rope_cache_attention(e->attn, xin, e->w(f.ln_1), kEps, e->w(f.qkv_w),
                                              e->w(f.qkv_b), e->qkv, e->kc(l), e->vc(l), e->attn_out,
                                              pos, (int)c.max_seqlen, NH, QD_HEAD_DIM, e->stream);
    if (rc == QD_OK) rc = qd_proj_residual(e->attn_out, e->w(f.proj_w), xin, e->x, H, H, e->stream);
    if (rc == QD_OK)
      rc = qd_ffn_up_swiglu(e->x, e->w(f.ln_2), kEps, e->w(f.w1), e->w(f.w2), e->act, H, I, e->stream);
    if (rc == QD_OK) rc = qd_proj_residual(e->act, e->w(f.w_down), e->x, e->x, H, I, e->stream);
    if (rc != QD_OK) return rc;
    xin = e->x;
  }
  return QD_OK;
}

// Prompt tokens at positions pos0.. through all layers in batches, in the
// decode kernels' arithmetic (qd_prefill.hip): the KV rows written are
// bit-identical to run_layers() token by token.
int prefill_batched(qd_engine* e, const int* tokens, int T, int pos0) {
  const qd_model_cfg& c = e->cfg;
  const int H = (int)c.hidden_size, I = (int)c.intermediate_size, NH = (int)c.num_heads;
  hipError_t he = hipMemcpyAsync(e->p_tokens, tokens, sizeof(int) * (size_t)T, hipMemcpyHostToDevice,
                                 e->stream);
  if (he == hipSuccess) he = qd::launch_embed(e->w(e->lay.wte), e->p_tokens, e->p_x, H, T, e->stream);
  auto gemv = [&](const uint16_t* x, long long ldx, const uint16_t* w, int n, int k, uint16_t* y,
                  long long ldy, int epi) {
    qd::BatchedGemvParams p{x, ldx, w, n, k, T, y, ldy, y};
    if (e->prefill_mode == QD_GEMM_MFMA && k % 64 == 0)
      return qd::launch_gemm_mfma_split(p, epi, e->p_split, qd::kGemmSplitWsBytes, e->stream);
    return qd::launch_gemv_batched(p, epi, e->stream);
  };
  for (uint32_t l = 0; l < c.num_layers && he == hipSuccess; ++l) {
    const LayerOff& f = e->lay.layers[l];
    he = qd::launch_rmsnorm_batched(e->p_x, e->w(f.ln_1), kEps, e->p_xn, H, T, e->stream);
    if (he == hipSuccess) he = gemv(e->p_xn, H, e->w(f.qkv_w), 3 * H, H, e->p_qkv, 3 * H, 0);
    if (he == hipSuccess)
      he = qd::launch_rope_batched(e->p_qkv, e->w(f.qkv_b), e->kc(l), e->vc(l), e->attn->rope_cs,
                                   e->attn->cfg.kv_row_stride, e->attn->cfg.kv_head_stride, pos0, NH,
                                   T, e->stream);
    if (he != hipSuccess) break;
    const int rc = e->prefill_mode == QD_GEMM_MFMA
                       ? qd::attention_prefill_mfma(e->attn, e->p_qkv, 3 * H, e->kc(l), e->vc(l),
                                                    e->p_att, H, pos0, T, e->stream)
                       : qd::attention_prefill(e->attn, e->p_qkv, 3 * H, e->kc(l), e->vc(l), e->p_att,
                                               H, pos0, T, e->stream);
    if (rc != QD_OK) return rc;
    he = gemv(e->p_att, H, e->w(f.proj_w), H, H, e->p_x, H, 1);
    if (he == hipSuccess) he = qd::launch_rmsnorm_batched(e->p_x, e->w(f.ln_2), kEps, e->p_xn, H, T, e->stream);
    bool joint = false;                          // gate/up GEMM with the SwiGLU in its epilogue
    if (he == hipSuccess && e->prefill_mode == QD_GEMM_MFMA && !joint) {
      qd::BatchedGemvParams q{e->p_xn, H, e->w(f.w1), I, H, T, e->p_act, I, nullptr};
      q.w2 = e->w(f.w2);
      const hipError_t je = qd::launch_gemm_mfma_swiglu(q, e->stream);
      joint = je == hipSuccess;
      if (je != hipSuccess && je != hipErrorNotSupported) he = je;
    }
    if (he == hipSuccess && !joint) he = gemv(e->p_xn, H, e->w(f.w1), I, H, e->p_g, I, 0);
    if (he == hipSuccess && !joint) he = gemv(e->p_xn, H, e->w(f.w2), I, H, e->p_u, I, 0);
    if (he == hipSuccess && !joint)
      he = qd::launch_swiglu_batched(e->p_g, e->p_u, e->p_act, T, I, I, e->stream);
    if (he == hipSuccess) he = gemv(e->p_act, I, e->w(f.w_down), H, I, e->p_x, H, 1);
  }
  return he == hipSuccess ? QD_OK : hip_fail(he, "prefill launch");
}

int check_engine(const qd_engine* e) {
  if (!e) return fail(QD_EINVAL, "engine is NULL");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != e->device)
    return fail(QD_EINVAL, "current device %d is not the engine's device %d", dev, e->device);
  return QD_OK;
}

}  // namespace

extern "C" {

// ----------------------------------------------------------------- decode.h

int qd_proj_residual(const uint16_t* x, const uint16_t* w, const uint16_t* residual, uint16_t* out,
                     int n_out, int k_in, hipStream_t stream) {
  if (!x || !w || !residual || !out) return fail(QD_EINVAL, "x, w, residual and out must be non-NULL");
  if (!aligned16(x) || !aligned16(w)) return fail(QD_EINVAL, "x and w must be 16-byte aligned");
  if (!aligned2(residual) || !aligned2(out)) return fail(QD_EINVAL, "residual and out must be 2-byte aligned");
  if (n_out < 1) return fail(QD_EINVAL, "n_out %d must be >= 1", n_out);
  if (k_in < 8 || k_in % 8 != 0 || k_in > 8192)
    return fail(QD_EINVAL, "k_in %d must be a multiple of 8 in [8, 8192]", k_in);
  const size_t ob = (size_t)n_out * 2;
  if (overlaps(out, ob, x, (size_t)k_in * 2) || overlaps(out, ob, w, (size_t)n_out * k_in * 2) ||
      (residual != out && overlaps(out, ob, residual, ob)))
    return fail(QD_EINVAL, "out overlaps x, w or (other than exactly) residual");
  qd::ProjResidualParams p{x, w, residual, out, n_out, k_in};
  hipError_t e = qd::launch_proj_residual(p, stream);
  return e == hipSuccess ? QD_OK : hip_fail(e, "proj_residual launch");
}

int qd_ffn_up_swiglu(const uint16_t* x, const uint16_t* norm_w, float eps, const uint16_t* w1,
                     const uint16_t* w2, uint16_t* act, int hidden, int inter, hipStream_t stream) {
  if (!x || !norm_w || !w1 || !w2 || !act)
    return fail(QD_EINVAL, "x, norm_w, w1, w2 and act must be non-NULL");
  if (!aligned16(x) || !aligned16(norm_w) || !aligned16(w1) || !aligned16(w2))
    return fail(QD_EINVAL, "x, norm_w, w1 and w2 must be 16-byte aligned");
  if (!aligned2(act)) return fail(QD_EINVAL, "act must be 2-byte aligned");
  if (hidden < 512 || hidden % 512 != 0 || hidden > 4096)
    return fail(QD_EINVAL, "hidden %d unsupported (multiple of 512, at most 4096)", hidden);
  if (inter < 1) return fail(QD_EINVAL, "inter %d must be >= 1", inter);
  if (!(eps >= 0.0f)) return fail(QD_EINVAL, "eps must be >= 0");
  const size_t ab = (size_t)inter * 2, hb = (size_t)hidden * 2, wb = (size_t)inter * hidden * 2;
  if (overlaps(act, ab, x, hb) || overlaps(act, ab, norm_w, hb) || overlaps(act, ab, w1, wb) ||
      overlaps(act, ab, w2, wb))
    return fail(QD_EINVAL, "act overlaps x, norm_w, w1 or w2");
  qd::FfnUpParams p{x, norm_w, eps, w1, w2, act, hidden, inter};
  hipError_t e = qd::launch_ffn_up(p, stream);
  return e == hipSuccess ? QD_OK : hip_fail(e, "ffn_up launch");
}

int qd_gemm_nt(const uint16_t* x, long long ldx, const uint16_t* w, const uint16_t* residual,
               uint16_t* y, long long ldy, int m, int n, int k, int mode, hipStream_t stream) {
  if (!x || !w || !y) return fail(QD_EINVAL, "x, w and y must be non-NULL");
  if (mode != QD_GEMM_EXACT && mode != QD_GEMM_MFMA) return fail(QD_EINVAL, "unknown mode %d", mode);
  if (m < 1 || n < 1) return fail(QD_EINVAL, "m %d and n %d must be >= 1", m, n);
  if (mode == QD_GEMM_EXACT && (k < 8 || k % 8 != 0 || k > 8192))
    return fail(QD_EINVAL, "k %d must be a multiple of 8 in [8, 8192] (exact mode)", k);
  if (mode == QD_GEMM_MFMA && (k < 64 || k % 64 != 0))
    return fail(QD_EINVAL, "k %d must be a positive multiple of 64 (MFMA mode)", k);
  if (ldx < k || ldx % 8 != 0 || ldy < n)
    return fail(QD_EINVAL, "ldx %lld must be a multiple of 8 and at least k, ldy %lld at least n", ldx, ldy);
  if (!aligned16(x) || !aligned16(w)) return fail(QD_EINVAL, "x and w must be 16-byte aligned");
  if (!aligned2(y) || (residual && !aligned2(residual))) return fail(QD_EINVAL, "y and residual must be 2-byte aligned");
  const size_t yb = ((size_t)(m - 1) * ldy + n) * 2;
  if (overlaps(y, yb, x, ((size_t)(m - 1) * ldx + k) * 2) || overlaps(y, yb, w, (size_t)n * k * 2) ||
      (residual && residual != y && overlaps(y, yb, residual, yb)))
    return fail(QD_EINVAL, "y overlaps x, w or (other than exactly) residual");
  qd::BatchedGemvParams p{x, ldx, w, n, k, m, y, ldy, residual ? residual : y};
  const int epi = residual ? 1 : 0;
  const hipError_t e = mode == QD_GEMM_MFMA ? qd::launch_gemm_mfma(p, epi, stream)
                                            : qd::launch_gemv_batched(p, epi, stream);
  return e == hipSuccess ? QD_OK : hip_fail(e, "gemm launch");
}

int qd_gemm_swiglu(const uint16_t* x, long long ldx, const uint16_t* w1, const uint16_t* w2,
                   uint16_t* act, long long ldy, int m, int n, int k, hipStream_t stream) {
  if (!x || !w1 || !w2 || !act) return fail(QD_EINVAL, "x, w1, w2 and act must be non-NULL");
  if (m < 1 || n < 1) return fail(QD_EINVAL, "m %d and n %d must be >= 1", m, n);
  if (k < 64 || k % 64 != 0) return fail(QD_EINVAL, "k %d must be a positive multiple of 64", k);
  if (ldx < k || ldx % 8 != 0 || ldy < n)
    return fail(QD_EINVAL, "ldx %lld must be a multiple of 8 and at least k, ldy %lld at least n", ldx, ldy);
  if (!aligned16(x) || !aligned16(w1) || !aligned16(w2))
    return fail(QD_EINVAL, "x, w1 and w2 must be 16-byte aligned");
  if (!aligned2(act)) return fail(QD_EINVAL, "act must be 2-byte aligned");
  const size_t ab = ((size_t)(m - 1) * ldy + n) * 2, wb = (size_t)n * k * 2;
  if (overlaps(act, ab, x, ((size_t)(m - 1) * ldx + k) * 2) || overlaps(act, ab, w1, wb) ||
      overlaps(act, ab, w2, wb))
    return fail(QD_EINVAL, "act overlaps x, w1 or w2");
  qd::BatchedGemvParams p{x, ldx, w1, n, k, m, act, ldy, nullptr};
  p.w2 = w2;
  const hipError_t e = qd::launch_gemm_mfma_swiglu(p, stream);
  return e == hipSuccess ? QD_OK : hip_fail(e, "gate/up GEMM launch");
}

size_t qd_lm_head_workspace_bytes(int vocab) {
  return vocab < 1 ? 0 : (size_t)qd::lm_head_parts(vocab) * sizeof(unsigned long long);
}

int qd_lm_head_argmax(const uint16_t* x, const uint16_t* norm_w, float eps, const uint16_t* w,
                      uint16_t* logits, int vocab, int hidden, void* workspace,
                      size_t workspace_bytes, int* token, hipStream_t stream) {
  if (!x || !norm_w || !w || !logits || !workspace || !token)
    return fail(QD_EINVAL, "x, norm_w, w, logits, workspace and token must be non-NULL");
  if (!aligned16(x) || !aligned16(norm_w) || !aligned16(w))
    return fail(QD_EINVAL, "x, norm_w and w must be 16-byte aligned");
  if (!aligned2(logits) || !aligned8(workspace) || (reinterpret_cast<uintptr_t>(token) & 3u))
    return fail(QD_EINVAL, "logits, workspace or token misaligned");
  if (hidden < 512 || hidden % 512 != 0 || hidden > 4096)
    return fail(QD_EINVAL, "hidden %d unsupported (multiple of 512, at most 4096)", hidden);
  if (vocab < 1 || vocab >= (1 << 30)) return fail(QD_EINVAL, "vocab %d out of range", vocab);
  if (workspace_bytes < qd_lm_head_workspace_bytes(vocab))
    return fail(QD_EINVAL, "workspace of %zu bytes below the %zu needed", workspace_bytes,
                qd_lm_head_workspace_bytes(vocab));
  if (!(eps >= 0.0f)) return fail(QD_EINVAL, "eps must be >= 0");
  {
    const size_t lb = (size_t)vocab * 2, hb = (size_t)hidden * 2, wb = (size_t)vocab * hidden * 2;
    const size_t kb = qd_lm_head_workspace_bytes(vocab);
    const void* in[3] = {x, norm_w, w};
    const size_t in_b[3] = {hb, hb, wb};
    for (int j = 0; j < 3; ++j)
      if (overlaps(logits, lb, in[j], in_b[j]) || overlaps(workspace, kb, in[j], in_b[j]) ||
          overlaps(token, sizeof(int), in[j], in_b[j]))
        return fail(QD_EINVAL, "logits, workspace or token overlaps x, norm_w or w");
    if (overlaps(logits, lb, workspace, kb) || overlaps(token, sizeof(int), logits, lb) ||
        overlaps(token, sizeof(int), workspace, kb))
      return fail(QD_EINVAL, "logits, workspace and token must not overlap each other");
  }
  qd::LmHeadParams p{x, norm_w, eps, w, logits, static_cast<unsigned long long*>(workspace), vocab,
                     hidden};
  hipError_t e = qd::launch_lm_head_argmax(p, token, stream);
  return e == hipSuccess ? QD_OK : hip_fail(e, "lm_head_argmax launch");
}

// ----------------------------------------------------------------- engine.h

long long qd_model_image_bytes(const qd_model_cfg* cfg) {
  if (!cfg_valid(cfg)) return -1;
  return QD_MODEL_HEADER_BYTES + 2 * layout_of(*cfg).total;
}

int qd_model_fill_random(void* image, long long bytes, const qd_model_cfg* cfg, uint64_t seed,
                         float std, int nthreads) {
  if (!image || !cfg_valid(cfg)) return fail(QD_EINVAL, "NULL image or invalid model configuration");
  if (bytes != qd_model_image_bytes(cfg))
    return fail(QD_EINVAL, "image holds %lld bytes, the configuration needs %lld", bytes,
                qd_model_image_bytes(cfg));
  if (!(std >= 0.0f) || !(std < 1e4f)) return fail(QD_EINVAL, "std must be in [0, 1e4)");
  const uint32_t hdr[7] = {QD_MODEL_MAGIC,  cfg->vocab_size,        cfg->hidden_size, cfg->num_layers,
                           cfg->num_heads,  cfg->intermediate_size, cfg->max_seqlen};
  std::memcpy(image, hdr, sizeof(hdr));
  const ModelLayout L = layout_of(*cfg);
  std::vector<std::pair<long long, long long>> ones;
  for (const LayerOff& f : L.layers) {
    ones.push_back({f.ln_1, f.ln_1 + cfg->hidden_size});
    ones.push_back({f.ln_2, f.ln_2 + cfg->hidden_size});
  }
  ones.push_back({L.ln_f, L.ln_f + cfg->hidden_size});
  // the sum of four uniforms on [0, 65535] has variance 4 * (65536^2 - 1) / 12
  const float scale = (float)((double)std / std::sqrt(4.0 * (65536.0 * 65536.0 - 1.0) / 12.0));
  uint16_t* t = reinterpret_cast<uint16_t*>(static_cast<char*>(image) + QD_MODEL_HEADER_BYTES);
  nthreads = std::max(1, std::min(nthreads, 256));
  const long long chunk = (L.total + nthreads - 1) / nthreads;
  std::vector<std::thread> th;
  for (int i = 0; i < nthreads; ++i) {
    const long long b = i * chunk, e = std::min(L.total, b + chunk);
    if (b >= e) break;
    th.emplace_back(fill_range, t, b, e, seed, scale, std::cref(ones));
  }
  for (auto& x : th) x.join();
  return QD_OK;
}

int qd_model_write_random(const char* path, const qd_model_cfg* cfg, uint64_t seed, float std) {
  if (!path) return fail(QD_EINVAL, "path is NULL");
  const long long bytes = qd_model_image_bytes(cfg);
  if (bytes < 0) return fail(QD_EINVAL, "invalid model configuration");
  std::vector<char> img;
  try {
    img.resize((size_t)bytes);
  } catch (...) {
    return fail(QD_ENOMEM, "cannot allocate %lld host bytes", bytes);
  }
  const unsigned hw = std::thread::hardware_concurrency();
  int rc = qd_model_fill_random(img.data(), bytes, cfg, seed, std, (int)std::min(16u, hw ? hw : 1u));
  if (rc != QD_OK) return rc;
  FILE* f = std::fopen(path, "wb");
  if (!f) return fail(QD_EINVAL, "cannot open %s for writing", path);
  const size_t n = std::fwrite(img.data(), 1, img.size(), f);
  const int cl = std::fclose(f);
  if (n != img.size() || cl != 0) return fail(QD_EINVAL, "short write to %s", path);
  return QD_OK;
}

int qd_engine_create_from_image(const void* image, long long bytes, qd_engine** out) {
  if (!out) return fail(QD_EINVAL, "out is NULL");
  *out = nullptr;
  if (!image || bytes < QD_MODEL_HEADER_BYTES) return fail(QD_EINVAL, "image too small for a header");
  uint32_t hdr[7];
  std::memcpy(hdr, image, sizeof(hdr));
  if (hdr[0] != QD_MODEL_MAGIC)
    return fail(QD_EINVAL, "magic number mismatch: expected 0x%08x, got 0x%08x", QD_MODEL_MAGIC, hdr[0]);
  qd_model_cfg cfg{hdr[1], hdr[2], hdr[3], hdr[4], hdr[5], hdr[6]};
  if (!cfg_valid(&cfg))
    return fail(QD_EINVAL, "unsupported configuration (vocab %u hidden %u layers %u heads %u inter %u max_seqlen %u)",
                cfg.vocab_size, cfg.hidden_size, cfg.num_layers, cfg.num_heads, cfg.intermediate_size,
                cfg.max_seqlen);
  if (bytes != qd_model_image_bytes(&cfg))
    return fail(QD_EINVAL, "image holds %lld bytes, its header describes %lld", bytes,
                qd_model_image_bytes(&cfg));
  qd_engine* e = new (std::nothrow) qd_engine;
  if (!e) return fail(QD_ENOMEM, "host allocation failed");
  e->cfg = cfg;
  e->lay = layout_of(cfg);
  const long long H = cfg.hidden_size, I = cfg.intermediate_size, V = cfg.vocab_size;
  hipError_t he = hipGetDevice(&e->device);
  if (he != hipSuccess) {
    engine_free(e);
    return hip_fail(he, "hipGetDevice");
  }
  const qd_cfg acfg = {(int)cfg.num_heads, QD_HEAD_DIM, (int)cfg.max_seqlen, H, QD_HEAD_DIM, 10000.0f};
  int rc = qd_ctx_create(&acfg, &e->attn);
  if (rc != QD_OK) {
    engine_free(e);
    return rc;
  }
  e->kv_bytes = (long long)cfg.num_layers * cfg.max_seqlen * H * 2;
  e->lm_ws_bytes = qd_lm_head_workspace_bytes((int)V);
  const long long wbytes = bytes - QD_MODEL_HEADER_BYTES;
  struct { void** p; long long n; } allocs[] = {
      {(void**)&e->weights, wbytes},  {(void**)&e->k_cache, e->kv_bytes}, {(void**)&e->v_cache, e->kv_bytes},
      {(void**)&e->x, H * 2},         {(void**)&e->qkv, 3 * H * 2},     {(void**)&e->attn_out, H * 2},
      {(void**)&e->act, I * 2},       {(void**)&e->logits, V * 2},      {&e->lm_ws, (long long)e->lm_ws_bytes},
      {(void**)&e->p_split, (long long)qd::kGemmSplitWsBytes}};
  for (auto& a : allocs) {
    if ((he = hipMalloc(a.p, (size_t)a.n)) != hipSuccess) {
      engine_free(e);
      return fail(QD_ENOMEM, "hipMalloc of %lld bytes failed: %s", a.n, hipGetErrorString(he));
    }
  }
  if ((rc = resize_prefill_scratch(e, std::min(kPrefillChunk, (int)cfg.max_seqlen))) != QD_OK) {
    engine_free(e);
    return rc;
  }
  // The next token goes straight from the argmax kernel into mapped pinned
  // memory: no device-to-host copy (a blit kernel of its own) per token.
  if ((he = hipHostMalloc((void**)&e->h_token, sizeof(int), hipHostMallocMapped)) != hipSuccess ||
      (he = hipHostGetDevicePointer((void**)&e->h_token_dev, e->h_token, 0)) != hipSuccess ||
      (he = hipStreamCreate(&e->stream)) != hipSuccess ||
      (he = hipMemcpy(e->weights, static_cast<const char*>(image) + QD_MODEL_HEADER_BYTES,
                      (size_t)wbytes, hipMemcpyHostToDevice)) != hipSuccess) {
    engine_free(e);
    return hip_fail(he, "engine setup");
  }
  if ((rc = qd_engine_reset(e)) != QD_OK) {
    engine_free(e);
    return rc;
  }
  *out = e;
  return QD_OK;
}

int qd_engine_create(const char* path, qd_engine** out) {
  if (!out) return fail(QD_EINVAL, "out is NULL");
  *out = nullptr;
  if (!path) return fail(QD_EINVAL, "path is NULL");
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return fail(QD_EINVAL, "cannot open model weights file %s", path);
  struct stat st;
  if (::fstat(fd, &st) != 0 || st.st_size < QD_MODEL_HEADER_BYTES) {
    ::close(fd);
    return fail(QD_EINVAL, "%s is too small for a model file", path);
  }
  void* m = ::mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return fail(QD_EINVAL, "cannot map %s", path);
  const int rc = qd_engine_create_from_image(m, (long long)st.st_size, out);
  ::munmap(m, (size_t)st.st_size);
  return rc;
}

int qd_engine_destroy(qd_engine* eng) {
  engine_free(eng);
  return QD_OK;
}

int qd_engine_config(const qd_engine* eng, qd_model_cfg* cfg) {
  if (!eng || !cfg) return fail(QD_EINVAL, "NULL argument");
  *cfg = eng->cfg;
  return QD_OK;
}

int qd_engine_reset(qd_engine* e) {
  int rc = check_engine(e);
  if (rc != QD_OK) return rc;
  const long long H = e->cfg.hidden_size;
  hipError_t he;
  if ((he = hipMemsetAsync(e->k_cache, 0, (size_t)e->kv_bytes, e->stream)) != hipSuccess ||
      (he = hipMemsetAsync(e->v_cache, 0, (size_t)e->kv_bytes, e->stream)) != hipSuccess ||
      (he = hipMemsetAsync(e->x, 0, (size_t)H * 2, e->stream)) != hipSuccess ||
      (he = hipMemsetAsync(e->qkv, 0, (size_t)H * 6, e->stream)) != hipSuccess ||
      (he = hipMemsetAsync(e->attn_out, 0, (size_t)H * 2, e->stream)) != hipSuccess ||
      (he = hipMemsetAsync(e->act, 0, (size_t)e->cfg.intermediate_size * 2, e->stream)) != hipSuccess ||
      (he = hipMemsetAsync(e->logits, 0, (size_t)e->cfg.vocab_size * 2, e->stream)) != hipSuccess ||
      (he = hipStreamSynchronize(e->stream)) != hipSuccess)
    return hip_fail(he, "engine reset");
  return QD_OK;
}

int qd_engine_set_prefill_mode(qd_engine* e, int mode) {
  if (!e) return fail(QD_EINVAL, "engine is NULL");
  if (mode != QD_GEMM_EXACT && mode != QD_GEMM_MFMA) return fail(QD_EINVAL, "unknown prefill mode %d", mode);
  const int cap = std::min(kPrefillChunkMfma, (int)e->cfg.max_seqlen);
  if (mode == QD_GEMM_MFMA && e->p_cap < cap) {
    int rc = check_engine(e);
    if (rc != QD_OK) return rc;
    const hipError_t he = hipStreamSynchronize(e->stream);
    if (he != hipSuccess) return hip_fail(he, "prefill mode");
    if ((rc = resize_prefill_scratch(e, cap)) != QD_OK) return rc;
  }
  e->prefill_mode = mode;
  return QD_OK;
}

int qd_engine_prefill(qd_engine* e, const int* tokens, int n, int* pos) {
  int rc = check_engine(e);
  if (rc != QD_OK) return rc;
  if (!pos || (n > 0 && !tokens) || n < 0) return fail(QD_EINVAL, "invalid tokens, n or pos");
  if (*pos < 0 || (long long)*pos + n > (long long)e->cfg.max_seqlen)
    return fail(QD_EINVAL, "positions [%d, %lld) exceed max_seqlen %u", *pos, (long long)*pos + n,
                e->cfg.max_seqlen);
  for (int i = 0; i < n; ++i)
    if (tokens[i] < 0 || (uint32_t)tokens[i] >= e->cfg.vocab_size)
      return fail(QD_EINVAL, "token %d outside [0, %u)", tokens[i], e->cfg.vocab_size);
  const int chunk = e->prefill_mode == QD_GEMM_MFMA ? e->p_cap : std::min(kPrefillChunk, e->p_cap);
  for (int i = 0; i < n; i += chunk) {
    const int T = std::min(chunk, n - i);
    if ((rc = prefill_batched(e, tokens + i, T, *pos + i)) != QD_OK) return rc;
    // the token upload of the next chunk reuses p_tokens: finish this chunk first
    hipError_t he = hipStreamSynchronize(e->stream);
    if (he != hipSuccess) return hip_fail(he, "prefill");
  }
  hipError_t he = hipStreamSynchronize(e->stream);
  if (he != hipSuccess) return hip_fail(he, "prefill");
  *pos += n;
  return QD_OK;
}

int qd_engine_step(qd_engine* e, int token, int pos, int* next_token) {
  int rc = check_engine(e);
  if (rc != QD_OK) return rc;
  if (!next_token) return fail(QD_EINVAL, "next_token is NULL");
  if (token < 0 || (uint32_t)token >= e->cfg.vocab_size)
    return fail(QD_EINVAL, "token %d outside [0, %u)", token, e->cfg.vocab_size);
  if (pos < 0 || (uint32_t)pos >= e->cfg.max_seqlen)
    return fail(QD_EINVAL, "pos %d outside [0, %u)", pos, e->cfg.max_seqlen);
  if ((rc = run_layers(e, token, pos)) != QD_OK) return rc;
  rc = qd_lm_head_argmax(e->x, e->w(e->lay.ln_f), kEps, e->w(e->lay.lm_head), e->logits,
                         (int)e->cfg.vocab_size, (int)e->cfg.hidden_size, e->lm_ws, e->lm_ws_bytes,
                         e->h_token_dev, e->stream);
  if (rc != QD_OK) return rc;
  const hipError_t he = hipStreamSynchronize(e->stream);
  if (he != hipSuccess) return hip_fail(he, "decode step");
  *next_token = *static_cast<volatile int*>(e->h_token);
  return QD_OK;
}

int qd_engine_logits(qd_engine* e, uint16_t* host_logits) {
  int rc = check_engine(e);
  if (rc != QD_OK) return rc;
  if (!host_logits) return fail(QD_EINVAL, "host_logits is NULL");
  hipError_t he = hipMemcpy(host_logits, e->logits, (size_t)e->cfg.vocab_size * 2, hipMemcpyDeviceToHost);
  return he == hipSuccess ? QD_OK : hip_fail(he, "logits copy");
}

int qd_engine_kv_rows(qd_engine* e, int layer, int pos0, int n, uint16_t* host_k, uint16_t* host_v) {
  int rc = check_engine(e);
  if (rc != QD_OK) return rc;
  if (layer < 0 || (uint32_t)layer >= e->cfg.num_layers || pos0 < 0 || n < 0 ||
      (long long)pos0 + n > (long long)e->cfg.max_seqlen)
    return fail(QD_EINVAL, "rows [%d, %lld) of layer %d outside the cache (%u layers, %u rows)", pos0,
                (long long)pos0 + n, layer, e->cfg.num_layers, e->cfg.max_seqlen);
  hipError_t he = hipStreamSynchronize(e->stream);
  const size_t off = (size_t)pos0 * e->cfg.hidden_size, bytes = (size_t)n * e->cfg.hidden_size * 2;
  if (he == hipSuccess && host_k && n) he = hipMemcpy(host_k, e->kc(layer) + off, bytes, hipMemcpyDeviceToHost);
  if (he == hipSuccess && host_v && n) he = hipMemcpy(host_v, e->vc(layer) + off, bytes, hipMemcpyDeviceToHost);
  return he == hipSuccess ? QD_OK : hip_fail(he, "KV rows copy");
}

int qd_engine_generate(qd_engine* e, const int* prompt, int n_prompt, int max_new, int stop_at_eos,
                       int* out_tokens, int* n_out) {
  int rc = check_engine(e);
  if (rc != QD_OK) return rc;
  if (!prompt || n_prompt < 1 || max_new < 0 || (max_new > 0 && !out_tokens) || !n_out)
    return fail(QD_EINVAL, "invalid prompt, max_new or outputs");
  *n_out = 0;
  int pos = 0;
  if (n_prompt > 1 && (rc = qd_engine_prefill(e, prompt, n_prompt - 1, &pos)) != QD_OK) return rc;
  int last = prompt[n_prompt - 1];
  for (int i = 0; i < max_new && (uint32_t)pos < e->cfg.max_seqlen; ++i) {
    int next = 0;
    if ((rc = qd_engine_step(e, last, pos, &next)) != QD_OK) return rc;
    ++pos;
    if (stop_at_eos && (next == kEosA || next == kEosB)) break;
    out_tokens[(*n_out)++] = next;
    last = next;
  }
  return QD_OK;
}

}  // extern "C"
