/*
 * qd_oracle_model.c -- CPU restatement of the whole greedy decode step in the
 * order of this build's gfx950 kernels: the decode-step ops of
 * include/qdiy/decode.h and the engine of include/qdiy/engine.h.
 *
 * TEST INFRASTRUCTURE ONLY: this file is a checker.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the product
 * library never links or calls it.  Built with -ffp-contract=off: each
 * `a*b + c` rounds twice, fmaf() once.
 *
 * Reference call sites restated (framework_src/qwen_infer.cu):
 *   :617       embedding row
 *   :626-642   RMSNorm, QKV GEMV, bias, RoPE, KV append (qd_oracle_qkv_front)
 *   :644-678   decode attention (qd_oracle_attention_planned)
 *   :701-704   o-proj GEMV + residual          (qd_oracle_proj_residual)
 *   :708-715   RMSNorm, W1/W2 GEMVs, SwiGLU    (qd_oracle_ffn_up_swiglu)
 *   :718-721   c_proj GEMV + residual          (qd_oracle_proj_residual)
 *   :725-731   RMSNorm, lm_head GEMV, argmax   (qd_oracle_lm_head_argmax)
 *   :780-817   prompt + greedy generation loop (qd_oracle_generate)
 * with the reduction order of the gfx950 kernels (QD_ORDER_WAVE64 in
 * qd_oracle.h) instead of the reference's, the exp of SwiGLU taken as
 * qd_oracle_exp2(-u * log2 e) instead of __expf, and argmax ties broken by the
 * lowest index.  Each of those is pinned on its own in tests/ against the
 * reference-order functions and float64.
 *
 * A model made with order QD_ORDER_REF instead follows the reference kernels'
 * own arithmetic throughout: the 512-thread RMSNorm (rmsnorm.cuh:15-45), GEMV
 * sums with k ascending (hgemm_final.cuh:278-293), the engine's attention
 * dispatch with fp16 partials (qd_oracle_decode_attention, QD_ORACLE_ENGINE:
 * qwen_infer.cu:646-678), SwiGLU as w1 * (w2 / (1 + exp(-w2)))
 * (swiglu.cuh:11-13, with glibc expf and an IEEE division where the
 * reference's fast-math build uses __expf and an approximate division), and
 * argmax_kernel's tie order (argmax.cuh:7-72: per-thread chunks of
 * ceil(V/512) ids, first maximum in a chunk, then xor-butterflies that keep
 * their own value on ties).
 */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "qd_oracle.h"

/* ------------------------------------------------------------------------ */
/* fp16 -> fp32 by table (exact: built from qd_oracle_h2f)                   */

static float g_h2f[65536];
static pthread_once_t g_h2f_once = PTHREAD_ONCE_INIT;

static void h2f_init(void) {
  for (int i = 0; i < 65536; ++i) g_h2f[i] = qd_oracle_h2f((uint16_t)i);
}

static const float* h2f_table(void) {
  pthread_once(&g_h2f_once, h2f_init);
  return g_h2f;
}

/* ------------------------------------------------------------------------ */
/* A persistent pool: run fn(arg, i) for i in [0, n) on nthreads threads.    */

typedef struct pool pool;
typedef void (*pool_fn)(void* arg, int i);

struct pool {
  int nthreads;
  pthread_t* th;
  pthread_mutex_t mu;
  pthread_cond_t go, done;
  pool_fn fn;
  void* arg;
  int n, next, active, generation, quit;
};

static void pool_work(pool* p) {
  for (;;) {
    int i = __atomic_fetch_add(&p->next, 1, __ATOMIC_RELAXED);
    if (i >= p->n) break;
    p->fn(p->arg, i);
  }
}

static void* pool_main(void* a) {
  pool* p = (pool*)a;
  int seen = 0;
  pthread_mutex_lock(&p->mu);
  for (;;) {
    while (!p->quit && p->generation == seen) pthread_cond_wait(&p->go, &p->mu);
    if (p->quit) break;
    seen = p->generation;
    pthread_mutex_unlock(&p->mu);
    pool_work(p);
    pthread_mutex_lock(&p->mu);
    if (--p->active == 0) pthread_cond_signal(&p->done);
  }
  pthread_mutex_unlock(&p->mu);
  return NULL;
}

static pool* pool_new(int nthreads) {
  pool* p = (pool*)calloc(1, sizeof(pool));
  if (!p) return NULL;
  p->nthreads = nthreads < 1 ? 1 : (nthreads > 256 ? 256 : nthreads);
  pthread_mutex_init(&p->mu, NULL);
  pthread_cond_init(&p->go, NULL);
  pthread_cond_init(&p->done, NULL);
  p->th = (pthread_t*)calloc((size_t)p->nthreads, sizeof(pthread_t));
  int started = 0;
  for (int i = 1; i < p->nthreads; ++i)
    if (pthread_create(&p->th[i], NULL, pool_main, p) == 0) started = i;
    else break;
  p->nthreads = started + 1;
  return p;
}

static void pool_run(pool* p, pool_fn fn, void* arg, int n) {
  if (p->nthreads == 1 || n <= 1) {
    for (int i = 0; i < n; ++i) fn(arg, i);
    return;
  }
  pthread_mutex_lock(&p->mu);
  p->fn = fn;
  p->arg = arg;
  p->n = n;
  p->next = 0;
  p->active = p->nthreads - 1;
  p->generation++;
  pthread_cond_broadcast(&p->go);
  pthread_mutex_unlock(&p->mu);
  pool_work(p);
  pthread_mutex_lock(&p->mu);
  while (p->active > 0) pthread_cond_wait(&p->done, &p->mu);
  pthread_mutex_unlock(&p->mu);
}

static void pool_free(pool* p) {
  if (!p) return;
  pthread_mutex_lock(&p->mu);
  p->quit = 1;
  pthread_cond_broadcast(&p->go);
  pthread_mutex_unlock(&p->mu);
  for (int i = 1; i < p->nthreads; ++i) pthread_join(p->th[i], NULL);
  pthread_mutex_destroy(&p->mu);
  pthread_cond_destroy(&p->go);
  pthread_cond_destroy(&p->done);
  free(p->th);
  free(p);
}

/* ------------------------------------------------------------------------ */
/* GEMV rows in the wave64 order                                             */

/* sum_k xf[k] * W[row][k]: lane l adds k = 512j + 8l + e (j, then e
 * ascending, k < K) sequentially; the 64 lanes by qd_oracle_wave64_sum. */
static float row_wave64(const float* xf, const uint16_t* w_row, int K, const float* T) {
  float lanes[64];
  for (int l = 0; l < 64; ++l) lanes[l] = 0.0f;
  const int nfull = K / 512, rem = K % 512;
  for (int j = 0; j < nfull; ++j) {
    const uint16_t* wj = w_row + 512 * j;
    const float* xj = xf + 512 * j;
    for (int l = 0; l < 64; ++l) {
      const uint16_t* wl = wj + 8 * l;
      const float* xl = xj + 8 * l;
      float a = lanes[l];
      for (int e = 0; e < 8; ++e) a += xl[e] * T[wl[e]];   /* exact product, one rounding */
      lanes[l] = a;
    }
  }
  for (int l = 0; 8 * l < rem; ++l) {
    const uint16_t* wl = w_row + 512 * nfull + 8 * l;
    const float* xl = xf + 512 * nfull + 8 * l;
    float a = lanes[l];
    for (int e = 0; e < 8; ++e) a += xl[e] * T[wl[e]];
    lanes[l] = a;
  }
  return qd_oracle_wave64_sum(lanes);
}

/* sum_k xf[k] * W[row][k] with k ascending, one rounding per add: the
 * reference's hgemv_kernel (hgemm_final.cuh:278-293; products of two fp16
 * values are exact in fp32, so contraction cannot change them). */
static float row_seq(const float* xf, const uint16_t* w_row, int K, const float* T) {
  float s = 0.0f;
  for (int k = 0; k < K; ++k) s += xf[k] * T[w_row[k]];
  return s;
}

typedef struct {
  const float* xf;
  const uint16_t* W;
  int K;
  float* out;           /* fp32 row sums */
  int rows_per_task, n;
  int order;            /* QD_ORDER_WAVE64 or QD_ORDER_REF */
} gemv_job;

static void gemv_task(void* a, int t) {
  gemv_job* j = (gemv_job*)a;
  const float* T = h2f_table();
  const int b = t * j->rows_per_task;
  const int e = b + j->rows_per_task < j->n ? b + j->rows_per_task : j->n;
  for (int r = b; r < e; ++r)
    j->out[r] = j->order == QD_ORDER_REF ? row_seq(j->xf, j->W + (long long)r * j->K, j->K, T)
                                         : row_wave64(j->xf, j->W + (long long)r * j->K, j->K, T);
}

static void gemv_sums_order(pool* p, const float* xf, const uint16_t* W, int N, int K, float* out,
                            int order) {
  gemv_job j = {xf, W, K, out, 64, N, order};
  pool_run(p, gemv_task, &j, (N + 63) / 64);
}


static void to_float(const uint16_t* h, float* f, int n) {
  const float* T = h2f_table();
  for (int i = 0; i < n; ++i) f[i] = T[h[i]];
}

/* ------------------------------------------------------------------------ */
/* Decode-step ops                                                           */

static void proj_residual_pool(pool* p, const uint16_t* x, const uint16_t* W,
                               const uint16_t* residual, uint16_t* out, int n_out, int k_in,
                               int order) {
  float* xf = (float*)malloc(sizeof(float) * (size_t)k_in);
  float* s = (float*)malloc(sizeof(float) * (size_t)n_out);
  to_float(x, xf, k_in);
  gemv_sums_order(p, xf, W, n_out, k_in, s, order);
  for (int n = 0; n < n_out; ++n)
    out[n] = qd_oracle_f2h(qd_oracle_h2f(residual[n]) + qd_oracle_h2f(qd_oracle_f2h(s[n])));
  free(s);
  free(xf);
}

static uint16_t swiglu(float gsum, float usum) {
  const float g = qd_oracle_h2f(qd_oracle_f2h(gsum));
  const float u = qd_oracle_h2f(qd_oracle_f2h(usum));
  const float e = qd_oracle_exp2(-u * 1.44269504088896340736f);
  const float silu = u / (1.0f + e);
  return qd_oracle_f2h(g * silu);
}

/* swiglu.cuh:11-13: out = half(w1 * (w2 / (1 + exp(-w2)))) of the fp16 GEMV
 * outputs, exp as glibc expf. */
static uint16_t swiglu_ref(float gsum, float usum) {
  const float g = qd_oracle_h2f(qd_oracle_f2h(gsum));
  const float u = qd_oracle_h2f(qd_oracle_f2h(usum));
  const float silu = u / (1.0f + expf(-u));
  return qd_oracle_f2h(g * silu);
}

static void ffn_up_pool(pool* p, const uint16_t* x, const uint16_t* norm_w, float eps,
                        const uint16_t* w1, const uint16_t* w2, uint16_t* act, int hidden,
                        int inter, int order) {
  uint16_t* xn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)hidden);
  float* xf = (float*)malloc(sizeof(float) * (size_t)hidden);
  float* g = (float*)malloc(sizeof(float) * (size_t)inter);
  float* u = (float*)malloc(sizeof(float) * (size_t)inter);
  qd_oracle_rmsnorm(x, norm_w, hidden, eps, xn, order);
  to_float(xn, xf, hidden);
  gemv_sums_order(p, xf, w1, inter, hidden, g, order);
  gemv_sums_order(p, xf, w2, inter, hidden, u, order);
  for (int i = 0; i < inter; ++i) act[i] = order == QD_ORDER_REF ? swiglu_ref(g[i], u[i]) : swiglu(g[i], u[i]);
  free(u);
  free(g);
  free(xf);
  free(xn);
}

static unsigned long long argmax_key(uint16_t b, int row) {
  if (b == 0x8000u) b = 0;
  unsigned int k;
  if ((b & 0x7FFFu) > 0x7C00u) k = 0;
  else k = (b & 0x8000u) ? (~(unsigned)b & 0xFFFFu) : ((unsigned)b | 0x8000u);
  return ((unsigned long long)k << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)row);
}

/* argmax_kernel<<<1, 512>>> (argmax.cuh:7-72): thread t scans ids
 * [t*c, t*c + c), c = ceil(V/512), keeping the first strictly larger value;
 * each 32-lane warp then runs xor-butterflies (masks 16..1) in which a lane
 * takes its partner's (value, id) only when strictly larger; warp w's lane 0
 * result goes to slot w, and warp 0 repeats the butterfly over slots 0..15
 * (-inf, id -1 beyond).  Thread 0's id is the token.  NaN never wins (every
 * comparison with it is false); -1 if no value exceeds -inf. */
static int argmax_ref(const uint16_t* logits, int vocab) {
  enum { kThreads = 512, kWarps = 16 };
  const int c = (vocab + kThreads - 1) / kThreads;
  float val[kThreads];
  int idx[kThreads];
  for (int t = 0; t < kThreads; ++t) {
    val[t] = -INFINITY;
    idx[t] = -1;
    for (int i = 0; i < c; ++i) {
      const int id = t * c + i;
      if (id < vocab) {
        const float v = qd_oracle_h2f(logits[id]);
        if (v > val[t]) { val[t] = v; idx[t] = id; }
      }
    }
  }
  float sv[32];
  int si[32];
  for (int w = 0; w < kWarps; ++w) {
    float* v = val + 32 * w;
    int* x = idx + 32 * w;
    for (int mask = 16; mask >= 1; mask >>= 1) {
      float nv[32];
      int ni[32];
      for (int l = 0; l < 32; ++l) {
        nv[l] = v[l]; ni[l] = x[l];
        if (v[l ^ mask] > v[l]) { nv[l] = v[l ^ mask]; ni[l] = x[l ^ mask]; }
      }
      memcpy(v, nv, sizeof(nv));
      memcpy(x, ni, sizeof(ni));
    }
    sv[w] = v[0];
    si[w] = x[0];
  }
  for (int l = kWarps; l < 32; ++l) { sv[l] = -INFINITY; si[l] = -1; }
  for (int mask = 16; mask >= 1; mask >>= 1) {
    float nv[32];
    int ni[32];
    for (int l = 0; l < 32; ++l) {
      nv[l] = sv[l]; ni[l] = si[l];
      if (sv[l ^ mask] > sv[l]) { nv[l] = sv[l ^ mask]; ni[l] = si[l ^ mask]; }
    }
    memcpy(sv, nv, sizeof(nv));
    memcpy(si, ni, sizeof(ni));
  }
  return si[0];
}

int qd_oracle_argmax_ref(const uint16_t* logits, int vocab) {
  if (!logits || vocab < 1) return -1;
  return argmax_ref(logits, vocab);
}

uint16_t qd_oracle_swiglu_ref(uint16_t g, uint16_t u) {
  return swiglu_ref(qd_oracle_h2f(g), qd_oracle_h2f(u));
}

static int lm_head_pool(pool* p, const uint16_t* x, const uint16_t* norm_w, float eps,
                        const uint16_t* W, uint16_t* logits, int vocab, int hidden, int order) {
  uint16_t* xn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)hidden);
  float* xf = (float*)malloc(sizeof(float) * (size_t)hidden);
  float* s = (float*)malloc(sizeof(float) * (size_t)vocab);
  qd_oracle_rmsnorm(x, norm_w, hidden, eps, xn, order);
  to_float(xn, xf, hidden);
  gemv_sums_order(p, xf, W, vocab, hidden, s, order);
  if (order == QD_ORDER_REF) {
    uint16_t* lg = logits ? logits : (uint16_t*)malloc(sizeof(uint16_t) * (size_t)vocab);
    for (int v = 0; v < vocab; ++v) lg[v] = qd_oracle_f2h(s[v]);
    const int t = argmax_ref(lg, vocab);
    if (!logits) free(lg);
    free(s);
    free(xf);
    free(xn);
    return t;
  }
  unsigned long long best = 0;
  for (int v = 0; v < vocab; ++v) {
    const uint16_t h = qd_oracle_f2h(s[v]);
    if (logits) logits[v] = h;
    const unsigned long long k = argmax_key(h, v);
    if (k > best) best = k;
  }
  free(s);
  free(xf);
  free(xn);
  return (int)(0xFFFFFFFFu - (unsigned)(best & 0xFFFFFFFFull));
}

void qd_oracle_proj_residual(const uint16_t* x, const uint16_t* W, const uint16_t* residual,
                             uint16_t* out, int n_out, int k_in, int nthreads) {
  pool* p = pool_new(nthreads);
  proj_residual_pool(p, x, W, residual, out, n_out, k_in, QD_ORDER_WAVE64);
  pool_free(p);
}

void qd_oracle_ffn_up_swiglu(const uint16_t* x, const uint16_t* norm_w, float eps,
                             const uint16_t* w1, const uint16_t* w2, uint16_t* act, int hidden,
                             int inter, int nthreads) {
  pool* p = pool_new(nthreads);
  ffn_up_pool(p, x, norm_w, eps, w1, w2, act, hidden, inter, QD_ORDER_WAVE64);
  pool_free(p);
}

uint16_t qd_oracle_swiglu(uint16_t g, uint16_t u) {
  return swiglu(qd_oracle_h2f(g), qd_oracle_h2f(u));
}

int qd_oracle_lm_head_argmax(const uint16_t* x, const uint16_t* norm_w, float eps,
                             const uint16_t* W, uint16_t* logits, int vocab, int hidden,
                             int nthreads) {
  pool* p = pool_new(nthreads);
  const int t = lm_head_pool(p, x, norm_w, eps, W, logits, vocab, hidden, QD_ORDER_WAVE64);
  pool_free(p);
  return t;
}

/* ------------------------------------------------------------------------ */
/* The model                                                                 */

typedef struct {
  long long ln_1, qkv_w, qkv_b, proj_w, ln_2, w1, w2, w_down;
} layer_off;

struct qd_oracle_model {
  long long V, H, NL, NH, I;
  int max_pos;
  const uint16_t* t;            /* tensor data of the image (not copied) */
  layer_off* lo;
  const uint16_t *wte, *ln_f, *lm_head;
  long long layer_cache;
  uint16_t *kc, *vc, *x, *qkv, *attn, *act, *xn, *logits;
  float *xf, *sums;
  pool* p;
  int order;                    /* QD_ORDER_WAVE64 or QD_ORDER_REF */
};

void qd_oracle_model_free(qd_oracle_model* m) {
  if (!m) return;
  pool_free(m->p);
  free(m->logits);
  free(m->sums);
  free(m->xf);
  free(m->xn);
  free(m->act);
  free(m->attn);
  free(m->qkv);
  free(m->x);
  free(m->vc);
  free(m->kc);
  free(m->lo);
  free(m);
}

qd_oracle_model* qd_oracle_model_new(const void* image, long long bytes, int max_pos, int nthreads) {
  return qd_oracle_model_new_order(image, bytes, max_pos, nthreads, QD_ORDER_WAVE64);
}

qd_oracle_model* qd_oracle_model_new_order(const void* image, long long bytes, int max_pos,
                                           int nthreads, int order) {
  if (!image || bytes < 28 || max_pos < 1) return NULL;
  if (order != QD_ORDER_WAVE64 && order != QD_ORDER_REF) return NULL;
  uint32_t hdr[7];
  memcpy(hdr, image, sizeof(hdr));
  if (hdr[0] != 0x46445751u) return NULL;
  const long long V = hdr[1], H = hdr[2], NL = hdr[3], NH = hdr[4], I = hdr[5];
  if (H != NH * 128 || H % 512 != 0 || I % 8 != 0 || I < 8 || V < 1 || NL < 1) return NULL;
  const long long per_layer = H + 3 * H * H + 3 * H + H * H + H + 2 * I * H + H * I;
  if (bytes != 28 + 2 * (V * H + NL * per_layer + H + V * H) || max_pos > (int)hdr[6]) return NULL;
  qd_oracle_model* m = (qd_oracle_model*)calloc(1, sizeof(qd_oracle_model));
  if (!m) return NULL;
  m->V = V; m->H = H; m->NL = NL; m->NH = NH; m->I = I; m->max_pos = max_pos; m->order = order;
  m->t = (const uint16_t*)((const char*)image + 28);
  m->lo = (layer_off*)malloc(sizeof(layer_off) * (size_t)NL);
  long long o = V * H;
  for (long long l = 0; l < NL; ++l) {
    m->lo[l].ln_1 = o;   o += H;
    m->lo[l].qkv_w = o;  o += 3 * H * H;
    m->lo[l].qkv_b = o;  o += 3 * H;
    m->lo[l].proj_w = o; o += H * H;
    m->lo[l].ln_2 = o;   o += H;
    m->lo[l].w1 = o;     o += I * H;
    m->lo[l].w2 = o;     o += I * H;
    m->lo[l].w_down = o; o += H * I;
  }
  m->wte = m->t;
  m->ln_f = m->t + o;
  m->lm_head = m->t + o + H;
  m->layer_cache = (long long)max_pos * H;
  m->kc = (uint16_t*)calloc((size_t)(NL * m->layer_cache), sizeof(uint16_t));
  m->vc = (uint16_t*)calloc((size_t)(NL * m->layer_cache), sizeof(uint16_t));
  m->x = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)H);
  m->qkv = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(3 * H));
  m->attn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)H);
  m->act = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)I);
  m->xn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)H);
  m->xf = (float*)malloc(sizeof(float) * (size_t)H);
  m->sums = (float*)malloc(sizeof(float) * (size_t)(3 * H));
  m->logits = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)V);
  m->p = pool_new(nthreads);
  if (!m->lo || !m->kc || !m->vc || !m->x || !m->qkv || !m->attn || !m->act || !m->xn || !m->xf ||
      !m->sums || !m->logits || !m->p) {
    qd_oracle_model_free(m);
    return NULL;
  }
  return m;
}

int qd_oracle_model_forward(qd_oracle_model* m, int token, int pos, const qd_oracle_plan* plan,
                            int want_logits, uint16_t* logits_out) {
  if (!m || (!plan && m->order != QD_ORDER_REF) || token < 0 || token >= m->V || pos < 0 ||
      pos >= m->max_pos)
    return -1;
  const int order = m->order;
  const long long H = m->H, NH = m->NH, I = m->I;
  const float eps = 1e-6f;
  const uint16_t* t = m->t;
  const uint16_t* xin = m->wte + (long long)token * H;                 /* :617 */
  for (long long l = 0; l < m->NL; ++l) {
    const layer_off* f = &m->lo[l];
    uint16_t* K = m->kc + l * m->layer_cache;
    uint16_t* Vv = m->vc + l * m->layer_cache;
    /* front end: RMSNorm(ln_1), QKV GEMV, bias, RoPE, append (:626-642) */
    qd_oracle_rmsnorm(xin, t + f->ln_1, (int)H, eps, m->xn, order);
    to_float(m->xn, m->xf, (int)H);
    gemv_sums_order(m->p, m->xf, t + f->qkv_w, (int)(3 * H), (int)H, m->sums, order);
    for (long long n = 0; n < 3 * H; ++n) m->qkv[n] = qd_oracle_f2h(m->sums[n]);
    qd_oracle_qkv_bias_rope_cache(m->qkv, t + f->qkv_b, K, Vv, pos, (int)NH, 128, H, 128, 10000.0f);
    const int rc = order == QD_ORDER_REF
                       ? qd_oracle_decode_attention(m->qkv, K, Vv, m->attn, pos + 1, (int)NH, H, 128,
                                                    QD_ORACLE_ENGINE, 1)
                       : qd_oracle_attention_planned(m->qkv, K, Vv, m->attn, pos + 1, (int)NH, H, 128,
                                                     plan, 1);
    if (rc != 0) return -1;
    proj_residual_pool(m->p, m->attn, t + f->proj_w, xin, m->x, (int)H, (int)H, order);
    ffn_up_pool(m->p, m->x, t + f->ln_2, eps, t + f->w1, t + f->w2, m->act, (int)H, (int)I, order);
    proj_residual_pool(m->p, m->act, t + f->w_down, m->x, m->x, (int)H, (int)I, order);
    xin = m->x;
  }
  if (!want_logits) return 0;
  const int next =
      lm_head_pool(m->p, m->x, m->ln_f, eps, m->lm_head, m->logits, (int)m->V, (int)H, order);
  if (logits_out) memcpy(logits_out, m->logits, sizeof(uint16_t) * (size_t)m->V);
  return next;
}

int qd_oracle_generate(const void* image, long long bytes, const int* prompt, int n_prompt,
                       int n_new, int stop_at_eos, const qd_oracle_plan* plans, int n_plans,
                       int* out_tokens, int* n_out, uint16_t* last_logits, int nthreads) {
  if (!prompt || n_prompt < 1 || n_new < 0 || !n_out || !plans) return -1;
  const int max_pos = n_prompt + n_new;
  if (n_plans < max_pos) return -1;
  qd_oracle_model* m = qd_oracle_model_new(image, bytes, max_pos, nthreads);
  if (!m) return -1;
  int count = 0, pos = 0, last = prompt[n_prompt - 1], rc = 0;
  for (int i = 0; i < n_prompt - 1 && rc == 0; ++i, ++pos)
    rc = qd_oracle_model_forward(m, prompt[i], pos, &plans[pos], 0, NULL);
  for (int i = 0; i < n_new && rc >= 0; ++i) {
    const int next = qd_oracle_model_forward(m, last, pos, &plans[pos], 1, last_logits);
    ++pos;
    if (next < 0) { rc = -1; break; }
    if (stop_at_eos && (next == 151645 || next == 151643)) break;
    if (out_tokens) out_tokens[count] = next;
    ++count;
    last = next;
  }
  *n_out = count;
  qd_oracle_model_free(m);
  return rc < 0 ? -1 : 0;
}
