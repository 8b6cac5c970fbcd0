/*
 * qd_oracle.c -- CPU fp32 restatement of the reference decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY: this file is the checker.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The
 * product library (llm-inference-diy_amd/) never links or calls it.
 *
 * Must be compiled with -ffp-contract=off (see oracle/Makefile) so that every
 * `a*b + c` below rounds twice, exactly as written; fmaf() marks the places
 * where the reference itself calls __fmaf_rn.
 *
 * Warp-level structure is simulated explicitly: a "warp" is 32 lanes, lane l
 * owns dims 4l..4l+3 of the 128-dim head (flash_decode_q1_opt.cuh:442,454),
 * and the dot product is an xor butterfly over masks 16,8,4,2,1
 * (flash_decode_q1_opt.cuh:479-481).
 */
#include "qd_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QD_D 128
#define QD_LANES 32
#define QD_DPT (QD_D / QD_LANES) /* 4 dims per lane */

/* ------------------------------------------------------------------------ */
/* binary16 conversions                                                      */
/* ------------------------------------------------------------------------ */

float qd_oracle_h2f(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t man = (uint32_t)h & 0x3ffu;
  uint32_t bits;
  float f;
  if (exp == 0) {
    /* zero or subnormal: value = man * 2^-24, exact in binary32 */
    f = ldexpf((float)man, -24);
    return sign ? -f : f;
  }
  if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp - 15u + 127u) << 23) | (man << 13);
  }
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t qd_oracle_f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {            /* inf / nan */
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  }
  if (ax >= 0x477ff000u) {            /* >= 65520 rounds to inf */
    return (uint16_t)(sign | 0x7c00u);
  }
  if (ax >= 0x38800000u) {            /* normal binary16 range, >= 2^-14 */
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry may bump exponent: still correct */
    return (uint16_t)(sign | h);
  }
  /* binary16 subnormal or zero: m = RNE(|f| * 2^24) */
  {
    uint32_t e = ax >> 23;
    if (e == 0) return (uint16_t)sign;  /* binary32 subnormal: far below 2^-25 */
    uint32_t M = (ax & 0x7fffffu) | 0x800000u; /* value = M * 2^(e-150) */
    uint32_t shift = 126u - e;                 /* m = M >> shift (>= 14 here) */
    if (shift >= 25u) return (uint16_t)sign;   /* < 2^-25 (or == 2^-25 tie -> even 0) */
    uint32_t m = M >> shift;
    uint32_t rem = M & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1u);
    if (rem > halfway || (rem == halfway && (m & 1u))) m++;
    return (uint16_t)(sign | m);
  }
}

void qd_oracle_h2f_array(const uint16_t* in, float* out, long long n) {
  for (long long i = 0; i < n; ++i) out[i] = qd_oracle_h2f(in[i]);
}

void qd_oracle_f2h_array(const float* in, uint16_t* out, long long n) {
  for (long long i = 0; i < n; ++i) out[i] = qd_oracle_f2h(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Flash-Decoding v5 restatement                                             */
/* ------------------------------------------------------------------------ */

typedef struct {
  float m;          /* row_max  */
  float l;          /* row_sum  */
  float o[QD_D];    /* O_acc of all 32 lanes, lane l at [4l, 4l+4) */
} warp_state;

/* 1/sqrt(128) as __frcp_rn(sqrtf(128)) (flash_decode_q1_opt.cuh:459,575). */
static float fd_scale(void) { return 1.0f / sqrtf((float)QD_D); }

/* The per-warp row loop of fd_v5_fused_kernel (flash_decode_q1_opt.cuh:460-497)
 * and fd_v5_split_stage1_kernel (:576-611): rows [r_begin, r_end). */
static void warp_scan(const float* qf, const uint16_t* k, const uint16_t* v,
                      long long row_stride, int r_begin, int r_end, float scale,
                      warp_state* st) {
  st->m = -INFINITY;
  st->l = 0.0f;
  for (int d = 0; d < QD_D; ++d) st->o[d] = 0.0f;
  for (int row = r_begin; row < r_end; ++row) {
    const uint16_t* kr = k + (long long)row * row_stride;
    const uint16_t* vr = v + (long long)row * row_stride;
    float lane[QD_LANES], tmp[QD_LANES];
    for (int ln = 0; ln < QD_LANES; ++ln) {
      float dot = 0.0f;
      for (int i = 0; i < QD_DPT; ++i)
        dot = fmaf(qf[ln * QD_DPT + i], qd_oracle_h2f(kr[ln * QD_DPT + i]), dot);
      lane[ln] = dot;
    }
    for (int mask = 16; mask >= 1; mask >>= 1) {   /* dot += shfl_xor(dot, mask) */
      for (int ln = 0; ln < QD_LANES; ++ln) tmp[ln] = lane[ln] + lane[ln ^ mask];
      memcpy(lane, tmp, sizeof(lane));
    }
    float score = lane[0] * scale;
    float m_new = fmaxf(st->m, score);
    float exp_diff = expf(st->m - m_new);
    float p = expf(score - m_new);
    st->l = fmaf(st->l, exp_diff, p);
    for (int d = 0; d < QD_D; ++d)
      st->o[d] = fmaf(st->o[d], exp_diff, p * qd_oracle_h2f(vr[d]));
    st->m = m_new;
  }
}

/* SMEM merge of the warps, in warp order (flash_decode_q1_opt.cuh:509-526,
 * :623-642): returns global max, total sum and the merged unnormalised O. */
static void block_merge(const warp_state* ws, int nw, float* gmax_out,
                        float* tsum_out, float* o) {
  float gmax = -INFINITY;
  for (int w = 0; w < nw; ++w) gmax = fmaxf(gmax, ws[w].m);
  float tsum = 0.0f;
  for (int d = 0; d < QD_D; ++d) o[d] = 0.0f;
  for (int w = 0; w < nw; ++w) {
    float rescale = expf(ws[w].m - gmax);
    tsum += ws[w].l * rescale;
    for (int d = 0; d < QD_D; ++d) o[d] = fmaf(rescale, ws[w].o[d], o[d]);
  }
  *gmax_out = gmax;
  *tsum_out = tsum;
}

static void load_q(const uint16_t* q, float* qf) {
  for (int d = 0; d < QD_D; ++d) qf[d] = qd_oracle_h2f(q[d]);
}

void qd_oracle_fd_fused_head(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             uint16_t* out, int seqlen, long long row_stride,
                             int rows_per_warp, int num_warps) {
  float qf[QD_D], o[QD_D], gmax, tsum;
  const float scale = fd_scale();
  warp_state* ws = (warp_state*)malloc(sizeof(warp_state) * (size_t)num_warps);
  load_q(q, qf);
  for (int w = 0; w < num_warps; ++w) {
    int start = w * rows_per_warp;                 /* :465-469 */
    int end = start + rows_per_warp;
    if (end > seqlen) end = seqlen;
    if (start >= seqlen) end = start;              /* empty warp: -inf, 0, 0 */
    warp_scan(qf, k, v, row_stride, start, end, scale, &ws[w]);
  }
  block_merge(ws, num_warps, &gmax, &tsum, o);
  float inv_sum = 1.0f / tsum;                     /* __frcp_rn, :530 */
  for (int d = 0; d < QD_D; ++d) out[d] = qd_oracle_f2h(o[d] * inv_sum);
  free(ws);
}

/* Stage 1 for one chunk (flash_decode_q1_opt.cuh:548-656). */
static void split_stage1_chunk(const float* qf, const uint16_t* k, const uint16_t* v,
                               long long row_stride, int seqlen, int chunk_id,
                               int chunk, int warps, uint16_t* part, float* lse) {
  float o[QD_D], gmax, tsum;
  const float scale = fd_scale();
  const int rows_per_warp = chunk / warps;
  warp_state* ws = (warp_state*)malloc(sizeof(warp_state) * (size_t)warps);
  for (int w = 0; w < warps; ++w) {
    int start = chunk_id * chunk + w * rows_per_warp;   /* :581 */
    int end = start + rows_per_warp;
    if (end > seqlen) end = seqlen;
    if (start >= seqlen) end = start;
    warp_scan(qf, k, v, row_stride, start, end, scale, &ws[w]);
  }
  block_merge(ws, warps, &gmax, &tsum, o);
  float inv_sum = 1.0f / tsum;                          /* :646 */
  for (int d = 0; d < QD_D; ++d) part[d] = qd_oracle_f2h(o[d] * inv_sum);
  *lse = logf(tsum) + gmax;                             /* :654 */
  free(ws);
}

/* Stage 2 (flash_decode_q1_opt.cuh:666-724): max over LSE, then warp 0's
 * sequential weighted sum in chunk order. */
static void split_stage2(const uint16_t* part, const float* lse, int nchunks,
                         uint16_t* out) {
  float max_lse = -INFINITY;
  for (int c = 0; c < nchunks; ++c) max_lse = fmaxf(max_lse, lse[c]);
  float sum_w = 0.0f, o[QD_D];
  for (int d = 0; d < QD_D; ++d) o[d] = 0.0f;
  for (int c = 0; c < nchunks; ++c) {
    float w = expf(lse[c] - max_lse);
    sum_w += w;
    for (int d = 0; d < QD_D; ++d)
      o[d] = fmaf(w, qd_oracle_h2f(part[(long long)c * QD_D + d]), o[d]);
  }
  float inv_w = 1.0f / sum_w;                           /* :717 */
  for (int d = 0; d < QD_D; ++d) out[d] = qd_oracle_f2h(o[d] * inv_w);
}

void qd_oracle_fd_split_head(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             uint16_t* out, int seqlen, long long row_stride,
                             int chunk, int warps, uint16_t* partial, float* lse) {
  float qf[QD_D];
  int nchunks = (seqlen + chunk - 1) / chunk;
  uint16_t* part = partial ? partial : (uint16_t*)malloc(sizeof(uint16_t) * QD_D * (size_t)nchunks);
  float* l = lse ? lse : (float*)malloc(sizeof(float) * (size_t)nchunks);
  load_q(q, qf);
  for (int c = 0; c < nchunks; ++c)
    split_stage1_chunk(qf, k, v, row_stride, seqlen, c, chunk, warps,
                       part + (long long)c * QD_D, &l[c]);
  split_stage2(part, l, nchunks, out);
  if (!partial) free(part);
  if (!lse) free(l);
}

/* ------------------------------------------------------------------------ */
/* All-heads driver with a small worker pool (CPU baseline)                 */
/* ------------------------------------------------------------------------ */

typedef struct {
  const uint16_t *q, *k, *v;
  uint16_t* out;
  int seqlen, num_heads, variant;
  long long row_stride, head_stride;
  int fused_warps;          /* fused variant */
  int chunk, warps, nchunks;/* split variant */
  uint16_t* part;           /* [H][nchunks][128] */
  float* lse;               /* [H][nchunks] */
  int ntasks;
  int next;                 /* atomic task counter */
  int phase;                /* 0: stage-1 / fused tasks, 1: stage-2 tasks */
} attn_job;

static void run_task(attn_job* j, int t) {
  if (j->variant == QD_ORACLE_FUSED || (j->variant == QD_ORACLE_ENGINE && j->nchunks == 1)) {
    int h = t;
    qd_oracle_fd_fused_head(j->q + (long long)h * QD_D, j->k + (long long)h * j->head_stride,
                            j->v + (long long)h * j->head_stride, j->out + (long long)h * QD_D,
                            j->seqlen, j->row_stride, 32, j->fused_warps);
    return;
  }
  if (j->phase == 0) {
    int h = t / j->nchunks, c = t % j->nchunks;
    float qf[QD_D];
    load_q(j->q + (long long)h * QD_D, qf);
    split_stage1_chunk(qf, j->k + (long long)h * j->head_stride, j->v + (long long)h * j->head_stride,
                       j->row_stride, j->seqlen, c, j->chunk, j->warps,
                       j->part + ((long long)h * j->nchunks + c) * QD_D,
                       &j->lse[(long long)h * j->nchunks + c]);
  } else {
    int h = t;
    split_stage2(j->part + (long long)h * j->nchunks * QD_D, j->lse + (long long)h * j->nchunks,
                 j->nchunks, j->out + (long long)h * QD_D);
  }
}

static void* worker(void* arg) {
  attn_job* j = (attn_job*)arg;
  for (;;) {
    int t = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
    if (t >= j->ntasks) break;
    run_task(j, t);
  }
  return NULL;
}

static void run_pool(attn_job* j, int ntasks, int nthreads) {
  j->ntasks = ntasks;
  j->next = 0;
  if (nthreads > ntasks) nthreads = ntasks;
  if (nthreads <= 1) {
    worker(j);
    return;
  }
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  int started = 0;
  for (int i = 0; i < nthreads; ++i)
    if (pthread_create(&th[i], NULL, worker, j) == 0) started++;
    else break;
  if (started == 0) worker(j);
  for (int i = 0; i < started; ++i) pthread_join(th[i], NULL);
  free(th);
}

int qd_oracle_decode_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               uint16_t* out, int seqlen, int num_heads,
                               long long row_stride, long long head_stride,
                               int variant, int nthreads) {
  if (!q || !k || !v || !out || seqlen < 1 || num_heads < 1) return -1;
  if (variant < QD_ORACLE_ENGINE || variant > QD_ORACLE_SPLIT) return -1;
  attn_job j;
  memset(&j, 0, sizeof(j));
  j.q = q; j.k = k; j.v = v; j.out = out;
  j.seqlen = seqlen; j.num_heads = num_heads; j.variant = variant;
  j.row_stride = row_stride; j.head_stride = head_stride;
  j.chunk = 256; j.warps = 8;                           /* qwen_infer.cu:650,671 */
  j.nchunks = (seqlen + j.chunk - 1) / j.chunk;
  if (variant == QD_ORACLE_ENGINE && j.nchunks == 1) {
    j.fused_warps = 8;                                  /* fd_v5_fused_kernel<128,8,32><<<1,256>>> */
  } else if (variant == QD_ORACLE_FUSED) {
    int nw = (seqlen + 31) / 32;                        /* bench_fd_opt.cu:304-307 */
    if (nw > 32) return -1;                             /* > 1024 rows: no single block */
    j.fused_warps = nw;
  }
  if (nthreads < 1) nthreads = 1;
  if (j.fused_warps > 0) {
    run_pool(&j, num_heads, nthreads);
    return 0;
  }
  j.part = (uint16_t*)malloc(sizeof(uint16_t) * QD_D * (size_t)num_heads * (size_t)j.nchunks);
  j.lse = (float*)malloc(sizeof(float) * (size_t)num_heads * (size_t)j.nchunks);
  if (!j.part || !j.lse) { free(j.part); free(j.lse); return -1; }
  j.phase = 0;
  run_pool(&j, num_heads * j.nchunks, nthreads);
  j.phase = 1;
  run_pool(&j, num_heads, nthreads);
  free(j.part);
  free(j.lse);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* QKV bias + RoPE + KV-cache append                                         */
/* ------------------------------------------------------------------------ */

void qd_oracle_rope_cos_sin(int pos, int i, int head_dim, float rope_base,
                            float* cos_out, float* sin_out) {
  /* float theta = pos * powf(10000.0f, -2.0f * tid / head_dim);
   * (fused_qkv_rope_cache.cuh:36): int*float and float/int promote to float. */
  float theta = (float)pos * powf(rope_base, (-2.0f * (float)i) / (float)head_dim);
  *cos_out = cosf(theta);
  *sin_out = sinf(theta);
}

int qd_oracle_qkv_bias_rope_cache(uint16_t* qkv, const uint16_t* bias,
                                  uint16_t* k_cache, uint16_t* v_cache, int pos,
                                  int num_heads, int head_dim,
                                  long long row_stride, long long head_stride,
                                  float rope_base) {
  if (!qkv || !k_cache || !v_cache || pos < 0 || num_heads < 1 || head_dim < 2 || (head_dim & 1))
    return -1;
  const int hidden = num_heads * head_dim;
  const int half = head_dim / 2;
  if (bias) {                                           /* bias.cuh:6-11 over 3*hidden */
    for (int j = 0; j < 3 * hidden; ++j)
      qkv[j] = qd_oracle_f2h(qd_oracle_h2f(qkv[j]) + qd_oracle_h2f(bias[j]));
  }
  for (int h = 0; h < num_heads; ++h) {
    for (int t = 0; t < half; ++t) {                    /* fused_qkv_rope_cache.cuh:15-54 */
      int idx1 = h * head_dim + t;
      int idx2 = idx1 + half;
      float q1 = qd_oracle_h2f(qkv[idx1]);
      float q2 = qd_oracle_h2f(qkv[idx2]);
      float k1 = qd_oracle_h2f(qkv[hidden + idx1]);
      float k2 = qd_oracle_h2f(qkv[hidden + idx2]);
      float v1 = qd_oracle_h2f(qkv[2 * hidden + idx1]);
      float v2 = qd_oracle_h2f(qkv[2 * hidden + idx2]);
      float c, s;
      qd_oracle_rope_cos_sin(pos, t, head_dim, rope_base, &c, &s);
      qkv[idx1] = qd_oracle_f2h(q1 * c - q2 * s);
      qkv[idx2] = qd_oracle_f2h(q2 * c + q1 * s);
      long long base = (long long)pos * row_stride + (long long)h * head_stride;
      k_cache[base + t] = qd_oracle_f2h(k1 * c - k2 * s);
      k_cache[base + half + t] = qd_oracle_f2h(k2 * c + k1 * s);
      v_cache[base + t] = qd_oracle_f2h(v1);
      v_cache[base + half + t] = qd_oracle_f2h(v2);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Adjacent decode-step ops: RMSNorm, GEMV, QKV front end                    */
/* ------------------------------------------------------------------------ */

float qd_oracle_wave64_sum(const float* a) {
  float rows[4];
  for (int r = 0; r < 4; ++r) {
    const float* x = a + 16 * r;
    float q[4];
    for (int i = 0; i < 4; ++i) q[i] = (x[4 * i] + x[4 * i + 1]) + (x[4 * i + 2] + x[4 * i + 3]);
    rows[r] = (q[0] + q[1]) + (q[2] + q[3]);
  }
  return (rows[0] + rows[1]) + (rows[2] + rows[3]);
}

/* 32-lane xor butterfly (masks 16..1), the value every lane ends with. */
static float warp32_sum(float* lane) {
  float tmp[32];
  for (int mask = 16; mask >= 1; mask >>= 1) {
    for (int ln = 0; ln < 32; ++ln) tmp[ln] = lane[ln] + lane[ln ^ mask];
    memcpy(lane, tmp, sizeof(tmp));
  }
  return lane[0];
}

/* Sequential per-lane sums of f(k) over the wave64 element layout. */
static void wave64_lane_sums(int n, const float* v, float* lanes) {
  const int chunks = (n + 511) / 512;
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int j = 0; j < chunks; ++j)
      for (int e = 0; e < 8; ++e) {
        int k = 512 * j + 8 * l + e;
        if (k < n) acc += v[k];
      }
    lanes[l] = acc;
  }
}

void qd_oracle_rmsnorm(const uint16_t* x, const uint16_t* w, int n, float eps,
                       uint16_t* out, int order) {
  float* sq = (float*)malloc(sizeof(float) * (size_t)n);
  for (int k = 0; k < n; ++k) {
    float v = qd_oracle_h2f(x[k]);
    sq[k] = v * v;                                  /* exact: 22-bit product */
  }
  float total;
  if (order == QD_ORDER_WAVE64) {
    float lanes[64];
    wave64_lane_sums(n, sq, lanes);
    total = qd_oracle_wave64_sum(lanes);
  } else {
    /* rmsnorm.cuh:9-45 with blockDim 512: thread t sums its n/512 contiguous
     * items, warps reduce by xor butterfly, warp 0 reduces the 16 warp sums. */
    const int per = n / 512;
    float warp_sums[32];
    for (int wp = 0; wp < 16; ++wp) {
      float lane[32];
      for (int ln = 0; ln < 32; ++ln) {
        int t = wp * 32 + ln;
        float acc = 0.0f;
        for (int i = 0; i < per; ++i) acc += sq[t * per + i];
        lane[ln] = acc;
      }
      warp_sums[wp] = warp32_sum(lane);
    }
    for (int ln = 16; ln < 32; ++ln) warp_sums[ln] = 0.0f;
    total = warp32_sum(warp_sums);
  }
  const float var = total / (float)n;
  const float r = 1.0f / sqrtf(var + eps);
  for (int k = 0; k < n; ++k)
    out[k] = qd_oracle_f2h(qd_oracle_h2f(x[k]) * r * qd_oracle_h2f(w[k]));
  free(sq);
}

static float gemv_row(const uint16_t* x, const uint16_t* W, int N, int K, int layout,
                      int order, int n, float* scratch) {
  for (int k = 0; k < K; ++k) {
    uint16_t wk = layout == 0 ? W[(long long)n * K + k] : W[(long long)k * N + n];
    scratch[k] = qd_oracle_h2f(x[k]) * qd_oracle_h2f(wk);   /* exact product */
  }
  if (order == QD_ORDER_WAVE64) {
    float lanes[64];
    wave64_lane_sums(K, scratch, lanes);
    return qd_oracle_wave64_sum(lanes);
  }
  float sum = 0.0f;                                  /* hgemm_final.cuh:278-293 */
  for (int k = 0; k < K; ++k) sum += scratch[k];
  return sum;
}

void qd_oracle_gemv(const uint16_t* x, const uint16_t* W, int N, int K, int layout,
                    int order, uint16_t* out) {
  float* scratch = (float*)malloc(sizeof(float) * (size_t)K);
  for (int n = 0; n < N; ++n) out[n] = qd_oracle_f2h(gemv_row(x, W, N, K, layout, order, n, scratch));
  free(scratch);
}

int qd_oracle_qkv_front(const uint16_t* x, const uint16_t* norm_w, float eps,
                        const uint16_t* w_qkv, const uint16_t* bias, uint16_t* qkv_out,
                        uint16_t* k_cache, uint16_t* v_cache, int pos, int num_heads,
                        int head_dim, long long row_stride, long long head_stride,
                        float rope_base, int order) {
  if (!x || !w_qkv || !qkv_out || !k_cache || !v_cache || pos < 0 || num_heads < 1 ||
      head_dim < 2 || (head_dim & 1))
    return -1;
  const int hidden = num_heads * head_dim;
  uint16_t* xn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)hidden);
  if (norm_w) qd_oracle_rmsnorm(x, norm_w, hidden, eps, xn, order);
  else memcpy(xn, x, sizeof(uint16_t) * (size_t)hidden);
  qd_oracle_gemv(xn, w_qkv, 3 * hidden, hidden, 0, order, qkv_out);   /* qwen_infer.cu:629 */
  free(xn);
  return qd_oracle_qkv_bias_rope_cache(qkv_out, bias, k_cache, v_cache, pos, num_heads, head_dim,
                                       row_stride, head_stride, rope_base);
}

/* ------------------------------------------------------------------------ */
/* The gfx950 kernels' own arithmetic: exp2 and decode attention             */
/* ------------------------------------------------------------------------ */

/* exp2_rep of llm-inference-diy_amd/csrc/qd_device.h, step for step. */
float qd_oracle_exp2(float x) {
  if (!(x > -125.0f)) return 0.0f;
  if (x >= 128.0f) return INFINITY;
  const float n = rintf(x);
  const float f = x - n;
  const float f2 = f * f;
  const float a = fmaf(0x1.ebfbdcp-3f, f, 0x1.62e430p-1f);
  const float b = fmaf(0x1.3b2d4ep-7f, f, 0x1.c6aee8p-5f);
  const float c = fmaf(0x1.41fbb0p-13f, f, 0x1.5f3e54p-10f);
  const float q = fmaf(fmaf(c, f2, b), f2, a);
  return ldexpf(fmaf(q, f, 1.0f), (int)n);
}

void qd_oracle_exp2_array(const float* x, float* out, long long n) {
  for (long long i = 0; i < n; ++i) out[i] = qd_oracle_exp2(x[i]);
}

static float safe_base(float m) { return m == -INFINITY ? 0.0f : m; }

/* Online-softmax state of one 16-lane group; lane t owns dims 8t..8t+7. */
typedef struct {
  float m, l;
  float o[QD_D];
} gstate;

static void gstate_init(gstate* st) {
  st->m = -INFINITY;
  st->l = 0.0f;
  for (int d = 0; d < QD_D; ++d) st->o[d] = 0.0f;
}

/* wave_merge, max-first: M = max of the four groups' m, each group scaled by
 * exp2(m - M), summed as (g0 + g1) + (g2 + g3).  Result in g[0]. */
static void wave_merge4(gstate* g) {
  float M = fmaxf(fmaxf(g[0].m, g[1].m), fmaxf(g[2].m, g[3].m));
  const float base = safe_base(M);
  float sc[4];
  for (int i = 0; i < 4; ++i) sc[i] = qd_oracle_exp2(g[i].m - base);
  float l[4];
  for (int i = 0; i < 4; ++i) l[i] = g[i].l * sc[i];
  g[0].l = (l[0] + l[1]) + (l[2] + l[3]);
  for (int d = 0; d < QD_D; ++d) {
    float o[4];
    for (int i = 0; i < 4; ++i) o[i] = g[i].o[d] * sc[i];
    g[0].o[d] = (o[0] + o[1]) + (o[2] + o[3]);
  }
  g[0].m = M;
}

/* The score of one row for one 16-lane group: lane t starts from the exact
 * product k0*q0 and adds its other 7 products with fmaf in element order
 * (decode_attention_scan_kernel's dot8), then the 16-lane tree of row16_sum. */
static float group_score(const float* qf, const uint16_t* krow) {
  float lanes[16];
  for (int t = 0; t < 16; ++t) {
    float acc = qd_oracle_h2f(krow[8 * t]) * qf[8 * t];   /* exact */
    for (int e = 1; e < 8; ++e) acc = fmaf(qd_oracle_h2f(krow[8 * t + e]), qf[8 * t + e], acc);
    lanes[t] = acc;
  }
  float q4[4];
  for (int i = 0; i < 4; ++i) q4[i] = (lanes[4 * i] + lanes[4 * i + 1]) + (lanes[4 * i + 2] + lanes[4 * i + 3]);
  return (q4[0] + q4[1]) + (q4[2] + q4[3]);
}

static float gfx_scale_log2(void) { return (float)(1.4426950408889634 / sqrt(128.0)); }

/* Layer row of a split's j-th row (decode_attention_scan_kernel's split_row):
 * j for a contiguous range (whose first row the k/v base already holds), or,
 * for blocks of `block` rows dealt to `splits` splits in turn, row
 * ((j / block) * splits + c) * block + j % block. */
static long long split_row(int j, int block, int splits, int c) {
  if (block == 0) return j;
  return ((long long)(j / block) * splits + c) * block + j % block;
}

/* Rows of split c of an interleaved plan (qd::interleaved_rows). */
static int interleaved_rows(int seqlen, int block, int splits, int c) {
  const int full = seqlen / block, rem = seqlen % block;
  const int nfull = full > c ? (full - 1 - c) / splits + 1 : 0;
  return nfull * block + (rem > 0 && full % splits == c ? rem : 0);
}

/* One workgroup of decode_attention_scan_kernel<NW, U, *>: the split's rows
 * j in [0, nrows), row j at k/v + split_row(j, block, splits, c)*row_stride.
 * Returns the LDS fold (M, L, O[128]). */
static void scan_workgroup(const float* qf, const uint16_t* k, const uint16_t* v,
                           long long row_stride, int nrows, int nw, int u_rows, int block,
                           int splits, int c, float* M_out, float* L_out, float* O_out) {
  const float scale = gfx_scale_log2();
  gstate* st = (gstate*)malloc(sizeof(gstate) * (size_t)nw * 4);
  float* s = (float*)malloc(sizeof(float) * (size_t)u_rows);
  int* rr = (int*)malloc(sizeof(int) * (size_t)u_rows);
  for (int i = 0; i < nw * 4; ++i) gstate_init(&st[i]);
  for (int w = 0; w < nw; ++w) {
    for (int blk = w * 4 * u_rows; blk < nrows; blk += nw * 4 * u_rows) {
      for (int g = 0; g < 4; ++g) {
        gstate* x = &st[w * 4 + g];
        for (int u = 0; u < u_rows; ++u) {
          const int row = blk + 4 * u + g;
          rr[u] = row < nrows - 1 ? row : nrows - 1;       /* clamped load row */
          const float d = group_score(qf, k + split_row(rr[u], block, splits, c) * row_stride);
          s[u] = row < nrows ? d * scale : -INFINITY;
        }
        float mt = s[0];
        for (int u = 1; u < u_rows; ++u) mt = fmaxf(mt, s[u]);
        const float mn = fmaxf(x->m, mt);
        const float base = safe_base(mn);
        const float alpha = qd_oracle_exp2(x->m - base);   /* consume_tile */
        x->l *= alpha;
        for (int d = 0; d < QD_D; ++d) x->o[d] *= alpha;
        for (int u = 0; u < u_rows; ++u) {
          const float p = qd_oracle_exp2(s[u] - base);
          x->l += p;
          const uint16_t* vrow = v + split_row(rr[u], block, splits, c) * row_stride;
          for (int d = 0; d < QD_D; ++d) x->o[d] = fmaf(qd_oracle_h2f(vrow[d]), p, x->o[d]);
        }
        x->m = mn;
      }
    }
  }
  for (int w = 0; w < nw; ++w) wave_merge4(&st[w * 4]);
  /* LDS fold by threads 0..127, one dim each */
  float M = -INFINITY;
  for (int w = 0; w < nw; ++w) M = fmaxf(M, st[w * 4].m);
  const float base = safe_base(M);
  float L = 0.0f;
  for (int d = 0; d < QD_D; ++d) O_out[d] = 0.0f;
  for (int w = 0; w < nw; ++w) {
    const float wt = qd_oracle_exp2(st[w * 4].m - base);
    L = fmaf(wt, st[w * 4].l, L);
    for (int d = 0; d < QD_D; ++d) O_out[d] = fmaf(wt, st[w * 4].o[d], O_out[d]);
  }
  *M_out = M;
  *L_out = L;
  free(rr);
  free(s);
  free(st);
}

/* decode_attention_merge_kernel<256> for one head, max-first: M = max of all
 * splits' m; slice s (of 8) sums w_c*l_c and w_c*O_c, w_c = exp2(m_c - M),
 * over splits c = s, s+8, ... in ascending order with fmaf; the slice sums
 * are added in slice order; out = half(O / L). */
static void merge_head(const float* part_o, const float* part_m, const float* part_l,
                       int splits, uint16_t* out) {
  enum { P = 8 };
  float M = -INFINITY;
  for (int s = 0; s < P; ++s) {
    float mm = -INFINITY;
    for (int c = s; c < splits; c += P) mm = fmaxf(mm, part_m[c]);
    M = s == 0 ? mm : fmaxf(M, mm);
  }
  const float base = safe_base(M);
  float sl[P];
  static __thread float so[P][QD_D];
  for (int s = 0; s < P; ++s) {
    float ll = 0.0f;
    for (int d = 0; d < QD_D; ++d) so[s][d] = 0.0f;
    for (int c = s; c < splits; c += P) {
      const float w = qd_oracle_exp2(part_m[c] - base);
      ll = fmaf(w, part_l[c], ll);
      for (int d = 0; d < QD_D; ++d) so[s][d] = fmaf(w, part_o[(long long)c * QD_D + d], so[s][d]);
    }
    sl[s] = ll;
  }
  for (int d = 0; d < QD_D; ++d) {
    float L = sl[0], O = so[0][d];
    for (int s = 1; s < P; ++s) {
      L += sl[s];
      O += so[s][d];
    }
    out[d] = qd_oracle_f2h(O / L);
  }
}

typedef struct {
  const uint16_t *q, *k, *v;
  uint16_t* out;
  int seqlen, num_heads;
  long long row_stride, head_stride;
  qd_oracle_plan plan;
  int next;
} gfx_job;

static void gfx_head(gfx_job* j, int h) {
  float qf[QD_D];
  for (int d = 0; d < QD_D; ++d) qf[d] = qd_oracle_h2f(j->q[(long long)h * QD_D + d]);
  const uint16_t* kh = j->k + (long long)h * j->head_stride;
  const uint16_t* vh = j->v + (long long)h * j->head_stride;
  uint16_t* oh = j->out + (long long)h * QD_D;
  const qd_oracle_plan* pl = &j->plan;
  if (pl->variant == 0) {
    float M, L, O[QD_D];
    scan_workgroup(qf, kh, vh, j->row_stride, j->seqlen, pl->waves, pl->rows_per_tile, 0, 1, 0,
                   &M, &L, O);
    for (int d = 0; d < QD_D; ++d) oh[d] = qd_oracle_f2h(O[d] / L);
    return;
  }
  const int S = pl->num_splits;
  float* po = (float*)malloc(sizeof(float) * (size_t)S * QD_D);
  float* pm = (float*)malloc(sizeof(float) * (size_t)S);
  float* plv = (float*)malloc(sizeof(float) * (size_t)S);
  for (int c = 0; c < S; ++c) {
    if (pl->block_rows) {
      scan_workgroup(qf, kh, vh, j->row_stride, interleaved_rows(j->seqlen, pl->block_rows, S, c),
                     pl->waves, pl->rows_per_tile, pl->block_rows, S, c, &pm[c], &plv[c],
                     po + (long long)c * QD_D);
      continue;
    }
    const int r0 = c * pl->rows_per_split;
    int nrows = j->seqlen - r0;
    if (nrows > pl->rows_per_split) nrows = pl->rows_per_split;
    scan_workgroup(qf, kh + (long long)r0 * j->row_stride, vh + (long long)r0 * j->row_stride,
                   j->row_stride, nrows, pl->waves, pl->rows_per_tile, 0, 1, 0, &pm[c], &plv[c],
                   po + (long long)c * QD_D);
  }
  merge_head(po, pm, plv, S, oh);
  free(plv);
  free(pm);
  free(po);
}

static void* gfx_worker(void* arg) {
  gfx_job* j = (gfx_job*)arg;
  for (;;) {
    int h = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
    if (h >= j->num_heads) break;
    gfx_head(j, h);
  }
  return NULL;
}

int qd_oracle_attention_planned(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                uint16_t* out, int seqlen, int num_heads, long long row_stride,
                                long long head_stride, const qd_oracle_plan* plan, int nthreads) {
  if (!q || !k || !v || !out || !plan || seqlen < 1 || num_heads < 1) return -1;
  if (plan->rows_per_tile < 1 || plan->waves < 1) return -1;
  if (plan->variant != 0 && plan->block_rows) {
    /* blocks of one load round of the workgroup; every split has a block */
    if (plan->num_splits < 1 || plan->block_rows != plan->waves * 4 * plan->rows_per_tile) return -1;
    if ((long long)(plan->num_splits - 1) * plan->block_rows >= seqlen) return -1;
  } else if (plan->variant != 0) {
    if (plan->num_splits < 1 || plan->rows_per_split < 1) return -1;
    /* every split workgroup has rows, and together they cover [0, seqlen) */
    if ((long long)(plan->num_splits - 1) * plan->rows_per_split >= seqlen) return -1;
    if ((long long)plan->num_splits * plan->rows_per_split < seqlen) return -1;
  } else if (plan->block_rows) {
    return -1;
  }
  gfx_job j = {q, k, v, out, seqlen, num_heads, row_stride, head_stride, *plan, 0};
  if (nthreads > num_heads) nthreads = num_heads;
  if (nthreads <= 1) {
    gfx_worker(&j);
    return 0;
  }
  pthread_t th[256];
  if (nthreads > 256) nthreads = 256;
  int started = 0;
  for (int i = 0; i < nthreads; ++i)
    if (pthread_create(&th[i], NULL, gfx_worker, &j) == 0) started++;
    else break;
  if (started == 0) gfx_worker(&j);
  for (int i = 0; i < started; ++i) pthread_join(th[i], NULL);
  return 0;
}
