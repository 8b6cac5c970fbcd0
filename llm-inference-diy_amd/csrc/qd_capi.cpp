// C ABI of the decode-attention hot path: context lifetime, argument checks,
// launch planning.  Declared in include/qdiy/attn.h.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <vector>

#include "qd_internal.h"
#include "qdiy/bench.h"
#include "qdiy/decode.h"

namespace {
thread_local char g_err[512] = "";
}  // namespace

namespace qd {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(QD_EHIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace qd

namespace {

using qd::aligned16;
using qd::fail;
using qd::hip_fail;

// Launch planner, from measured sweeps on MI355X (16 heads, cold KV, the
// bit-reproducible kernels):
//   * short lengths: one 16-wave workgroup per head, no merge -- up to
//     kFusedMaxRowsX rows when the context merges split plans inside the scan
//     kernel (fused 4.7 us at 128 rows against 5.0 split, 5.3 against 5.1 at
//     160), else up to kFusedMaxRows (split + merge kernel costs ~7 us there);
//   * longer: one split workgroup per CU in total (16 splits at 16 heads), each
//     looping over its rows (qd::auto_split); other split counts or more waves
//     per workgroup measured no better (L=8192: 14.7 us at 16 splits, 15.6 at
//     32, 16.7 at 64, 17.1 at 24).  Up to kXMergeMaxRows rows the last split
//     of each head merges in the scan kernel (4.9-5.2 us at 256-512 rows, 5.6
//     at 768, 6.4-6.7 at 1280-1536, against 6.9-7.4 with a merge kernel; 7.24
//     against 7.29 at 2048, 8.42 against 8.49 at 3072); beyond, the splits'
//     rows are dealt to them in interleaved blocks of 64 rows and the merge
//     stays in the scan kernel (qd::auto_plan), where the context can merge
//     there; else contiguous ranges and a merge kernel.
constexpr int kFusedMaxRows = 224;
constexpr int kFusedMaxRowsX = 128;
using qd::kXMergeMaxRows;
constexpr int kPrefillBatch = 256;   // split-plan prefill queries per batched launch pair

qd::AttnPlan plan_fused(int seqlen) {
  qd::AttnPlan plan;
  plan.variant = 0;
  plan.splits = 1;
  plan.rows_per_split = seqlen;
  plan.rows_per_tile = 4;
  plan.waves = 16;
  plan.xmerge = 0;
  plan.depth = 1;
  plan.block_rows = 0;
  return plan;
}

// A split plan: the automatic one (requested <= 0; qd::auto_plan, whose long
// plans interleave their rows where merges_in_kernel), else `requested` splits
// over contiguous ranges.
qd::AttnPlan plan_split(int num_cus, int num_heads, int seqlen, int requested, bool merges_in_kernel) {
  int splits, rows, block = 0;
  if (requested <= 0) {
    qd::auto_plan(seqlen, num_cus, num_heads, merges_in_kernel, &splits, &rows, &block);
  } else {
    splits = std::min(requested, qd::kMaxSplits);
    rows = (seqlen + splits - 1) / splits;
    rows = (rows + 3) & ~3;                    // one load instruction covers 4 rows
    splits = (seqlen + rows - 1) / rows;       // no empty workgroups
  }
  qd::AttnPlan plan;
  plan.variant = 1;
  plan.rows_per_split = rows;
  plan.splits = splits;
  plan.waves = 4;
  plan.rows_per_tile = block ? block / 16 : rows >= 64 ? 4 : 2;   // a block: one 4-wave load round
  plan.xmerge = 0;
  plan.depth = 1;
  plan.block_rows = block;
  return plan;
}

// A split plan recast with `waves` waves of `rows_per_tile`-row tiles per
// workgroup, and, when `interleave`, its rows dealt to the splits in blocks of
// one load round (waves * 4 * rows_per_tile rows): same split count, at most
// one split per block.
qd::AttnPlan reshape_split(const qd::AttnPlan& in, int seqlen, int waves, int rows_per_tile,
                           int interleave) {
  qd::AttnPlan plan = in;
  if (plan.variant != 1) return plan;
  plan.waves = waves;
  plan.rows_per_tile = rows_per_tile;
  if (interleave) {
    const int block = waves * 4 * rows_per_tile;
    plan.block_rows = block;
    plan.splits = std::max(1, std::min(plan.splits, (seqlen + block - 1) / block));
    plan.rows_per_split = qd::interleaved_rows(seqlen, block, plan.splits, 0);   // split 0's, the most
  }
  return plan;
}

// The context's split plan.  Its automatic long plans interleave where the
// context can merge in the scan kernel at all (ctx->xmerge_ok), whatever the
// merge mode, so that every mode gives the same bits; a forced shape
// (qd_ctx_set_split_shape) recasts the contiguous plan.
qd::AttnPlan plan_split(const qd_ctx* ctx, int seqlen, int requested) {
  if (ctx->shape_waves)
    return reshape_split(plan_split(ctx->num_cus, ctx->cfg.num_heads, seqlen, requested, false), seqlen,
                         ctx->shape_waves, ctx->shape_tile, ctx->shape_inter);
  return plan_split(ctx->num_cus, ctx->cfg.num_heads, seqlen, requested, ctx->xmerge_ok);
}

// The automatic plan: fused up to fused_max rows, else the automatic split.
qd::AttnPlan plan_auto(int num_cus, int num_heads, int seqlen, int fused_max, bool merges_in_kernel) {
  return seqlen <= fused_max ? plan_fused(seqlen)
                             : plan_split(num_cus, num_heads, seqlen, 0, merges_in_kernel);
}

// Round-robin period of workgroup dispatch over the XCDs of `device` (workgroup
// i of a 256-workgroup launch on XCD (k + i) mod period; 1 if every workgroup
// ran on one XCD, 0 if the placement was not round-robin in three tries).
// Probed once per device and process, into the 256-word device buffer
// `probe_buf` (whose contents it overwrites) with one kernel on the null
// stream and a synchronous 1 KiB copy to the host; later calls return the
// cached answer, so every context and every allocation-free call of a process
// plans the same way on one device.  Must be called with `device` current.
int dispatch_period(int device, unsigned* probe_buf, int* period) {
  static std::mutex mu;
  static int cached[64];
  static bool probed[64];
  std::lock_guard<std::mutex> lock(mu);
  const int slot = device >= 0 && device < 64 ? device : -1;
  if (slot >= 0 && probed[slot]) {
    *period = cached[slot];
    return QD_OK;
  }
  constexpr int kProbe = 256;
  unsigned xcc[kProbe];
  int p = 0;
  for (int attempt = 0; attempt < 3 && p == 0; ++attempt) {
    hipError_t e;
    if ((e = qd::launch_xcd_probe(probe_buf, kProbe, nullptr)) != hipSuccess ||
        (e = hipMemcpy(xcc, probe_buf, sizeof(xcc), hipMemcpyDeviceToHost)) != hipSuccess)
      return hip_fail(e, "XCD placement probe");
    p = qd::round_robin_period(xcc, kProbe);
  }
  if (slot >= 0) {
    probed[slot] = true;
    cached[slot] = p;
  }
  *period = p;
  return QD_OK;
}

// Whether the context's split plans can merge in the scan kernel: it found
// round-robin dispatch with num_heads a multiple of its period, and the
// caller did not ask for two launches.
bool xmerge_available(const qd_ctx* ctx) {
  return ctx->xmerge_ok && ctx->merge_mode != QD_MERGE_TWO_LAUNCHES;
}

// Longest length the automatic plan runs fused.
int fused_max_rows(const qd_ctx* ctx) {
  return xmerge_available(ctx) ? kFusedMaxRowsX : kFusedMaxRows;
}

qd::AttnPlan plan_auto(const qd_ctx* ctx, int seqlen) {
  return seqlen <= fused_max_rows(ctx) ? plan_fused(seqlen) : plan_split(ctx, seqlen, 0);
}


int check_attention_args(const qd_ctx* ctx, const uint16_t* q, const uint16_t* k,
                         const uint16_t* v, const uint16_t* out, int seqlen, int num_heads,
                         int head_dim) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  if (!q || !k || !v || !out) return fail(QD_EINVAL, "q, k_layer, v_layer and out must be non-NULL");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(QD_EINVAL, "q, k_layer, v_layer and out must be 16-byte aligned");
  if (head_dim != QD_HEAD_DIM || head_dim != ctx->cfg.head_dim)
    return fail(QD_EINVAL, "head_dim %d unsupported (must be %d)", head_dim, QD_HEAD_DIM);
  if (num_heads != ctx->cfg.num_heads)
    return fail(QD_EINVAL, "num_heads %d differs from the context's %d", num_heads, ctx->cfg.num_heads);
  if (seqlen < 1 || seqlen > ctx->cfg.max_seqlen)
    return fail(QD_EINVAL, "seqlen %d outside [1, %d]", seqlen, ctx->cfg.max_seqlen);
  // out may alias q (each head reads its q before any output is written) but
  // not the cache rows other workgroups are still reading
  const size_t ob = (size_t)num_heads * QD_HEAD_DIM * 2;
  const size_t kvb = ((size_t)(seqlen - 1) * ctx->cfg.kv_row_stride +
                      (size_t)(num_heads - 1) * ctx->cfg.kv_head_stride + QD_HEAD_DIM) * 2;
  if (qd::overlaps(out, ob, k, kvb) || qd::overlaps(out, ob, v, kvb))
    return fail(QD_EINVAL, "out overlaps the k_layer or v_layer rows being read");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != ctx->device)
    return fail(QD_EINVAL, "current device %d is not the context's device %d", dev, ctx->device);
  return QD_OK;
}

qd::AttnParams make_params(qd_ctx* ctx, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           uint16_t* out, int seqlen, const qd::AttnPlan& plan) {
  qd::AttnParams p;
  p.q = q;
  p.k = k;
  p.v = v;
  p.out = out;
  p.part_o = ctx->part_o;
  p.part_ml = ctx->part_ml;
  p.row_stride = ctx->cfg.kv_row_stride;
  p.head_stride = ctx->cfg.kv_head_stride;
  p.seqlen = seqlen;
  p.num_heads = ctx->cfg.num_heads;
  p.splits = plan.splits;
  p.rows_per_split = plan.rows_per_split;
  p.scale_log2 = (float)(1.4426950408889634 / std::sqrt(128.0));  // log2(e)/sqrt(128)
  p.q_batch_stride = 0;
  p.out_batch_stride = 0;
  p.num_cus = ctx->num_cus;
  p.split_stride = plan.splits;
  p.xpart = ctx->xpart;
  p.xcnt = ctx->xcnt;
  p.cnt_base = 0u;
  p.tag = 0u;
  p.recompute_mask = ctx->recompute_mask;
  p.count_merges = ctx->count_merges;
  p.block_rows = plan.block_rows;
  p.long_inter = ctx->xmerge_ok && !ctx->shape_waves;
  return p;
}

// Whether a split plan of this context merges inside the scan kernel: the
// merge is available, the length is at most kXMergeMaxRows (any length under
// QD_MERGE_IN_KERNEL), and the grid is at most one workgroup per CU -- then
// every split of a head runs on one XCD (measured: with two workgroups per
// CU, about 13 of a head's 32 splits landed on other XCDs, and the merger had
// to scan them again) -- and the merger reads the head's splits in one batch
// of loads.
bool use_xmerge(const qd_ctx* ctx, const qd::AttnPlan& plan, int seqlen) {
  return plan.variant == 1 && xmerge_available(ctx) &&
         (seqlen <= kXMergeMaxRows || plan.block_rows || ctx->merge_mode == QD_MERGE_IN_KERNEL) &&
         (plan.waves == 4 || plan.block_rows) && plan.splits <= qd::kXMaxSplits &&
         (long long)plan.splits * ctx->cfg.num_heads <= ctx->num_cus;
}

// The launch details that do not change the bits: whether the merge runs in
// the scan kernel, and how many tiles a wave loads per round.  Measured (16
// heads, cold): with the merge in the kernel, two tiles per round where a
// wave has two or more (768 rows: 5.80 against 6.25 us, 1280: 6.53 against
// 7.15, 1536: 6.81 against 7.25); one otherwise, and always with a merge
// kernel (two per round was 0.1-0.7 us slower from 2048 rows up; four per
// round slower everywhere).
// The planner's depth for a split plan (finish_plan's, and the
// allocation-free entry point's): 4-wave interleaved plans of 2-row tiles keep
// the next tile's loads in flight while consuming one (depth 0; 8192 rows:
// 13.78 against 18.41 us with one tile per round); contiguous 4-wave plans
// that merge in the kernel load two tiles per round where a wave has two.
int auto_depth(const qd::AttnPlan& plan, bool xmerge) {
  if (plan.variant != 1) return 1;
  if (plan.block_rows) return plan.waves == 4 && plan.rows_per_tile == 2 ? 0 : 1;
  if (plan.waves != 4) return 1;
  const int tiles = (plan.rows_per_split + 16 * plan.rows_per_tile - 1) / (16 * plan.rows_per_tile);
  return xmerge && tiles >= 2 ? 2 : 1;
}

qd::AttnPlan finish_plan(const qd_ctx* ctx, const qd::AttnPlan& plan_in, int seqlen) {
  qd::AttnPlan plan = plan_in;
  plan.xmerge = use_xmerge(ctx, plan, seqlen) ? 1 : 0;
  if (plan.variant == 1 && ctx->scan_depth == QD_SCAN_ROLLING) {
    plan.depth = 0;
  } else if (plan.variant == 1 && ctx->scan_depth != 0) {   // forced; interleaved plans: 1 per round
    plan.depth = plan.waves == 4 && !plan.block_rows ? ctx->scan_depth : 1;
  } else {
    plan.depth = auto_depth(plan, plan.xmerge != 0);
  }
  return plan;
}

// A fresh tag for a call that merges in the kernel (and its arrival counters'
// base); tag 0 is never used, and after 2^32 calls, once the tags wrap, the
// slots and the fused front end's words are cleared so that no stale word can
// carry the tag of the call that reads it.
int next_xmerge_tag(qd_ctx* ctx, qd::AttnParams& p, hipStream_t stream) {
  if (++ctx->xtag == 0u) {
    hipError_t e = hipMemsetAsync(ctx->xpart, 0,
                                  (size_t)ctx->cfg.num_heads * qd::kXMaxSplits * qd::kXSlotBytes, stream);
    if (e == hipSuccess)
      e = hipMemsetAsync(ctx->ftag, 0, (size_t)ctx->cfg.num_heads * 3 * 128 * sizeof(float2), stream);
    if (e != hipSuccess) return hip_fail(e, "clearing the in-kernel merge slots");
    ctx->xtag = 1u;
  }
  p.tag = ctx->xtag;
  p.cnt_base = ctx->xcnt_sum;
  return QD_OK;
}

int run_attention(qd_ctx* ctx, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                  uint16_t* out, int seqlen, const qd::AttnPlan& plan_in, hipStream_t stream,
                  int stages = qd::kStageScan | qd::kStageMerge) {
  const qd::AttnPlan plan = finish_plan(ctx, plan_in, seqlen);
  qd::AttnParams p = make_params(ctx, q, k, v, out, seqlen, plan);
  if (plan.xmerge && (stages & qd::kStageScan)) {
    const int rc = next_xmerge_tag(ctx, p, stream);
    if (rc != QD_OK) return rc;
  }
  hipError_t e = qd::launch_decode_attention(p, plan, stream, stages);
  if (e != hipSuccess) return hip_fail(e, "decode attention launch");
  // every split of every head but its merger arrives once on its head's counter
  if (plan.xmerge && (stages & qd::kStageScan)) ctx->xcnt_sum += (unsigned)(plan.splits - 1);
  return QD_OK;
}

}  // namespace

namespace qd {

int attention_prefill(qd_ctx* ctx, const uint16_t* q, long long q_stride, const uint16_t* k,
                      const uint16_t* v, uint16_t* out, long long out_stride, int pos0, int tokens,
                      hipStream_t stream) {
  if (tokens < 1) return QD_OK;
  int rc = check_attention_args(ctx, q, k, v, out, pos0 + 1, ctx ? ctx->cfg.num_heads : 0, QD_HEAD_DIM);
  if (rc != QD_OK) return rc;
  if (ctx->shape_waves)
    return fail(QD_EINVAL, "the context's split shape is forced (qd_ctx_set_split_shape): batched "
                           "queries plan the automatic shape, so they would not give its bits");
  if (pos0 + tokens > ctx->cfg.max_seqlen)
    return fail(QD_EINVAL, "positions up to %d exceed max_seqlen %d", pos0 + tokens, ctx->cfg.max_seqlen);
  // queries whose length plan_auto makes fused: one launch for all of them
  const int n_fused = std::max(0, std::min(tokens, fused_max_rows(ctx) - pos0));
  if (n_fused > 0) {
    qd::AttnParams p = make_params(ctx, q, k, v, out, pos0 + 1, plan_fused(pos0 + 1));
    p.q_batch_stride = q_stride;
    p.out_batch_stride = out_stride;
    const hipError_t e = qd::launch_decode_attention_fused_batch(p, n_fused, stream);
    if (e != hipSuccess) return hip_fail(e, "batched fused attention launch");
  }
  // The others take split plans.  Runs of consecutive queries whose plans
  // share a tile depth go out as one batched split launch pair, every query
  // under its own plan (at most kPrefillBatch queries per pair).
  if (n_fused >= tokens) return QD_OK;
  if (!ctx->pf_part_o) {
    // slots for kPrefillBatch queries x H heads x the largest automatic split count
    const int stride = std::max(1, std::min(qd::kMaxSplits, ctx->num_cus / ctx->cfg.num_heads));
    const size_t slots = (size_t)kPrefillBatch * ctx->cfg.num_heads * stride;
    hipError_t e = hipMalloc(&ctx->pf_part_o, slots * 128 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&ctx->pf_part_ml, slots * sizeof(float2));
    if (e != hipSuccess) {
      (void)hipFree(ctx->pf_part_o);
      ctx->pf_part_o = nullptr;
      ctx->pf_part_ml = nullptr;
      return fail(QD_ENOMEM, "hipMalloc of %zu bytes of prefill attention scratch failed", slots * 130 * 4);
    }
    ctx->pf_tokens = kPrefillBatch;
    ctx->pf_stride = stride;
  }
  for (int t = n_fused; t < tokens;) {
    const qd::AttnPlan first = plan_auto(ctx, pos0 + t + 1);
    int t1 = t + 1, max_splits = first.splits;
    for (; t1 < tokens && t1 - t < ctx->pf_tokens; ++t1) {
      const qd::AttnPlan pl = plan_auto(ctx, pos0 + t1 + 1);
      if (pl.rows_per_tile != first.rows_per_tile) break;
      max_splits = std::max(max_splits, pl.splits);
    }
    if (max_splits > ctx->pf_stride)
      return fail(QD_EINVAL, "internal: %d splits above the prefill scratch's %d", max_splits, ctx->pf_stride);
    qd::AttnParams p = make_params(ctx, q + t * q_stride, k, v, out + t * out_stride, pos0 + t + 1, first);
    p.q_batch_stride = q_stride;
    p.out_batch_stride = out_stride;
    p.part_o = ctx->pf_part_o;
    p.part_ml = ctx->pf_part_ml;
    p.num_cus = ctx->num_cus;
    p.split_stride = max_splits;
    const hipError_t e = qd::launch_decode_attention_split_batch(p, first.rows_per_tile, t1 - t, stream);
    if (e != hipSuccess) return hip_fail(e, "batched split attention launch");
    t = t1;
  }
  return QD_OK;
}

int attention_prefill_mfma(qd_ctx* ctx, const uint16_t* q, long long q_stride, const uint16_t* k,
                           const uint16_t* v, uint16_t* out, long long out_stride, int pos0,
                           int tokens, hipStream_t stream) {
  FlashPrefillParams p;
  p.q = q;
  p.q_stride = q_stride;
  p.k = k;
  p.v = v;
  p.row_stride = ctx->cfg.kv_row_stride;
  p.head_stride = ctx->cfg.kv_head_stride;
  p.out = out;
  p.out_stride = out_stride;
  p.pos0 = pos0;
  p.tokens = tokens;
  p.num_heads = ctx->cfg.num_heads;
  p.scale_log2 = (float)(1.4426950408889634 / std::sqrt(128.0));
  const hipError_t e = launch_flash_prefill(p, stream);
  return e == hipSuccess ? QD_OK : hip_fail(e, "prefill attention launch");
}

}  // namespace qd

namespace {
// The checks and parameters of qd_qkv_proj_rope_cache (QD_OK, or the error
// with its message).
int front_params(qd_ctx* ctx, const uint16_t* x, const uint16_t* norm_w, float eps,
                 const uint16_t* w_qkv, const uint16_t* qkv_bias, uint16_t* qkv, uint16_t* k_layer,
                 uint16_t* v_layer, int pos, int max_seqlen, int num_heads, int head_dim,
                 qd::QkvFrontParams& p);
}  // namespace

extern "C" {

int qd_ctx_create(const qd_cfg* cfg, qd_ctx** out_ctx) {
  if (!out_ctx) return fail(QD_EINVAL, "out_ctx is NULL");
  *out_ctx = nullptr;
  if (!cfg) return fail(QD_EINVAL, "cfg is NULL");
  if (cfg->head_dim != QD_HEAD_DIM) return fail(QD_EINVAL, "head_dim must be %d", QD_HEAD_DIM);
  if (cfg->num_heads < 1 || cfg->num_heads > 4096) return fail(QD_EINVAL, "num_heads out of range");
  if (cfg->max_seqlen < 1) return fail(QD_EINVAL, "max_seqlen must be >= 1");
  if (cfg->kv_row_stride < 1 || cfg->kv_head_stride < 1 || (cfg->kv_row_stride % 8) ||
      (cfg->kv_head_stride % 8))
    return fail(QD_EINVAL, "kv strides must be positive multiples of 8 elements");
  if (!(cfg->rope_base > 0.0f)) return fail(QD_EINVAL, "rope_base must be > 0");
  // the kernels address a row as (32-bit byte offset) from a per-head base
  if ((long long)cfg->max_seqlen * cfg->kv_row_stride * 2 > 0xFFFFFF00LL)
    return fail(QD_EINVAL, "max_seqlen * kv_row_stride * 2 bytes must stay below 4 GiB");

  qd_ctx* ctx = new (std::nothrow) qd_ctx;
  if (!ctx) return fail(QD_ENOMEM, "host allocation failed");
  std::memset(ctx, 0, sizeof(*ctx));
  ctx->cfg = *cfg;
  hipError_t e = hipGetDevice(&ctx->device);
  if (e != hipSuccess) {
    delete ctx;
    return hip_fail(e, "hipGetDevice");
  }
  e = hipDeviceGetAttribute(&ctx->num_cus, hipDeviceAttributeMultiprocessorCount, ctx->device);
  if (e != hipSuccess || ctx->num_cus < 1) {
    delete ctx;
    return hip_fail(e, "hipDeviceGetAttribute(multiProcessorCount)");
  }
  const size_t H = (size_t)cfg->num_heads;
  const size_t S = (size_t)cfg->max_seqlen;
  auto cleanup = [&](int code) {
    qd_ctx_destroy(ctx);
    return code;
  };
  if ((e = hipMalloc(&ctx->part_o, H * qd::kMaxSplits * 128 * sizeof(float))) != hipSuccess ||
      (e = hipMalloc(&ctx->part_ml, H * qd::kMaxSplits * sizeof(float2))) != hipSuccess ||
      (e = hipMalloc(&ctx->rope_cs, S * 64 * sizeof(float2))) != hipSuccess) {
    int code = hip_fail(e, "hipMalloc of context scratch");
    return cleanup(code == QD_EHIP ? QD_ENOMEM : code);
  }

  // RoPE table: theta = float(pos) * powf(base, (-2*i)/head_dim), then fp32
  // cosf/sinf (fused_qkv_rope_cache.cuh:36-38), evaluated once per context.
  std::vector<float2> cs;
  try {
    cs.resize(S * 64);
  } catch (...) {
    return cleanup(fail(QD_ENOMEM, "host allocation of the RoPE table failed"));
  }
  float inv_freq[64];
  for (int i = 0; i < 64; ++i)
    inv_freq[i] = powf(cfg->rope_base, (-2.0f * (float)i) / (float)cfg->head_dim);
  for (size_t pos = 0; pos < S; ++pos) {
    for (int i = 0; i < 64; ++i) {
      const float theta = (float)pos * inv_freq[i];
      cs[pos * 64 + i] = float2{cosf(theta), sinf(theta)};
    }
  }
  if ((e = hipMemcpy(ctx->rope_cs, cs.data(), S * 64 * sizeof(float2), hipMemcpyHostToDevice)) !=
      hipSuccess)
    return cleanup(hip_fail(e, "hipMemcpy of the RoPE table"));

  // In-kernel merge: tagged slots (all words tag 0, which no call uses) and
  // zeroed arrival counters; then the dispatch placement it is fast under.
  const size_t xpart_bytes = H * qd::kXMaxSplits * qd::kXSlotBytes;
  const size_t xcnt_bytes = H * qd::kXCounterStride * sizeof(unsigned);
  const size_t ftag_bytes = H * 3 * 128 * sizeof(float2);
  // The fused front end's tagged words follow the slots in their allocation.
  if ((e = hipMalloc(&ctx->xpart, xpart_bytes + ftag_bytes)) != hipSuccess ||
      (e = hipMalloc(&ctx->xcnt, xcnt_bytes)) != hipSuccess) {
    int code = hip_fail(e, "hipMalloc of the in-kernel merge scratch");
    return cleanup(code == QD_EHIP ? QD_ENOMEM : code);
  }
  ctx->ftag = reinterpret_cast<float2*>(reinterpret_cast<char*>(ctx->xpart) + xpart_bytes);
  if ((e = hipMemset(ctx->xcnt, 0, xcnt_bytes)) != hipSuccess ||
      (e = hipMemset(ctx->ftag, 0, ftag_bytes)) != hipSuccess)
    return cleanup(hip_fail(e, "hipMemset of the merge counters"));
  // Which XCD each workgroup runs on, probed into the slot area (cleared
  // afterwards).  Round-robin with period n (workgroup i on XCD (k + i) mod n
  // for some start k) puts every split of head h on one XCD when num_heads is
  // a multiple of n; a single XCD for all is period 1.  Anything else leaves
  // the in-kernel merge off (it would still be correct, but would re-scan the
  // splits it cannot see).
  {
    int period = 0;
    const int rc = dispatch_period(ctx->device, reinterpret_cast<unsigned*>(ctx->xpart), &period);
    if (rc != QD_OK) return cleanup(rc);
    if ((e = hipMemset(ctx->xpart, 0, xpart_bytes)) != hipSuccess ||
        (e = hipDeviceSynchronize()) != hipSuccess)
      return cleanup(hip_fail(e, "clearing the in-kernel merge slots"));
    ctx->num_xcd = period;
    ctx->xmerge_ok = period > 0 && cfg->num_heads % period == 0;
  }
  ctx->xtag = 0u;
  ctx->xcnt_sum = 0u;
  ctx->merge_mode = QD_MERGE_AUTO;
  ctx->recompute_mask = 0u;
  ctx->count_merges = 0;
  ctx->scan_depth = 0;
  ctx->shape_waves = ctx->shape_tile = ctx->shape_inter = 0;
  ctx->force_front_local = 0;
  *out_ctx = ctx;
  return QD_OK;
}

int qd_ctx_destroy(qd_ctx* ctx) {
  if (!ctx) return QD_OK;
  int dev = -1;
  const bool switch_dev = hipGetDevice(&dev) == hipSuccess && dev != ctx->device;
  if (switch_dev) (void)hipSetDevice(ctx->device);
  if (ctx->part_o) (void)hipFree(ctx->part_o);
  if (ctx->part_ml) (void)hipFree(ctx->part_ml);
  if (ctx->rope_cs) (void)hipFree(ctx->rope_cs);
  if (ctx->pf_part_o) (void)hipFree(ctx->pf_part_o);
  if (ctx->pf_part_ml) (void)hipFree(ctx->pf_part_ml);
  if (ctx->xpart) (void)hipFree(ctx->xpart);
  if (ctx->xcnt) (void)hipFree(ctx->xcnt);
  if (switch_dev) (void)hipSetDevice(dev);
  delete ctx;
  return QD_OK;
}

int qd_qkv_bias_rope_cache(qd_ctx* ctx, uint16_t* qkv, const uint16_t* bias, uint16_t* k_layer,
                           uint16_t* v_layer, int pos, int max_seqlen, int num_heads,
                           int head_dim, hipStream_t stream) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  if (!qkv || !k_layer || !v_layer) return fail(QD_EINVAL, "qkv, k_layer and v_layer must be non-NULL");
  if (((uintptr_t)qkv | (uintptr_t)k_layer | (uintptr_t)v_layer | (uintptr_t)bias) & 1u)
    return fail(QD_EINVAL, "fp16 buffers must be 2-byte aligned");
  if (head_dim != QD_HEAD_DIM) return fail(QD_EINVAL, "head_dim %d unsupported (must be 128)", head_dim);
  if (num_heads != ctx->cfg.num_heads)
    return fail(QD_EINVAL, "num_heads %d differs from the context's %d", num_heads, ctx->cfg.num_heads);
  if (max_seqlen < 1 || max_seqlen > ctx->cfg.max_seqlen)
    return fail(QD_EINVAL, "max_seqlen %d outside [1, %d]", max_seqlen, ctx->cfg.max_seqlen);
  if (pos < 0 || pos >= max_seqlen) return fail(QD_EINVAL, "pos %d outside [0, %d)", pos, max_seqlen);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != ctx->device)
    return fail(QD_EINVAL, "current device %d is not the context's device %d", dev, ctx->device);
  qd::RopeParams p;
  p.qkv = qkv;
  p.bias = bias;
  p.k_layer = k_layer;
  p.v_layer = v_layer;
  p.rope_cs = ctx->rope_cs;
  p.row_stride = ctx->cfg.kv_row_stride;
  p.head_stride = ctx->cfg.kv_head_stride;
  p.pos = pos;
  p.num_heads = num_heads;
  hipError_t e = qd::launch_qkv_bias_rope_cache(p, stream);
  if (e != hipSuccess) return hip_fail(e, "qkv_bias_rope_cache launch");
  return QD_OK;
}

int qd_qkv_proj_rope_cache(qd_ctx* ctx, const uint16_t* x, const uint16_t* norm_w, float eps,
                           const uint16_t* w_qkv, const uint16_t* qkv_bias, uint16_t* qkv,
                           uint16_t* k_layer, uint16_t* v_layer, int pos, int max_seqlen,
                           int num_heads, int head_dim, hipStream_t stream) {
  qd::QkvFrontParams p;
  const int rc = front_params(ctx, x, norm_w, eps, w_qkv, qkv_bias, qkv, k_layer, v_layer, pos,
                              max_seqlen, num_heads, head_dim, p);
  if (rc != QD_OK) return rc;
  hipError_t e = qd::launch_qkv_front(p, stream);
  if (e != hipSuccess) return hip_fail(e, "qkv_proj_rope_cache launch");
  return QD_OK;
}

// The fused front end + attention runs where the attention merges in its
// kernel by default.
constexpr int kFrontFusedMaxRows = kXMergeMaxRows;

int qd_qkv_proj_rope_cache_attention(qd_ctx* ctx, const uint16_t* x, const uint16_t* norm_w,
                                     float eps, const uint16_t* w_qkv, const uint16_t* qkv_bias,
                                     uint16_t* qkv, uint16_t* k_layer, uint16_t* v_layer,
                                     uint16_t* out, int pos, int max_seqlen, int num_heads,
                                     int head_dim, hipStream_t stream) {
  qd::QkvFrontParams f;
  int rc = front_params(ctx, x, norm_w, eps, w_qkv, qkv_bias, qkv, k_layer, v_layer, pos, max_seqlen,
                        num_heads, head_dim, f);
  if (rc != QD_OK) return rc;
  rc = check_attention_args(ctx, qkv, k_layer, v_layer, out, pos + 1, num_heads, head_dim);
  if (rc != QD_OK) return rc;
  const int hidden = num_heads * QD_HEAD_DIM;
  if (qd::overlaps(out, (size_t)hidden * 2, x, (size_t)hidden * 2) ||
      qd::overlaps(out, (size_t)hidden * 2, w_qkv, (size_t)3 * hidden * hidden * 2))
    return fail(QD_EINVAL, "out overlaps x or w_qkv");
  const int seqlen = pos + 1;
  const qd::AttnPlan plan = finish_plan(ctx, plan_auto(ctx, seqlen), seqlen);
  // One launch where the plan merges in the kernel with one workgroup per CU,
  // up to kFrontFusedMaxRows rows (measured on MI355X at 16 heads, cold, per
  // layer: 9.90 against 11.25 us for the two launches at 256 rows, 10.28
  // against 11.64 at 512, 11.12 against 12.22 at 1024, 12.94 against 13.94 at
  // 2048, 14.82 against 15.06 at 3072), and with out apart from qkv (whose
  // rows the producers store while splits finish); otherwise the two
  // launches, with the same outputs.
  const bool fused = seqlen <= kFrontFusedMaxRows && plan.variant == 1 && plan.xmerge && !plan.block_rows &&
                     (plan.depth == 1 || plan.depth == 2) &&
                     (num_heads == 8 || num_heads == 16) &&
                     std::max(num_heads * 16, plan.splits * num_heads) <= ctx->num_cus &&
                     !qd::overlaps(out, (size_t)hidden * 2, qkv, (size_t)3 * hidden * 2);
  if (!fused) {
    hipError_t e = qd::launch_qkv_front(f, stream);
    if (e != hipSuccess) return hip_fail(e, "qkv_proj_rope_cache launch");
    return run_attention(ctx, qkv, k_layer, v_layer, out, seqlen, plan_auto(ctx, seqlen), stream);
  }
  qd::AttnParams p = make_params(ctx, qkv, k_layer, v_layer, out, seqlen, plan);
  rc = next_xmerge_tag(ctx, p, stream);
  if (rc != QD_OK) return rc;
  const qd::FrontHandoff fh{ctx->ftag, ctx->force_front_local};
  const hipError_t e = qd::launch_qkv_attention(f, p, fh, plan, stream);
  if (e != hipSuccess) return hip_fail(e, "fused front end + attention launch");
  ctx->xcnt_sum += (unsigned)(plan.splits - 1);
  return QD_OK;
}

int qd_ctx_set_front_local(qd_ctx* ctx, int on) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  ctx->force_front_local = on != 0;
  return QD_OK;
}

}  // extern "C"

namespace {
int front_params(qd_ctx* ctx, const uint16_t* x, const uint16_t* norm_w, float eps,
                 const uint16_t* w_qkv, const uint16_t* qkv_bias, uint16_t* qkv, uint16_t* k_layer,
                 uint16_t* v_layer, int pos, int max_seqlen, int num_heads, int head_dim,
                 qd::QkvFrontParams& p) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  if (!x || !w_qkv || !qkv || !k_layer || !v_layer)
    return fail(QD_EINVAL, "x, w_qkv, qkv, k_layer and v_layer must be non-NULL");
  if (!aligned16(x) || !aligned16(w_qkv) || (norm_w && !aligned16(norm_w)))
    return fail(QD_EINVAL, "x, norm_w and w_qkv must be 16-byte aligned");
  if (((uintptr_t)qkv | (uintptr_t)k_layer | (uintptr_t)v_layer | (uintptr_t)qkv_bias) & 1u)
    return fail(QD_EINVAL, "fp16 buffers must be 2-byte aligned");
  if (head_dim != QD_HEAD_DIM) return fail(QD_EINVAL, "head_dim %d unsupported (must be 128)", head_dim);
  if (num_heads != ctx->cfg.num_heads)
    return fail(QD_EINVAL, "num_heads %d differs from the context's %d", num_heads, ctx->cfg.num_heads);
  const int hidden = num_heads * QD_HEAD_DIM;
  if (hidden % 512 != 0 || hidden > 4096)
    return fail(QD_EINVAL, "hidden size %d unsupported (multiple of 512, at most 4096)", hidden);
  if (!(eps >= 0.0f)) return fail(QD_EINVAL, "eps must be >= 0");
  if (max_seqlen < 1 || max_seqlen > ctx->cfg.max_seqlen)
    return fail(QD_EINVAL, "max_seqlen %d outside [1, %d]", max_seqlen, ctx->cfg.max_seqlen);
  if (pos < 0 || pos >= max_seqlen) return fail(QD_EINVAL, "pos %d outside [0, %d)", pos, max_seqlen);
  {
    const size_t qb = (size_t)3 * hidden * 2, hb = (size_t)hidden * 2;
    if (qd::overlaps(qkv, qb, x, hb) || qd::overlaps(qkv, qb, norm_w, hb) ||
        qd::overlaps(qkv, qb, w_qkv, qb * hidden) || qd::overlaps(qkv, qb, qkv_bias, qb))
      return fail(QD_EINVAL, "qkv overlaps x, norm_w, w_qkv or qkv_bias");
  }
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != ctx->device)
    return fail(QD_EINVAL, "current device %d is not the context's device %d", dev, ctx->device);
  p.x = x;
  p.norm_w = norm_w;
  p.eps = eps;
  p.w = w_qkv;
  p.bias = qkv_bias;
  p.qkv = qkv;
  p.k_layer = k_layer;
  p.v_layer = v_layer;
  p.rope_cs = ctx->rope_cs;
  p.row_stride = ctx->cfg.kv_row_stride;
  p.head_stride = ctx->cfg.kv_head_stride;
  p.pos = pos;
  p.num_heads = num_heads;
  return QD_OK;
}
}  // namespace

extern "C" {

int qd_decode_attention_plan(const qd_ctx* ctx, int seqlen, int* variant, int* num_splits) {
  if (!ctx || !variant || !num_splits) return fail(QD_EINVAL, "NULL argument");
  if (seqlen < 1 || seqlen > ctx->cfg.max_seqlen)
    return fail(QD_EINVAL, "seqlen %d outside [1, %d]", seqlen, ctx->cfg.max_seqlen);
  const qd::AttnPlan plan =
      plan_auto(ctx, seqlen);
  *variant = plan.variant;
  *num_splits = plan.splits;
  return QD_OK;
}

int qd_decode_attention_plan_detail(const qd_ctx* ctx, int seqlen, int entry, int num_splits,
                                    qd_attn_plan* plan) {
  if (!ctx || !plan) return fail(QD_EINVAL, "NULL argument");
  if (seqlen < 1 || seqlen > ctx->cfg.max_seqlen)
    return fail(QD_EINVAL, "seqlen %d outside [1, %d]", seqlen, ctx->cfg.max_seqlen);
  if (entry < 0 || entry > 2) return fail(QD_EINVAL, "entry %d is not 0, 1 or 2", entry);
  if (entry == 2 && num_splits > qd::kMaxSplits)
    return fail(QD_EINVAL, "num_splits %d above the maximum %d", num_splits, qd::kMaxSplits);
  const qd::AttnPlan p = finish_plan(ctx,
                                     entry == 0   ? plan_auto(ctx, seqlen)
                                     : entry == 1 ? plan_fused(seqlen)
                                                  : plan_split(ctx, seqlen, num_splits),
                                     seqlen);
  plan->variant = p.variant;
  plan->num_splits = p.splits;
  plan->rows_per_split = p.rows_per_split;
  plan->rows_per_tile = p.rows_per_tile;
  plan->waves = p.waves;
  plan->merge_in_kernel = p.xmerge;
  plan->loads_per_round = p.depth;
  plan->block_rows = p.block_rows;
  return QD_OK;
}

int qd_ctx_set_split_shape(qd_ctx* ctx, int waves, int rows_per_tile, int interleave) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  const bool off = waves == 0 && rows_per_tile == 0 && interleave == 0;
  const bool ok = (waves == 8 || waves == 4) && (rows_per_tile == 2 || rows_per_tile == 4) && interleave == 1;
  if (!off && !ok)
    return fail(QD_EINVAL, "split shape (%d waves, %d rows per tile, interleave %d) unsupported",
                waves, rows_per_tile, interleave);
  ctx->shape_waves = waves;
  ctx->shape_tile = rows_per_tile;
  ctx->shape_inter = interleave;
  return QD_OK;
}

int qd_ctx_set_merge(qd_ctx* ctx, int mode) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  if (mode != QD_MERGE_AUTO && mode != QD_MERGE_TWO_LAUNCHES && mode != QD_MERGE_IN_KERNEL)
    return fail(QD_EINVAL, "unknown merge mode %d", mode);
  ctx->merge_mode = mode;
  return QD_OK;
}

int qd_ctx_set_recompute_mask(qd_ctx* ctx, unsigned mask) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  ctx->recompute_mask = mask;
  return QD_OK;
}

int qd_ctx_set_scan_depth(qd_ctx* ctx, int depth) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  if (depth != 0 && depth != 1 && depth != 2 && depth != 4 && depth != QD_SCAN_ROLLING)
    return fail(QD_EINVAL, "scan depth must be 0, 1, 2, 4 or QD_SCAN_ROLLING, got %d", depth);
  ctx->scan_depth = depth;
  return QD_OK;
}

int qd_ctx_count_xmerges(qd_ctx* ctx, int on) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  ctx->count_merges = on != 0;
  return QD_OK;
}

int qd_ctx_xmerge_stats(const qd_ctx* ctx, unsigned long long* merges, unsigned long long* reads,
                        unsigned long long* rescans) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  const int H = ctx->cfg.num_heads;
  std::vector<unsigned> c((size_t)H * qd::kXCounterStride);
  const hipError_t e = hipMemcpy(c.data(), ctx->xcnt, c.size() * sizeof(unsigned), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpy of the merge counters");
  unsigned long long t[3] = {0ull, 0ull, 0ull};
  for (int h = 0; h < H; ++h)
    for (int i = 0; i < 3; ++i) t[i] += c[(size_t)h * qd::kXCounterStride + qd::kXStatMerges + i];
  if (merges) *merges = t[0];
  if (reads) *reads = t[1];
  if (rescans) *rescans = t[2];
  return QD_OK;
}

int qd_ctx_front_misses(const qd_ctx* ctx, unsigned long long* misses) {
  if (!ctx || !misses) return fail(QD_EINVAL, "NULL argument");
  const int H = ctx->cfg.num_heads;
  std::vector<unsigned> c((size_t)H * qd::kXCounterStride);
  const hipError_t e = hipMemcpy(c.data(), ctx->xcnt, c.size() * sizeof(unsigned), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpy of the merge counters");
  unsigned long long t = 0ull;
  for (int h = 0; h < H; ++h) t += c[(size_t)h * qd::kXCounterStride + qd::kXStatFrontMisses];
  *misses = t;
  return QD_OK;
}

int qd_ctx_xcd_period(const qd_ctx* ctx, int* period) {
  if (!ctx || !period) return fail(QD_EINVAL, "NULL argument");
  *period = ctx->num_xcd;
  return QD_OK;
}

int qd_xcd_placement(unsigned* xcc, int count) {
  if (!xcc || count < 1 || count > 65536) return fail(QD_EINVAL, "xcc must hold 1..65536 entries");
  unsigned* d = nullptr;
  hipError_t e = hipMalloc(&d, (size_t)count * sizeof(unsigned));
  if (e != hipSuccess) return hip_fail(e, "hipMalloc of the probe buffer");
  if ((e = qd::launch_xcd_probe(d, count, nullptr)) == hipSuccess)
    e = hipMemcpy(xcc, d, (size_t)count * sizeof(unsigned), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  return e == hipSuccess ? QD_OK : hip_fail(e, "XCD placement probe");
}

int qd_decode_attention(qd_ctx* ctx, const uint16_t* q, const uint16_t* k_layer,
                        const uint16_t* v_layer, uint16_t* out, int seqlen, int num_heads,
                        int head_dim, hipStream_t stream) {
  int rc = check_attention_args(ctx, q, k_layer, v_layer, out, seqlen, num_heads, head_dim);
  if (rc != QD_OK) return rc;
  const qd::AttnPlan plan =
      plan_auto(ctx, seqlen);
  return run_attention(ctx, q, k_layer, v_layer, out, seqlen, plan, stream);
}

int qd_decode_attention_stage(qd_ctx* ctx, const uint16_t* q, const uint16_t* k_layer,
                              const uint16_t* v_layer, uint16_t* out, int seqlen, int num_heads,
                              int head_dim, int stages, hipStream_t stream) {
  int rc = check_attention_args(ctx, q, k_layer, v_layer, out, seqlen, num_heads, head_dim);
  if (rc != QD_OK) return rc;
  if (stages < 1 || stages > (QD_STAGE_SCAN | QD_STAGE_MERGE))
    return fail(QD_EINVAL, "stages %d is not a non-empty set of QD_STAGE_SCAN, QD_STAGE_MERGE", stages);
  const qd::AttnPlan plan = finish_plan(ctx, plan_auto(ctx, seqlen), seqlen);
  if (stages == QD_STAGE_MERGE && (plan.variant == 0 || plan.xmerge))
    return fail(QD_EINVAL, "seqlen %d plans %s: there is no merge kernel to run alone", seqlen,
                plan.variant == 0 ? "one fused launch" : "the merge inside the scan kernel");
  return run_attention(ctx, q, k_layer, v_layer, out, seqlen, plan_auto(ctx, seqlen), stream,
                       stages);
}

int qd_decode_attention_fused(qd_ctx* ctx, const uint16_t* q, const uint16_t* k_layer,
                              const uint16_t* v_layer, uint16_t* out, int seqlen, int num_heads,
                              int head_dim, hipStream_t stream) {
  int rc = check_attention_args(ctx, q, k_layer, v_layer, out, seqlen, num_heads, head_dim);
  if (rc != QD_OK) return rc;
  return run_attention(ctx, q, k_layer, v_layer, out, seqlen, plan_fused(seqlen), stream);
}

int qd_decode_attention_split(qd_ctx* ctx, const uint16_t* q, const uint16_t* k_layer,
                              const uint16_t* v_layer, uint16_t* out, int seqlen, int num_heads,
                              int head_dim, int num_splits, hipStream_t stream) {
  int rc = check_attention_args(ctx, q, k_layer, v_layer, out, seqlen, num_heads, head_dim);
  if (rc != QD_OK) return rc;
  if (num_splits > qd::kMaxSplits)
    return fail(QD_EINVAL, "num_splits %d above the maximum %d", num_splits, qd::kMaxSplits);
  return run_attention(ctx, q, k_layer, v_layer, out, seqlen,
                       plan_split(ctx, seqlen, num_splits), stream);
}

int qd_decode_attention_noalloc(const uint16_t* q, const uint16_t* k_layer, const uint16_t* v_layer,
                                uint16_t* out, int seqlen, int num_heads, int head_dim,
                                long long kv_row_stride, long long kv_head_stride,
                                hipStream_t stream) {
  if (!q || !k_layer || !v_layer || !out)
    return fail(QD_EINVAL, "q, k_layer, v_layer and out must be non-NULL");
  if (!aligned16(q) || !aligned16(k_layer) || !aligned16(v_layer) || !aligned16(out))
    return fail(QD_EINVAL, "q, k_layer, v_layer and out must be 16-byte aligned");
  if (head_dim != QD_HEAD_DIM) return fail(QD_EINVAL, "head_dim %d unsupported (must be %d)", head_dim, QD_HEAD_DIM);
  if (num_heads < 1 || num_heads > 4096) return fail(QD_EINVAL, "num_heads %d outside [1, 4096]", num_heads);
  if (kv_row_stride < 1 || kv_head_stride < 1 || (kv_row_stride % 8) || (kv_head_stride % 8))
    return fail(QD_EINVAL, "kv strides must be positive multiples of 8 elements");
  if (seqlen < 1) return fail(QD_EINVAL, "seqlen %d must be >= 1", seqlen);
  // the kernels address a row as (32-bit byte offset) from a per-head base
  if ((long long)seqlen * kv_row_stride * 2 > 0xFFFFFF00LL)
    return fail(QD_EINVAL, "seqlen * kv_row_stride * 2 bytes must stay below 4 GiB");
  const size_t ob = (size_t)num_heads * QD_HEAD_DIM * 2;
  const size_t kvb = ((size_t)(seqlen - 1) * kv_row_stride + (size_t)(num_heads - 1) * kv_head_stride +
                      QD_HEAD_DIM) * 2;
  if (qd::overlaps(out, ob, k_layer, kvb) || qd::overlaps(out, ob, v_layer, kvb))
    return fail(QD_EINVAL, "out overlaps the k_layer or v_layer rows being read");
  int dev = -1, num_cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  e = hipDeviceGetAttribute(&num_cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess || num_cus < 1) return hip_fail(e, "hipDeviceGetAttribute(multiProcessorCount)");
  float* scratch_o = nullptr;
  float2* scratch_ml = nullptr;
  int rc = qd::static_scratch(&scratch_o, &scratch_ml);
  if (rc != QD_OK) return rc;
  // The plan qd_decode_attention picks with a default context of this device
  // and head count: such a context merges split plans inside the scan kernel,
  // and so runs fused plans only up to kFusedMaxRowsX rows, when the device's
  // dispatch is round-robin with a period dividing num_heads (probed once per
  // device; here into the static scratch, whose contents need not survive).
  // The partials are folded by a merge kernel here, which gives the in-kernel
  // merge's bits.
  int period = 0;
  rc = dispatch_period(dev, reinterpret_cast<unsigned*>(scratch_o), &period);
  if (rc != QD_OK) return rc;
  const bool ctx_merges_in_kernel = period > 0 && num_heads % period == 0;
  qd::AttnPlan plan = plan_auto(num_cus, num_heads, seqlen,
                                ctx_merges_in_kernel ? kFusedMaxRowsX : kFusedMaxRows,
                                ctx_merges_in_kernel);
  plan.depth = auto_depth(plan, false);
  const long long slots = (long long)num_heads * plan.splits;
  if (plan.variant == 1 && slots > qd::kStaticScratchSlots)
    return fail(QD_EINVAL,
                "%d heads x %d splits = %lld partial slots exceed the static scratch's %d "
                "(use qd_decode_attention with a context)",
                num_heads, plan.splits, slots, qd::kStaticScratchSlots);
  qd::AttnParams p;
  p.q = q;
  p.k = k_layer;
  p.v = v_layer;
  p.out = out;
  p.part_o = scratch_o;
  p.part_ml = scratch_ml;
  p.row_stride = kv_row_stride;
  p.head_stride = kv_head_stride;
  p.seqlen = seqlen;
  p.num_heads = num_heads;
  p.splits = plan.splits;
  p.rows_per_split = plan.rows_per_split;
  p.scale_log2 = (float)(1.4426950408889634 / std::sqrt(128.0));  // log2(e)/sqrt(128)
  p.q_batch_stride = 0;
  p.out_batch_stride = 0;
  p.num_cus = num_cus;
  p.split_stride = plan.splits;
  p.xpart = nullptr;      // two launches: the static scratch holds plain partials
  p.xcnt = nullptr;
  p.cnt_base = 0u;
  p.tag = 0u;
  p.recompute_mask = 0u;
  p.count_merges = 0;
  p.block_rows = plan.block_rows;
  p.long_inter = ctx_merges_in_kernel;
  e = qd::launch_decode_attention(p, plan, stream);
  if (e != hipSuccess) return hip_fail(e, "decode attention launch");
  return QD_OK;
}

int qd_prefill_attention(qd_ctx* ctx, const uint16_t* q, long long q_stride, const uint16_t* k_layer,
                         const uint16_t* v_layer, uint16_t* out, long long out_stride, int pos0,
                         int tokens, int num_heads, int head_dim, int mode, hipStream_t stream) {
  if (!ctx) return fail(QD_EINVAL, "ctx is NULL");
  if (!q || !k_layer || !v_layer || !out)
    return fail(QD_EINVAL, "q, k_layer, v_layer and out must be non-NULL");
  if (!aligned16(q) || !aligned16(k_layer) || !aligned16(v_layer) || !aligned16(out))
    return fail(QD_EINVAL, "q, k_layer, v_layer and out must be 16-byte aligned");
  if (head_dim != QD_HEAD_DIM || head_dim != ctx->cfg.head_dim)
    return fail(QD_EINVAL, "head_dim %d unsupported (must be %d)", head_dim, QD_HEAD_DIM);
  if (num_heads != ctx->cfg.num_heads)
    return fail(QD_EINVAL, "num_heads %d differs from the context's %d", num_heads, ctx->cfg.num_heads);
  if (mode != QD_GEMM_EXACT && mode != QD_GEMM_MFMA) return fail(QD_EINVAL, "unknown mode %d", mode);
  if (tokens < 1 || pos0 < 0 || (long long)pos0 + tokens > ctx->cfg.max_seqlen)
    return fail(QD_EINVAL, "positions [%d, %lld) outside [0, %d) or no tokens", pos0,
                (long long)pos0 + tokens, ctx->cfg.max_seqlen);
  const long long row = (long long)num_heads * QD_HEAD_DIM;
  if (q_stride < row || out_stride < row || (q_stride % 8) || (out_stride % 8))
    return fail(QD_EINVAL, "q_stride and out_stride must be multiples of 8 and >= %lld", row);
  const size_t ob = ((size_t)(tokens - 1) * out_stride + row) * 2;
  const size_t qb = ((size_t)(tokens - 1) * q_stride + row) * 2;
  const size_t kvb = ((size_t)(pos0 + tokens - 1) * ctx->cfg.kv_row_stride +
                      (size_t)(num_heads - 1) * ctx->cfg.kv_head_stride + QD_HEAD_DIM) * 2;
  if (qd::overlaps(out, ob, q, qb) || qd::overlaps(out, ob, k_layer, kvb) ||
      qd::overlaps(out, ob, v_layer, kvb))
    return fail(QD_EINVAL, "out overlaps q or the k_layer / v_layer rows being read");
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != ctx->device)
    return fail(QD_EINVAL, "current device %d is not the context's device %d", dev, ctx->device);
  if (mode == QD_GEMM_MFMA)
    return qd::attention_prefill_mfma(ctx, q, q_stride, k_layer, v_layer, out, out_stride, pos0,
                                      tokens, stream);
  return qd::attention_prefill(ctx, q, q_stride, k_layer, v_layer, out, out_stride, pos0, tokens,
                               stream);
}

int qd_max_splits(void) { return qd::kMaxSplits; }

const char* qd_last_error(void) { return g_err; }

const char* qd_version(void) { return "0.1.0"; }

}  // extern "C"
