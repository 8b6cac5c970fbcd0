// Internal declarations shared by the C-ABI layer and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qdiy/attn.h"

namespace qd {

// Largest split count (workgroups per head).  Scratch per context:
// num_heads * kMaxSplits * (128 + 2) floats (2.1 MB at 16 heads).
constexpr int kMaxSplits = 256;

// Partial slots (num_heads * splits) of the allocation-free entry point's
// static device scratch: 1024 * (128 + 2) floats = 520 KiB per GPU, enough for
// every automatic split plan on devices of up to 512 compute units.
constexpr int kStaticScratchSlots = 1024;

// The calling thread's current device's copy of the static scratch, as device
// addresses: O partials [kStaticScratchSlots][128], then the (m, l) pairs.
// The address is looked up with hipGetSymbolAddress on the first call per
// device and kept.  Returns a QD_* status (message via fail()).
int static_scratch(float** part_o, float2** part_ml);

// Split planner constants, from measured sweeps on MI355X (16 heads, cold KV):
// one split workgroup per CU in total, each split at least kMinRowsPerSplit
// rows.  (Two workgroups per CU between 1025 and 2048 rows measured within
// 0.1 us of one; one per CU keeps every split of a head on one XCD.)
constexpr int kMinRowsPerSplit = 16;

// The split plan of a query over `seqlen` rows when the caller names no split
// count: num_cus / num_heads workgroups per head, at most one per
// kMinRowsPerSplit rows, rows per split rounded up to a multiple of 4 (one
// load instruction covers 4 rows) and no empty workgroups.  The host planner
// and the batched prefill kernels, which plan every query for itself, both
// evaluate this one function.
__host__ __device__ inline void auto_split(int seqlen, int num_cus, int num_heads, int* splits, int* rows) {
  int s = num_cus / num_heads;
  const int by_rows = (seqlen + kMinRowsPerSplit - 1) / kMinRowsPerSplit;
  if (s > by_rows) s = by_rows;
  if (s < 1) s = 1;
  if (s > kMaxSplits) s = kMaxSplits;
  int r = (seqlen + s - 1) / s;
  r = (r + 3) & ~3;
  *rows = r;
  *splits = (seqlen + r - 1) / r;
}

// Per-launch arguments of the decode-attention kernels.  Offsets are in fp16
// elements.
struct AttnParams {
  const uint16_t* q;      // [H][128]
  const uint16_t* k;      // layer base; (pos, h, d) at pos*row_stride + h*head_stride + d
  const uint16_t* v;
  uint16_t* out;          // [H][128]
  float* part_o;          // [H][splits][128] unnormalised fp32 partial outputs
  float2* part_ml;        // [H][splits] (running max in log2 units, running sum)
  long long row_stride;
  long long head_stride;
  int seqlen;
  int num_heads;
  int splits;             // workgroups per head
  int rows_per_split;
  float scale_log2;       // log2(e) / sqrt(128)
  // Batched calls (prefill): grid.y = tokens; token b reads q + b*q_batch_stride,
  // writes out + b*out_batch_stride and attends over seqlen + b rows.  Zero
  // strides and grid.y = 1 for a single call.
  long long q_batch_stride;
  long long out_batch_stride;
  // Batched split calls only: each token plans itself with auto_split(seqlen +
  // b, num_cus, num_heads, ...); its partials sit at slots (b * num_heads + h) *
  // split_stride + c.
  int num_cus;
  int split_stride;
  // Split plans with interleaved blocks (0 for contiguous ranges): the rows
  // form blocks of block_rows (one load round of a workgroup), dealt to the
  // splits in turn -- split c scans blocks c, c + splits, ... (see
  // interleaved_rows) -- so that at any time the grid reads one run of rows.
  int block_rows;
  // In-kernel merge (decode_attention_xmerge_kernel) only: tagged slots
  // [H][kXMaxSplits][kXSlotWords] (value, tag) words, per-head arrival
  // counters (kXCounterStride apart; every head's counter holds cnt_base when
  // the call starts and only grows), this call's tag, and a test hook: splits
  // whose index mod 32 is set are treated as not visible.
  float2* xpart;
  unsigned* xcnt;
  unsigned cnt_base;
  unsigned tag;
  unsigned recompute_mask;
  int count_merges;       // nonzero: add to the merge and read totals (rescans always)
  // Batched split calls only: nonzero where the context's split plans can merge
  // in the scan kernel, so that each token's auto_plan deals the rows of a
  // long query in interleaved blocks, as qd_decode_attention plans it.
  int long_inter;
};

// In-kernel merge limits: at most kXMaxSplits splits per head (the merge
// reads them in one batch of loads); counters 128 bytes apart.  Word 0 of a
// head's counter block is its arrival counter; words kXStatMerges,
// kXStatReads and kXStatRescans total its merges, reads of its slots and
// splits scanned again (qd_ctx_xmerge_stats); word kXStatFrontMisses the
// splits of qkv_attention_kernel that computed the head's front end
// themselves because the producers' words stayed invisible (qd_ctx_front_misses).
constexpr int kXMaxSplits = 64;
constexpr int kXCounterStride = 32;
constexpr int kXSlotBytes = 1152;
constexpr int kXStatMerges = 1;
constexpr int kXStatReads = 2;
constexpr int kXStatRescans = 3;
constexpr int kXStatFrontMisses = 4;

struct RopeParams {
  uint16_t* qkv;          // [3][H][128]
  const uint16_t* bias;   // [3][H][128] or null
  uint16_t* k_layer;
  uint16_t* v_layer;
  const float2* rope_cs;  // [max_seqlen][64] (cos, sin)
  long long row_stride;
  long long head_stride;
  int pos;
  int num_heads;
};

// Attention front end of one decode layer: [RMSNorm] -> QKV GEMV -> bias ->
// RoPE -> KV append.  hidden = num_heads * 128, a multiple of 512 up to 4096.
struct QkvFrontParams {
  const uint16_t* x;      // [hidden] layer input
  const uint16_t* norm_w; // [hidden] RMSNorm weight, or null for no norm
  float eps;
  const uint16_t* w;      // [3*hidden][hidden] QKV weight, [out][in]
  const uint16_t* bias;   // [3*hidden] or null
  uint16_t* qkv;          // [3*hidden] out: rotated Q, biased K and V
  uint16_t* k_layer;
  uint16_t* v_layer;
  const float2* rope_cs;  // [max_seqlen][64] (cos, sin)
  long long row_stride;
  long long head_stride;
  int pos;
  int num_heads;
};

// out[n] = half(res[n] + half(W[n] . x)) for n < n_out; W is [n_out][k_in]
// ([out][in]), k_in a multiple of 8.  res and out may alias.
struct ProjResidualParams {
  const uint16_t* x;
  const uint16_t* w;
  const uint16_t* res;
  uint16_t* out;
  int n_out;
  int k_in;
};

// act[i] = half(g * (u / (1 + exp(-u)))) with g = half(W1[i] . xn),
// u = half(W2[i] . xn), xn = RMSNorm(x) * norm_w; W1/W2 are [inter][hidden].
struct FfnUpParams {
  const uint16_t* x;
  const uint16_t* norm_w;
  float eps;
  const uint16_t* w1;
  const uint16_t* w2;
  uint16_t* act;
  int hidden;
  int inter;
};

// logits[v] = half(W[v] . xn) for v < vocab, xn = RMSNorm(x) * norm_w; each
// workgroup also writes its best (logit, lowest index) as a packed key.
struct LmHeadParams {
  const uint16_t* x;
  const uint16_t* norm_w;
  float eps;
  const uint16_t* w;
  uint16_t* logits;
  unsigned long long* part;
  int vocab;
  int hidden;
};

// Rows per wave and waves per workgroup of the lm_head kernel; the number of
// per-workgroup keys for a vocabulary follows from them.
constexpr int kLmRowsPerWave = 8;
constexpr int kLmWaves = 4;
inline int lm_head_parts(int vocab) {
  const int rows = kLmRowsPerWave * kLmWaves;
  return (vocab + rows - 1) / rows;
}

// Batched GEMV of the prefill: Y[t][n] = sum_k X[t][k] W[n][k] for t < t_count,
// n < n, in the decode kernels' summation order; X rows ldx elements apart, Y
// (and the residual R, read at the same offsets) ldy apart.  k a multiple of 8,
// at most 8192.
struct BatchedGemvParams {
  const uint16_t* x;
  long long ldx;
  const uint16_t* w;
  int n;
  int k;
  int t;
  uint16_t* y;
  long long ldy;
  const uint16_t* res;    // epilogue 1 only
  // Split-K form of the MFMA product only: slice z of K (kslice wide) writes
  // its fp32 sums to part + z * t * n ([t][n] rows); set by launch_gemm_mfma_split.
  float* part;
  int kslice;
  // Joint gate/up form only (launch_gemm_mfma_swiglu): W2, the up weight, with
  // w as W1 and y = act.
  const uint16_t* w2;
  // Exact two-row form only: tokens per workgroup (0: 32); set by launch_gemv_batched.
  int tok_per_wg = 0;
};

// Causal prefill attention of `tokens` queries at positions pos0, pos0 + 1, ...
// on the matrix cores: query t (Q row q + t*q_stride, head h at + h*128)
// attends over cache rows [0, pos0 + t], its output row at out + t*out_stride.
struct FlashPrefillParams {
  const uint16_t* q;
  long long q_stride;
  const uint16_t* k;      // layer base; (pos, h, d) at pos*row_stride + h*head_stride + d
  const uint16_t* v;
  long long row_stride;
  long long head_stride;
  uint16_t* out;
  long long out_stride;
  int pos0;
  int tokens;
  int num_heads;
  float scale_log2;       // log2(e) / sqrt(128)
};

// Launch plan of one decode-attention call.
struct AttnPlan {
  int variant;            // 0 fused, 1 split
  int splits;             // workgroups per head
  int rows_per_split;     // rows each workgroup scans (the longest split's when interleaved)
  int rows_per_tile;      // rows per group per tile (template U)
  int waves;              // waves per split workgroup (4, 8 or 16)
  int xmerge;             // split plans: merge inside the scan kernel (one launch)
  int depth;              // 4-wave split plans: tiles per load round (1, 2 or 4; same bits)
  int block_rows;         // split plans: interleaved blocks of this many rows, 0 contiguous
};

// Rows of split c when the rows [0, seqlen) form blocks of block_rows dealt to
// `splits` splits in turn (split c takes blocks c, c + splits, ...; the last
// block may be short).  Its j-th row is row ((j / block_rows) * splits + c) *
// block_rows + j % block_rows of the layer.
__host__ __device__ inline int interleaved_rows(int seqlen, int block_rows, int splits, int c) {
  const int full = seqlen / block_rows, rem = seqlen % block_rows;
  const int nfull = full > c ? (full - 1 - c) / splits + 1 : 0;
  return nfull * block_rows + (rem > 0 && full % splits == c ? rem : 0);
}

// Longest automatic split plan with contiguous row ranges where split plans
// merge in the scan kernel (and longest length the automatic plan merges in
// the scan kernel with such ranges).
constexpr int kXMergeMaxRows = 3072;
// Longest automatic plan of 2-row tiles in 32-row interleaved blocks; longer
// ones take 4-row tiles in 64-row blocks.  (A block is one load round of a
// 4-wave workgroup: 4 waves x 4 groups x rows per tile.)
constexpr int kLongTile2MaxRows = 16384;

// The automatic split plan of a query over seqlen rows: auto_split's split
// count and rows per split, with the rows in contiguous ranges (*block = 0),
// or -- beyond kXMergeMaxRows rows, where the caller's split plans can merge
// in the scan kernel (merges_in_kernel: dispatch round-robin over the XCDs
// with a period dividing num_heads), with at most kXMaxSplits splits and one
// workgroup per CU -- dealt to the splits in interleaved blocks of 32 rows
// (2-row tiles of 4-wave workgroups) up to kLongTile2MaxRows rows and of 64
// rows (4-row tiles) beyond (*block; *rows then split 0's count, the most).
// Interleaved, at any time the grid reads one run of rows and the merge runs
// in the scan kernel; the 2-row plans' waves keep their next tile's loads in
// flight while they consume one (finish_plan's depth 0).  Measured on MI355X
// at 16 heads (cold, us per call; contiguous ranges with a merge kernel /
// 64-row blocks / 32-row blocks rolling): 4096 rows 9.71 / 9.41-9.78 / 9.25,
// 8192 14.74 / 14.15-14.46 / 13.78, 16384 24.00 / 23.44-23.57 / 23.28, 20480
// - / 27.44 / 27.92, 32768 41.54 / 40.79-41.80 / 42.68.  The host planner and
// the batched prefill kernels, which plan every query for itself, both
// evaluate this one function.
__host__ __device__ inline void auto_plan(int seqlen, int num_cus, int num_heads, bool merges_in_kernel,
                                          int* splits, int* rows, int* block) {
  auto_split(seqlen, num_cus, num_heads, splits, rows);
  *block = 0;
  if (merges_in_kernel && seqlen > kXMergeMaxRows && *splits <= kXMaxSplits &&
      (long long)*splits * num_heads <= num_cus) {
    const int b = seqlen <= kLongTile2MaxRows ? 32 : 64;
    const int nblocks = (seqlen + b - 1) / b;
    if (*splits > nblocks) *splits = nblocks;
    *rows = interleaved_rows(seqlen, b, *splits, 0);
    *block = b;
  }
}

// Error reporting of the C ABI: records a printf-style message for
// qd_last_error() on this host thread and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }
inline bool aligned2(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1u) == 0; }
// Whether byte ranges [a, a + na) and [b, b + nb) share a byte (null or empty
// ranges never do).  The entry points reject outputs that overlap inputs other
// workgroups are still reading.
inline bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  if (!a || !b || na == 0 || nb == 0) return false;
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + nb && y < x + na;
}

// stages: kStageScan launches the scan kernel (the only kernel of a fused
// plan), kStageMerge the merge kernel of a split plan; a call is both.
constexpr int kStageScan = 1;
constexpr int kStageMerge = 2;
// A split plan with plan.xmerge is one launch (scan and merge in one kernel;
// kStageScan launches it, kStageMerge alone launches nothing).
hipError_t launch_decode_attention(const AttnParams& p, const AttnPlan& plan, hipStream_t stream,
                                   int stages = kStageScan | kStageMerge);
// The attention front end (f: qkv_front_kernel's work) and an in-kernel-merge
// split plan's attention over f.pos + 1 rows (p, plan) in one launch, with
// the outputs of the two separate launches, bit for bit.  Requires plan.xmerge
// with 4-wave contiguous splits, num_heads 8 or 16 and a grid of at most
// num_cus workgroups (hipErrorInvalidValue otherwise, nothing launched).
// Fused front end + attention (qkv_attention_kernel) only, kept out of
// AttnParams, which every attention kernel takes: tagged words [H][3][128]
// (value, tag) of each head's rotated Q, rotated K row and V row at position
// seqlen - 1, and a test hook (nonzero: every split computes its head's front
// end itself, as it does when the words stay invisible to it).
struct FrontHandoff {
  float2* ftag;
  int force_local;
};
hipError_t launch_qkv_attention(const QkvFrontParams& f, const AttnParams& p, const FrontHandoff& fh,
                                const AttnPlan& plan,
                                hipStream_t stream);
// Writes the XCD index (HW_REG_XCC_ID) of each of `grid` one-wave workgroups
// to out[0..grid): the dispatch placement the in-kernel merge relies on for
// speed (every split of a head on one XCD).
hipError_t launch_xcd_probe(unsigned* out, int grid, hipStream_t stream);

// Period n of a round-robin placement xcc[i] = (xcc[0] + i) mod n over XCDs
// 0..n-1 (1 if all are equal), or 0 if the placement is not of that form.
inline int round_robin_period(const unsigned* xcc, int count) {
  unsigned hi = 0;
  bool same = true;
  for (int i = 0; i < count; ++i) {
    hi = xcc[i] > hi ? xcc[i] : hi;
    same = same && xcc[i] == xcc[0];
  }
  if (same) return 1;
  const unsigned n = hi + 1;
  for (int i = 1; i < count; ++i)
    if (xcc[i] != (xcc[i - 1] + 1) % n) return 0;
  return count >= (int)n ? (int)n : 0;
}
// Fused (one 16-wave workgroup per head, 4-row tiles) attention of `tokens`
// queries at once, token b over p.seqlen + b rows: the arithmetic of the fused
// plan of qd_decode_attention, query by query.
hipError_t launch_decode_attention_fused_batch(const AttnParams& p, int tokens, hipStream_t stream);
// Split attention of `tokens` queries at once, token b over p.seqlen + b rows,
// each under its own auto_split plan (the plan qd_decode_attention picks for
// that length): one scan launch of num_heads * p.split_stride workgroups per
// token (those past a token's split count exit at once) and one merge launch.
// Every token's plan must have rows_per_tile tile rows.
hipError_t launch_decode_attention_split_batch(const AttnParams& p, int rows_per_tile, int tokens,
                                               hipStream_t stream);
hipError_t launch_qkv_bias_rope_cache(const RopeParams& p, hipStream_t stream);
hipError_t launch_qkv_front(const QkvFrontParams& p, hipStream_t stream);
hipError_t launch_proj_residual(const ProjResidualParams& p, hipStream_t stream);
hipError_t launch_ffn_up(const FfnUpParams& p, hipStream_t stream);
// lm_head kernel, then the one-workgroup reduction of its keys into *token.
hipError_t launch_lm_head_argmax(const LmHeadParams& p, int* token, hipStream_t stream);


// Prefill kernels (qd_prefill.hip).  epi 0: Y = half(sum); epi 1: Y = half(R + half(sum)).
hipError_t launch_rmsnorm_batched(const uint16_t* x, const uint16_t* w, float eps, uint16_t* xn,
                                  int hidden, int T, hipStream_t stream);
hipError_t launch_gemv_batched(const BatchedGemvParams& p, int epi, hipStream_t stream);
// The same product on the matrix cores (fp32 accumulation in the hardware's
// order, not bit-reproducible on the host); p.k must be a multiple of 64.
hipError_t launch_gemm_mfma(const BatchedGemvParams& p, int epi, hipStream_t stream);
// The same, allowed to split K over up to 8 slices when the tile grid leaves
// CUs idle: fp32 partial sums in `workspace` (as many slices as it holds),
// then one launch folds them in slice order and applies the epilogue.
// Otherwise, and without a workspace, it is launch_gemm_mfma.
constexpr size_t kGemmSplitWsBytes = (size_t)64 << 20;
hipError_t launch_gemm_mfma_split(const BatchedGemvParams& p, int epi, float* workspace,
                                  size_t workspace_bytes, hipStream_t stream);
// act[t][i] = half(g * (u / (1 + exp(-u)))) with g = half(X W1^T), u = half(X W2^T)
// (p.w = W1, p.w2 = W2, p.n = inter, p.y = act) in one matrix-core launch, the
// SwiGLU applied in the GEMM's epilogue: from 128 tokens (act 8-byte aligned,
// ldy a multiple of 4) the 192 x 256 or 128 x 128 ring tile, else the 64 x 64
// tile.
// hipErrorNotSupported (nothing launched) unless k is a multiple of 64: the
// caller then runs the two projections and launch_swiglu_batched.
hipError_t launch_gemm_mfma_swiglu(const BatchedGemvParams& p, hipStream_t stream);
hipError_t launch_rope_batched(uint16_t* qkv, const uint16_t* bias, uint16_t* k_layer,
                               uint16_t* v_layer, const float2* rope_cs, long long row_stride,
                               long long head_stride, int pos0, int num_heads, int T,
                               hipStream_t stream);
// act (rows x cols, packed) from g and u at row stride ld.
hipError_t launch_swiglu_batched(const uint16_t* g, const uint16_t* u, uint16_t* act, int rows,
                                 int cols, long long ld, hipStream_t stream);
hipError_t launch_embed(const uint16_t* wte, const int* tokens, uint16_t* x, int hidden, int T,
                        hipStream_t stream);
// qd_flash_prefill.hip: one workgroup per (head, 64 queries), eight waves.
hipError_t launch_flash_prefill(const FlashPrefillParams& p, hipStream_t stream);

}  // namespace qd

struct qd_ctx;

namespace qd {
// Attention of `tokens` consecutive queries at positions pos0, pos0 + 1, ...
// (query t over pos0 + t + 1 rows; q and out rows q_stride / out_stride
// elements apart), each with the arithmetic of qd_decode_attention's own plan
// for its length: the fused-plan queries in one batched launch, the split-plan
// queries in batched scan + merge pairs, one per run of queries that share a
// tile depth.
int attention_prefill(qd_ctx* ctx, const uint16_t* q, long long q_stride, const uint16_t* k,
                      const uint16_t* v, uint16_t* out, long long out_stride, int pos0, int tokens,
                      hipStream_t stream);
// The same queries in one causal FlashAttention launch on the matrix cores.
int attention_prefill_mfma(qd_ctx* ctx, const uint16_t* q, long long q_stride, const uint16_t* k,
                           const uint16_t* v, uint16_t* out, long long out_stride, int pos0,
                           int tokens, hipStream_t stream);
}  // namespace qd

struct qd_ctx {
  qd_cfg cfg;
  int device;
  int num_cus;            // compute units of the device (256 on MI355X)
  float2* rope_cs;        // [max_seqlen][64]
  float* part_o;          // [H][kMaxSplits][128]
  float2* part_ml;        // [H][kMaxSplits]
  // Partials of batched split prefill attention, allocated on first use:
  // [pf_tokens][H][pf_stride] slots of (128 + 2) floats.
  float* pf_part_o;
  float2* pf_part_ml;
  int pf_tokens;
  int pf_stride;
  // In-kernel merge of split plans: tagged slots, arrival counters, the last
  // call's tag; num_xcd is the round-robin period of workgroup dispatch found
  // at creation (0 if dispatch was not round-robin), xmerge_ok whether
  // num_heads is a multiple of it; merge_mode QD_MERGE_*; recompute_mask the
  // test hook of AttnParams.
  float2* xpart;
  unsigned* xcnt;
  float2* ftag;           // [H][3][128] tagged words of the fused front end + attention
  unsigned xtag;
  unsigned xcnt_sum;      // value of every head's arrival counter between calls
  int num_xcd;
  int xmerge_ok;
  int merge_mode;
  unsigned recompute_mask;
  int count_merges;
  int scan_depth;         // 0: the planner's tiles per load round; else forced for split plans
  // Split-plan shape forced by qd_ctx_set_split_shape (0: the planner's).
  int shape_waves;
  int shape_tile;
  int shape_inter;
  int force_front_local;  // qd_ctx_set_front_local
};
