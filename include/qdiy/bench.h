/*
 * qdiy/bench.h -- measurement hooks of libqdiy.so.
 *
 * Not part of the drop-in boundary: no engine call site uses them.  They are
 * the counterpart of the reference's kernel benchmark, which launches and
 * times each Flash-Decoding kernel on its own (kernels/bench_fd_opt.cu:94-387,
 * timing at :139-147).
 */
#ifndef QDIY_BENCH_H
#define QDIY_BENCH_H

#include "qdiy/attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define QD_STAGE_SCAN 1   /* the scan kernel (the only kernel of a fused plan) */
#define QD_STAGE_MERGE 2  /* the merge kernel of a split plan */

/* The kernels of one qd_decode_attention call, selected by `stages` (a
 * non-empty set of QD_STAGE_*): QD_STAGE_SCAN | QD_STAGE_MERGE is the call
 * itself.  A loop of scan-only calls times the call's dominant kernel back
 * to back; a merge-only call folds whatever partials the context's scratch
 * holds (the last scan's), so its output is meaningful only right after a
 * scan-only call of the same seqlen.  A merge-only call at a length whose
 * plan has no merge kernel (fused, or merged inside the scan kernel) returns
 * QD_EINVAL.  Arguments as qd_decode_attention. */
int qd_decode_attention_stage(qd_ctx* ctx, const uint16_t* q, const uint16_t* k_layer,
                              const uint16_t* v_layer, uint16_t* out, int seqlen,
                              int num_heads, int head_dim, int stages, hipStream_t stream);

#define QD_MERGE_AUTO 0           /* in the scan kernel where it measured faster */
#define QD_MERGE_TWO_LAUNCHES 1   /* always a separate merge kernel */
#define QD_MERGE_IN_KERNEL 2      /* in the scan kernel wherever the context can */

/* How the context's split plans merge their partials (QD_MERGE_*); every mode
 * gives the same bits.  The scan kernel can fold them itself when the context
 * found round-robin workgroup dispatch whose period divides num_heads
 * (qd_ctx_xcd_period) and the grid is at most one workgroup per CU;
 * QD_MERGE_AUTO (the default) does so up to 3072 rows, where it measured
 * faster, and runs split plans with a merge kernel beyond.  A context that
 * merges in the kernel also runs fused plans only up to 128 rows (224
 * otherwise).  The other modes exist for A/B timing and tests. */
int qd_ctx_set_merge(qd_ctx* ctx, int mode);

/* Test hook of the in-kernel merge: the merging workgroup treats the partials
 * of every split whose index mod 32 is set in `mask` as not visible to it and
 * scans those splits again itself, as it does for partials written on another
 * XCD.  0 (the default) turns it off.  Outputs are unchanged either way. */
int qd_ctx_set_recompute_mask(qd_ctx* ctx, unsigned mask);

/* Tiles whose loads a wave of a split plan issues before it consumes them
 * (1, 2 or 4; consumed in the same order, so every depth gives the same
 * bits), or QD_SCAN_ROLLING: each wave issues tile i + 1's loads before it
 * consumes tile i (reported as loads_per_round 0; the same bits too); 0 (the
 * default) lets the planner choose.  For sweeps and tests. */
#define QD_SCAN_ROLLING (-1)
int qd_ctx_set_scan_depth(qd_ctx* ctx, int depth);

/* Shape of the context's split plans, for A/B timing and tests: `waves`
 * waves per workgroup, `rows_per_tile` rows per 16-lane group per tile, and,
 * with interleave 1, the rows dealt to the splits in blocks of waves * 4 *
 * rows_per_tile (qd_attn_plan.block_rows).  Supported: (8, 2, 1), (8, 4, 1),
 * (4, 4, 1), (4, 2, 1); (0, 0, 0) restores the planner's shape (whose plans
 * beyond 3072 rows are themselves interleaved: (4, 2, 1) up to 16384 rows,
 * (4, 4, 1) beyond, where the context can merge in the scan kernel).  Each
 * shape has its own summation order, so its bits differ from other shapes';
 * the plan of every call is reported by qd_decode_attention_plan_detail. */
int qd_ctx_set_split_shape(qd_ctx* ctx, int waves, int rows_per_tile, int interleave);

/* Test hook of qd_qkv_proj_rope_cache_attention's one-launch form: with on
 * nonzero, every split workgroup computes its head's front end itself, as it
 * does when the producers' words stay invisible to it (a producer ran on
 * another XCD).  Outputs are unchanged; 0 (the default) turns it off. */
int qd_ctx_set_front_local(qd_ctx* ctx, int on);

/* Split workgroups of qd_qkv_proj_rope_cache_attention's one-launch form that
 * computed their head's front end themselves because the producers' words
 * stayed invisible to them (summed over heads, over every call; those forced
 * by qd_ctx_set_front_local are not counted).  0 when the producers and the
 * splits of each head share an XCD, as the launch arranges.  Synchronous. */
int qd_ctx_front_misses(const qd_ctx* ctx, unsigned long long* misses);

/* Turns counting of in-kernel merges and their slot reads on (nonzero) or
 * off (the default: the counts are atomics issued after the output, and a
 * kernel ends only when they have completed, so they lengthen a call). */
int qd_ctx_count_xmerges(qd_ctx* ctx, int on);

/* Totals over the context's in-kernel merges (summed over heads; each total
 * wraps at 2^32): *merges heads merged and *reads reads of a head's slots by
 * its first merging wave (1 per merge when every partial was visible at the
 * first read), over the calls made while counting was on; *rescans splits a
 * merging workgroup scanned again because their partials stayed invisible to
 * it, over every call.  Synchronous (a device-to-host copy on the null
 * stream); any pointer may be null. */
int qd_ctx_xmerge_stats(const qd_ctx* ctx, unsigned long long* merges, unsigned long long* reads,
                        unsigned long long* rescans);

/* Round-robin period of workgroup dispatch over XCDs found at context
 * creation (8 on MI355X: workgroup i runs on XCD i mod 8), 1 if every
 * workgroup ran on one XCD, 0 if the placement was not round-robin. */
int qd_ctx_xcd_period(const qd_ctx* ctx, int* period);

/* The XCD (HW_REG_XCC_ID) each workgroup of one `count`-workgroup launch on
 * the current device ran on, into host array xcc[count].  Synchronous;
 * allocates a count-word device buffer.  The probe qd_ctx_create runs. */
int qd_xcd_placement(unsigned* xcc, int count);

#ifdef __cplusplus
}
#endif
#endif /* QDIY_BENCH_H */
