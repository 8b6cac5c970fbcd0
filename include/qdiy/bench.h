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
 * scan-only call of the same seqlen.  Arguments as qd_decode_attention. */
int qd_decode_attention_stage(qd_ctx* ctx, const uint16_t* q, const uint16_t* k_layer,
                              const uint16_t* v_layer, uint16_t* out, int seqlen,
                              int num_heads, int head_dim, int stages, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* QDIY_BENCH_H */
