/*
 * qdiy/engine.h -- the .bin weight format and the single-GPU greedy decode
 * engine built on qdiy/attn.h and qdiy/decode.h, with the reference engine's
 * surface (SeaTheDestiny/LLM-inference-DIY, framework_src/qwen_infer.cu).
 *
 * .bin format (model_weights/convert_weights.py:105-185, read by
 * qwen_infer.cu:119-227): a 28-byte little-endian header of seven uint32
 *   magic 0x46445751, vocab_size, hidden_size, num_layers, num_heads,
 *   intermediate_size, max_seqlen
 * followed by fp16 tensors, each row-major and contiguous:
 *   wte [vocab][hidden]
 *   per layer: ln_1 [hidden], qkv_w [3*hidden][hidden], qkv_b [3*hidden],
 *              attn_proj_w [hidden][hidden], ln_2 [hidden],
 *              ffn_w1 [inter][hidden], ffn_w2 [inter][hidden],
 *              ffn_proj_w [hidden][inter]
 *   ln_f [hidden], lm_head [vocab][hidden]
 *
 * Engine (QwenEngine, qwen_infer.cu:64-737): one process, one GPU.  Weights are
 * uploaded once in file order; the KV cache is [layers][max_seqlen][hidden]
 * for K and for V.  A decode step runs, per layer, qd_qkv_proj_rope_cache,
 * qd_decode_attention, qd_proj_residual, qd_ffn_up_swiglu, qd_proj_residual,
 * then qd_lm_head_argmax, on the engine's own stream, and synchronises once to
 * return the token.  Prompt tokens before the last one run the same per-layer
 * path (no logits); the reference runs them through its FlashAttention
 * prefill (qwen_infer.cu:372-611).
 *
 * All calls return a qd_status (qdiy/attn.h); qd_last_error() has the text.
 */
#ifndef QDIY_ENGINE_H
#define QDIY_ENGINE_H

#include <stdint.h>

#include "qdiy/attn.h"
#include "qdiy/decode.h"

#ifdef __cplusplus
extern "C" {
#endif

#define QD_MODEL_MAGIC 0x46445751u
#define QD_MODEL_HEADER_BYTES 28

typedef struct qd_model_cfg {
  uint32_t vocab_size;
  uint32_t hidden_size;        /* num_heads * 128, a multiple of 512, <= 4096 */
  uint32_t num_layers;
  uint32_t num_heads;
  uint32_t intermediate_size;  /* a multiple of 8, at most 8192 */
  uint32_t max_seqlen;
} qd_model_cfg;

/* Size in bytes of a .bin image (header + tensors) for cfg; -1 if invalid. */
long long qd_model_image_bytes(const qd_model_cfg* cfg);

/* Writes a complete .bin image into `image` (qd_model_image_bytes(cfg)
 * bytes): the header, then every tensor drawn from a counter-based
 * generator -- element i of the image gets the sum of four 16-bit uniforms
 * from splitmix64(seed, i), centred and scaled to standard deviation `std`
 * (an Irwin-Hall approximation of N(0, std^2)), rounded to fp16 -- except the
 * RMSNorm weights ln_1, ln_2 and ln_f, which are 1.0.  Deterministic for a
 * seed, independent of nthreads (>= 1 host threads). */
int qd_model_fill_random(void* image, long long bytes, const qd_model_cfg* cfg, uint64_t seed,
                         float std, int nthreads);

/* qd_model_fill_random into a file at `path`. */
int qd_model_write_random(const char* path, const qd_model_cfg* cfg, uint64_t seed, float std);

typedef struct qd_engine qd_engine;

/* Loads a .bin file (QwenEngine::QwenEngine, qwen_infer.cu:119-270). */
int qd_engine_create(const char* path, qd_engine** out);

/* Same from an in-memory .bin image of `bytes` bytes (copied to the GPU). */
int qd_engine_create_from_image(const void* image, long long bytes, qd_engine** out);

/* Frees the engine (QwenEngine::~QwenEngine).  NULL is accepted. */
int qd_engine_destroy(qd_engine* eng);

/* The model configuration from the header. */
int qd_engine_config(const qd_engine* eng, qd_model_cfg* cfg);

/* Clears the KV cache and activations (QwenEngine::reset, qwen_infer.cu:318-346). */
int qd_engine_reset(qd_engine* eng);

/* Runs the n tokens at positions *pos, *pos + 1, ... through all layers,
 * filling their KV-cache rows, and advances *pos by n (the role of
 * QwenEngine::prefill, qwen_infer.cu:372-611, which the reference runs for
 * prompt tokens 0..N-2).  In the default mode (QD_GEMM_EXACT) the KV rows it
 * writes are bit-identical to feeding the tokens one by one through
 * qd_engine_step. */
int qd_engine_prefill(qd_engine* eng, const int* tokens, int n, int* pos);

/* Selects how qd_engine_prefill multiplies its projections and computes its
 * attention (the modes of qd_gemm_nt and qd_prefill_attention):
 * QD_GEMM_EXACT (the default: bit-identical to token-by-token decode) or
 * QD_GEMM_MFMA (the matrix cores for both, as the reference's prefill uses its
 * tensor cores; the KV rows then differ from token-by-token decode by fp32
 * summation order and fp16 softmax weights, and greedy tokens after the prompt
 * can differ at near-ties).  Projections whose k is not a multiple of 64 stay
 * exact.  The matrix-core mode prefills up to 2048 tokens per pass (256 in the
 * exact mode): selecting it first grows the engine's prefill scratch to that
 * many tokens (~127 MB at Qwen-1.8B's shape) and returns QD_ENOMEM, keeping the
 * previous mode and scratch, if that allocation fails. */
int qd_engine_set_prefill_mode(qd_engine* eng, int mode);

/* One greedy decode step for `token` at position `pos`
 * (QwenEngine::step, qwen_infer.cu:614-735): *next_token receives the argmax
 * of the logits (ties to the lowest index). */
int qd_engine_step(qd_engine* eng, int token, int pos, int* next_token);

/* Copies the last step's vocab_size fp16 logits to host memory. */
int qd_engine_logits(qd_engine* eng, uint16_t* host_logits);

/* Copies KV-cache rows [pos0, pos0 + n) of `layer` to host memory: n x
 * hidden_size fp16 values of K (rotated) and of V, after the engine's queued
 * work.  The reference engine keeps its caches as members a test or tool can
 * read (d_kv_cache_k / d_kv_cache_v, qwen_infer.cu:245-249); this is that
 * access.  Either pointer may be NULL. */
int qd_engine_kv_rows(qd_engine* eng, int layer, int pos0, int n, uint16_t* host_k,
                      uint16_t* host_v);

/* main()'s per-request loop (qwen_infer.cu:780-817) without the printing:
 * prefill prompt[0..n_prompt-2] from position 0, then greedy steps from the
 * last prompt token, writing up to max_new tokens to out_tokens.  With
 * stop_at_eos, stops before emitting 151645 or 151643 as the reference does.
 * *n_out receives the number of tokens written. */
int qd_engine_generate(qd_engine* eng, const int* prompt, int n_prompt, int max_new,
                       int stop_at_eos, int* out_tokens, int* n_out);

#ifdef __cplusplus
}
#endif
#endif /* QDIY_ENGINE_H */
