/* rpg_hip.h -- token-level and kernel-level C entry points of the MI355X
 * engine, below the chat ABI of rpg_engine.h.
 *
 * These replace the reference's internal C++ seams for this path, which its
 * own parity tools and benchmarks drive (reference src/qwen3.h:83-142,
 * src/sampler.h:35-65, src/quant.h, src/matmul.h:35-64). Plain pointers and
 * sizes, no C++ types; host buffers in and out unless a name says "dev".
 * Return: >= 0 success (handles, counts), < 0 failure with the message in
 * rpg_hip_last_error(). Handles are int32 from 1, never reused.
 */
#ifndef RPG_HIP_H
#define RPG_HIP_H

#include <stdint.h>

#if defined(__GNUC__)
#define RPG_HIP_API __attribute__((visibility("default")))
#else
#define RPG_HIP_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

RPG_HIP_API const char* rpg_hip_last_error(void);

/* Number of visible GPUs (0 when none; never fails). */
RPG_HIP_API int32_t rpg_hip_device_count(void);

/* ---- model: reference Model::Load (src/model.cc:147-281) */
RPG_HIP_API int32_t rpg_hip_model_load(const char* gguf_path, int32_t max_pos);
RPG_HIP_API void rpg_hip_model_free(int32_t model);
/* out[9] = n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate,
 *          vocab, context_length, eos_id */
RPG_HIP_API int32_t rpg_hip_model_config(int32_t model, int32_t* out);
/* Bytes read from HBM for weights per decode token (all matrices incl.
 * lm_head, norms, one embedding row). */
RPG_HIP_API int64_t rpg_hip_model_decode_bytes(int32_t model);
/* RoPE table row of position pos: hd floats = cos(hd/2) | sin(hd/2)
 * (reference src/model.cc:122-145). */
RPG_HIP_API int32_t rpg_hip_model_rope_row(int32_t model, int64_t pos, float* out);

/* ---- session: KV cache + token loop (reference src/kv_cache.h, src/qwen3.h) */
RPG_HIP_API int32_t rpg_hip_session_new(int32_t model, int64_t max_seq);
RPG_HIP_API void rpg_hip_session_free(int32_t session);
RPG_HIP_API int64_t rpg_hip_session_len(int32_t session);
RPG_HIP_API int32_t rpg_hip_session_set_len(int32_t session, int64_t len);

/* ForwardFull with a cache (reference src/qwen3.cc:208-290): append n ids at
 * positions len..len+n-1. last_logits[vocab] and all_logits[n*vocab] may be
 * NULL. */
RPG_HIP_API int32_t rpg_hip_prefill(int32_t session, const int32_t* ids, int64_t n, float* last_logits,
                                    float* all_logits);

/* Generate (reference src/qwen3.cc:302-355). first_logits == NULL continues
 * from the last device logits. temperature <= 0 is greedy; top_k / top_p /
 * seed as SampleOptions (reference src/sampler.h:35-45). step_logits
 * (optional) receives [returned, vocab]. Returns the number of ids written to
 * out_ids (capacity max_tokens). */
RPG_HIP_API int32_t rpg_hip_generate(int32_t session, const float* first_logits, int32_t max_tokens,
                                     float temperature, int32_t top_k, float top_p, uint64_t seed,
                                     const int32_t* stop_ids, int32_t n_stop, int32_t* out_ids,
                                     float* step_logits);

/* Generate for n sessions of one model at once (1 <= n <= 8): each session
 * continues from its device logits with its own temperature[i], top_k[i],
 * top_p[i], seed[i] and produces max_tokens ids into out_ids[i * max_tokens
 * ...], the tokens it would produce alone (reference src/qwen3.cc:302-355 per
 * session); one decode step forwards all n tokens, each weight matrix read
 * once. No stop ids: every session needs room for max_tokens positions.
 * step_logits (optional, [n][max_tokens][vocab]) receives each session's
 * logits after each generated token (parity probe); decode_ms (optional)
 * the device time of the steps. Returns max_tokens. */
RPG_HIP_API int32_t rpg_hip_generate_batch(const int32_t* sessions, int32_t n, int32_t max_tokens,
                                           const float* temperature, const int32_t* top_k, const float* top_p,
                                           const uint64_t* seed, int32_t* out_ids, float* step_logits,
                                           double* decode_ms);

/* Teacher-forced decode (parity probes; no reference counterpart): like
 * rpg_hip_generate without stop ids, except that step i forwards
 * force_ids[i] instead of the id the sampler drew, which goes to
 * drawn_ids[i]. Every step then decides on the logits of the forced history,
 * so a caller holding another engine's ids and per-step logits can compare
 * every step. Returns max_tokens. */
RPG_HIP_API int32_t rpg_hip_generate_forced(int32_t session, const float* first_logits, int32_t max_tokens,
                                            float temperature, int32_t top_k, float top_p, uint64_t seed,
                                            const int32_t* force_ids, int32_t* drawn_ids, float* step_logits);

/* rpg_hip_generate_batch with teacher forcing: session i forwards
 * force_ids[i * max_tokens + t] at step t; drawn_ids[i * max_tokens + t]
 * receives the id drawn. No reference counterpart (parity probe). */
RPG_HIP_API int32_t rpg_hip_generate_batch_forced(const int32_t* sessions, int32_t n, int32_t max_tokens,
                                                  const float* temperature, const int32_t* top_k,
                                                  const float* top_p, const uint64_t* seed,
                                                  const int32_t* force_ids, int32_t* drawn_ids,
                                                  float* step_logits);

/* Failure injection for the out-of-memory contract (test hook; no reference
 * counterpart): after n more successful device allocations in this process,
 * the next one fails as a failed hipMalloc would, without calling it
 * (models, sessions, batches and the token-level buffers allocate this way);
 * n < 0 switches injection off. One failure per call. Returns 0. */
RPG_HIP_API int32_t rpg_hip_fail_alloc_after(int64_t n);

/* Which decode path the session runs: 0 = one launch per projection and
 * attention stage (the default), 1 = one persistent launch per token (only
 * when RPG_DECODE_STEP=1 was set at session creation and every projection is
 * Q4_K / Q6_K with a tile-major copy). No reference counterpart: a test
 * probe. */
RPG_HIP_API int32_t rpg_hip_session_decode_path(int32_t session);

/* Copy K (which = 0) or V (1) of (layer, kv_head, positions [0, n)), fp32. */
RPG_HIP_API int32_t rpg_hip_kv_read(int32_t session, int32_t which, int32_t layer, int32_t head, int64_t n,
                                    float* out);

/* Device milliseconds of the session's last prefill / generate call. */
RPG_HIP_API int32_t rpg_hip_session_timing(int32_t session, double* prefill_ms, double* decode_ms);

/* Roofline probe of the decode step's largest launch: `iters` back-to-back
 * gate+up (SwiGLU) matvecs on the session's stream, layers layer+1,
 * layer+2, ... (mod n_layers, so no launch re-reads cached weights), timed
 * with HIP events. out[0] = mean microseconds per launch, out[1] =
 * algorithmic bytes per launch (both weight matrices, input, norm gain,
 * output). No reference counterpart: measurement only. */
RPG_HIP_API int32_t rpg_hip_session_bench_gate_up(int32_t session, int32_t layer, int32_t iters, double* out);

/* The same launches where the decode step runs them: `tokens` greedy decode
 * steps from the session's state through the per-launch path, each layer's
 * gate+up launch bracketed by HIP events on the session stream (the interval
 * includes its dispatch after the previous kernel). out[0] = mean
 * microseconds per launch, out[1] = algorithmic bytes per launch. The session
 * must be prefilled and advances by `tokens`. Measurement only. */
RPG_HIP_API int32_t rpg_hip_session_instep_gate_up(int32_t session, int32_t tokens, double* out);

/* Device-to-device copy of `bytes` (a multiple of 16) by a plain grid-stride
 * kernel, `iters` times between two buffers: *us = mean microseconds per
 * copy. The measured stream bandwidth, and a kernel of known read and write
 * volume for calibrating byte counters. Measurement only. */
RPG_HIP_API int32_t rpg_hip_bench_copy(int64_t bytes, int32_t iters, double* us);

/* ---- kernels on host buffers (parity tests and microbenchmarks) */

/* DequantizeRow on the GPU, bit-exact (reference src/quant.cc:416-436). */
RPG_HIP_API int32_t rpg_hip_dequant(uint32_t type, const uint8_t* src, int64_t n, float* dst);

/* Y[t*rows + r] = X[t] . W[r] for t < n: the fused dequant matvec / blocked
 * matmul (reference src/matmul.h:35-64, QuantMatrix::MatMulBatch
 * src/model.cc:39-69). */
RPG_HIP_API int32_t rpg_hip_matmul(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols, const float* X,
                                   int64_t n, float* Y);

/* The few-token matvec the batched decode step runs (1 <= n <= 8 tokens,
 * Q4_K / Q6_K, cols % 256 == 0, cols <= 10240), on a tile-major copy it
 * makes: with norm_w (a [cols] gain) each row of X is RMS-normalised first
 * (reference src/qwen3.cc:131-134: double sum of squares, float scale,
 * (x * scale) * w); with `up` the output is silu(X[t] . W[r]) * (X[t] .
 * U[r]) (reference src/kernels.h:82-92); with add != 0, Y[t*rows + r] +=
 * X[t] . W[r] (the residual add, reference src/qwen3.cc:186-188), else
 * Y = X . W^T (reference src/matmul.h:35-64). Returns 0, or -1 on error. */
RPG_HIP_API int32_t rpg_hip_matvec_few(uint32_t type, const uint8_t* w, const uint8_t* up, int64_t rows, int64_t cols,
                                       const float* X, int64_t n, const float* norm_w, float eps, int32_t add,
                                       float* Y);

/* Y[t*rows + r] = silu(X[t] . G[r]) * (X[t] . U[r]) for t < n (n >= 2): the
 * prefill's gate/up projection with SwiGLU (reference src/kernels.h:82-92,
 * src/qwen3.cc:191-199). Returns 1 when the single fused GEMM launch ran, 0
 * when the two products and the SwiGLU pass ran, -1 on error. */
RPG_HIP_API int32_t rpg_hip_matmul_swiglu(uint32_t type, const uint8_t* gate, const uint8_t* up, int64_t rows,
                                          int64_t cols, const float* X, int64_t n, float* Y);

/* SampleToken (reference src/sampler.cc:96-112) with
 * u = CounterUniform(seed, counter) computed on the GPU; probs (optional,
 * [n]) receives FilterToProbs. Returns the token id. */
RPG_HIP_API int32_t rpg_hip_sample(const float* logits, int32_t n, float temperature, int32_t top_k, float top_p,
                                   uint64_t seed, int64_t counter, float* probs);

/* Number of sampler draws so far that took the sequential fallback. */
RPG_HIP_API int64_t rpg_hip_sampler_fallbacks(void);

/* Number of rpg_hip_sample draws so far whose top-p cut split a set of equal
 * probabilities, resolved by replaying the reference's std::sort order
 * (reference src/sampler.cc:72-82). Test probe. */
RPG_HIP_API int64_t rpg_hip_sampler_tie_orders(void);

/* rpg_hip_sample without any allocation. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops). Device buffers in and out: logits_dev [n]
 * fp32, token_dev [1], probs_dev [n] (optional, FilterToProbs); u =
 * CounterUniform(seed, counter). The work is enqueued on `stream` (a
 * hipStream_t; NULL = the null stream) and is complete when the stream is.
 * Scratch is a static device array of 8 MiB + 4 KiB per GPU (held until the
 * process ends): n must be at most 262144. Calls that overlap on one GPU
 * race on it. Returns 0 when enqueued, -1 on error. */
RPG_HIP_API int32_t rpg_hip_sample_noalloc(const float* logits_dev, int32_t n, float temperature, int32_t top_k,
                                           float top_p, uint64_t seed, int64_t counter, int32_t* token_dev,
                                           float* probs_dev, void* stream);

/* Causal GQA attention of a segment (the prefill kernel; reference
 * src/qwen3.cc:79-117): q [seq][n_heads][128] (QK-normed, rotated), the cache
 * contents k, v [n_kv][pos0 + seq][128], query t at position pos0 + t sees
 * positions 0 .. pos0 + t; out [seq][n_heads][128]. */
RPG_HIP_API int32_t rpg_hip_attention(const float* q, const float* k, const float* v, int32_t seq, int32_t n_heads,
                                      int32_t n_kv, int32_t pos0, float* out);

/* glibc-exact expf on the GPU over n inputs (parity probe). */
RPG_HIP_API int32_t rpg_hip_expf(const float* x, int64_t n, float* out);

/* Microbenchmark: for each token count ns[i], time `iters` launches of the
 * matmul y[n][rows] = x[n][cols] . W^T over `copies` device copies of W
 * (rotated so the weights stream from HBM; one upload, then device copies).
 * n = 1 takes the decode path (tile-major copies where the type has one).
 * out[i] = average milliseconds per launch at ns[i]. */
RPG_HIP_API int32_t rpg_hip_bench_matmul(uint32_t type, const uint8_t* w, int64_t rows, int64_t cols,
                                         const int32_t* ns, int32_t n_count, int32_t copies, int32_t iters,
                                         double* out);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* RPG_HIP_H */
