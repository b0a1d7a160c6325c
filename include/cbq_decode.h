/*
 * cbq_decode.h -- fused fp32 decoder glue of the always-compressed greedy
 * decode (libcbq_hip.so, csrc/cbq_decode.hip).
 *
 * These entry points have no counterpart in the reference's C/HIP libraries:
 * there the glue between compressed linears is HF Qwen3 modelling in PyTorch
 * (src/model_loader.py:213-277 swaps the compressed modules into
 * Qwen3ForCausalLM).  They exist so that one decode step is a short sequence
 * of launches (a HIP graph of ~12 kernels per layer) instead of several
 * dozen small PyTorch kernels per layer.  Semantics are HF Qwen3's, in fp32:
 * RMSNorm x * rsqrt(mean(x^2) + eps) (* weight), per-head q/k RMSNorm, the
 * default rotary embedding x * cos + rotate_half(x) * sin, grouped-query
 * attention with an fp32 softmax, and silu(g) * u.
 *
 * Conventions as cbq_hip.h: device pointers, asynchronous on `stream`,
 * no allocation, return 0 / 1 (HIP error) / 2 (invalid argument).
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* For each of the T rows of h [T, H]: h += delta (when delta is not NULL),
 * then out = h * rsqrt(mean(h^2) + eps) (* weight[H] when not NULL).
 * out may not alias h.  H <= 16384. */
int cbq_add_rmsnorm_f32(float *h, const float *delta, const float *weight, float *out,
                        int T, int H, float eps, hipStream_t stream);

/* Per token t < T at position pos[0] + t (pos: one device int64):
 *   q_out[t, i]  = rope(rmsnorm(q[t, i]) * q_weight)          i < n_q
 *   k_cache[j, pos + t] = rope(rmsnorm(k[t, j]) * k_weight)    j < n_kv
 *   v_cache[j, pos + t] = v[t, j]
 * q [T, n_q, hd], k and v [T, n_kv, hd]; caches [n_kv, max_len, hd];
 * cos/sin tables [max_len, hd].  Weights may be NULL (ones).  Tokens whose
 * position falls outside [0, max_len) are not written to the caches and
 * use table row 0.  hd even, 2 <= hd <= 256. */
int cbq_head_norm_rope_f32(const float *q, const float *k, const float *v,
                           const float *q_weight, const float *k_weight,
                           const float *cos_table, const float *sin_table,
                           const int64_t *pos, float *q_out, float *k_cache,
                           float *v_cache, int T, int n_q, int n_kv, int hd,
                           int max_len, float eps, hipStream_t stream);

/* Single-token causal attention over cache positions [0, pos[0]] (clamped
 * to [1, max_len] positions): query head i reads kv head i / (n_q / n_kv).
 * out[i] = softmax(q[i] . k[j] * scale) . v[j]; q and out [n_q, hd].
 * hd in {64, 128, 256}; n_q % n_kv == 0; max_len <= 32768. */
int cbq_attn_decode_f32(const float *q, const float *k_cache, const float *v_cache,
                        const int64_t *pos, float *out, int n_q, int n_kv, int hd,
                        int max_len, float scale, hipStream_t stream);

/* One decode token (T = 1) at position p = pos[0]: the q/k head norm and
 * rope of cbq_head_norm_rope_f32 and the attention of cbq_attn_decode_f32 in
 * one launch.  The new key/value row is stored at cache row p (when
 * p < max_len) and attended from on-chip memory; cached rows [0, p) come
 * from k_cache/v_cache.  q [n_q, hd], k and v [n_kv, hd], out [n_q, hd]. */
int cbq_attn_rope_decode_f32(const float *q, const float *k, const float *v,
                             const float *q_weight, const float *k_weight,
                             const float *cos_table, const float *sin_table,
                             const int64_t *pos, float *k_cache, float *v_cache,
                             float *out, int n_q, int n_kv, int hd, int max_len,
                             float scale, float eps, hipStream_t stream);

/* cbq_attn_rope_decode_f32 with the cached rows split over several blocks per
 * query head (flash decoding), then a second launch that merges the splits;
 * same arguments, results equal to rounding (the softmax is accumulated per
 * split and merged in split order).  workspace: device scratch of at least
 * cbq_attn_rope_decode_workspace(n_q, hd, max_len) bytes, 4-byte aligned,
 * overwritten by every call (no initial contents needed); calls that share a
 * workspace must not overlap.  hd in {64, 128, 256}.  No counterpart in the
 * reference (HF computes the attention there): decoder glue of this build. */
size_t cbq_attn_rope_decode_workspace(int n_q, int hd, int max_len);
int cbq_attn_rope_decode_ws_f32(const float *q, const float *k, const float *v,
                                const float *q_weight, const float *k_weight,
                                const float *cos_table, const float *sin_table,
                                const int64_t *pos, float *k_cache, float *v_cache,
                                float *out, int n_q, int n_kv, int hd, int max_len,
                                float scale, float eps, void *workspace,
                                size_t workspace_bytes, hipStream_t stream);

/* cbq_attn_rope_decode_ws_f32 for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  It has no counterpart in the reference.  Same
 * arguments as cbq_attn_rope_decode_f32, results bit-identical to
 * cbq_attn_rope_decode_ws_f32.  The split partials live in a static device
 * array of CBQ_ATTN_SCRATCH_BYTES (1 MiB) that the library holds on every
 * GPU it runs on until the process ends; shapes whose partials,
 * cbq_attn_rope_decode_workspace(n_q, hd, max_len) bytes, exceed it return
 * CK_ERR_ARG with a message (e.g. n_q * (hd + 2) > 16384 once max_len >
 * 960).  The first call on a device resolves the array's address
 * (hipGetSymbolAddress): make it outside stream capture.  Every call on a
 * GPU uses that GPU's one array, so calls that overlap on one GPU (other
 * streams, other host threads) race; the partials are fully rewritten by
 * each call, nothing needs clearing.  Allocates nothing. */
#define CBQ_ATTN_SCRATCH_BYTES (1u << 20)
int cbq_attn_rope_decode_noalloc_f32(const float *q, const float *k, const float *v,
                                     const float *q_weight, const float *k_weight,
                                     const float *cos_table, const float *sin_table,
                                     const int64_t *pos, float *k_cache, float *v_cache,
                                     float *out, int n_q, int n_kv, int hd, int max_len,
                                     float scale, float eps, hipStream_t stream);

/* Greedy pick of a captured decode step: tok = argmax(logits[0, n)) (first
 * maximum; NaN ranks highest, as torch.argmax); ids32[0] = tok;
 * toks[pos[0] - first] = tok when that index lies in [0, n_toks);
 * pos[0] += 1.  Two launches, no host round trip; workspace is device
 * scratch of >= 1024 bytes (partial maxima), overwritten by every call. */
int cbq_argmax_step(const float *logits, int n, void *workspace, int32_t *ids32,
                    int64_t *toks, int64_t *pos, int64_t first, int64_t n_toks,
                    hipStream_t stream);

/* out[i] = silu(g[i]) * u[i] = g / (1 + exp(-g)) * u, i < n. */
int cbq_silu_mul_f32(const float *g, const float *u, float *out, int64_t n,
                     hipStream_t stream);

#ifdef __cplusplus
}
#endif
