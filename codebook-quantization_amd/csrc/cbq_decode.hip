// Fused fp32 decoder glue for gfx950: residual add + RMSNorm, per-head
// RMSNorm + rotary embedding + KV-cache write, single-token grouped-query
// attention, and the SiLU-gated product.  HF Qwen3 semantics (the modelling
// code the reference's compressed modules plug into,
// src/model_loader.py:213-277); products and sums that PyTorch rounds one at
// a time are rounded one at a time here too (no contraction into FMAs),
// reductions run in a different order.
#include "cbq_device.h"
#include "../../include/cbq_decode.h"

#include <math.h>

namespace {

constexpr int kGlueBlock = 256;                     // 4 waves
constexpr int kAttnMaxLen = 32768;                  // scores live in LDS

// Sum over the block (all threads get the total); s_red holds one float per wave.
__device__ __forceinline__ float block_sum(float v, float *s_red)
{
    v = wave_sum(v);
    const int w = threadIdx.x / CBQ_WAVE;
    if ((threadIdx.x & (CBQ_WAVE - 1)) == 0) s_red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x / CBQ_WAVE); i++) t += s_red[i];
    __syncthreads();
    return t;
}

__device__ __forceinline__ float wave_max(float v)
{
    for (int o = CBQ_WAVE >> 1; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, CBQ_WAVE));
    return v;
}

__device__ __forceinline__ float block_max(float v, float *s_red)
{
    v = wave_max(v);
    const int w = threadIdx.x / CBQ_WAVE;
    if ((threadIdx.x & (CBQ_WAVE - 1)) == 0) s_red[w] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int i = 0; i < (int)(blockDim.x / CBQ_WAVE); i++) t = fmaxf(t, s_red[i]);
    __syncthreads();
    return t;
}

// One block per row.
__global__ __launch_bounds__(kGlueBlock) void add_rmsnorm_kernel(
    float *__restrict__ h, const float *__restrict__ delta, const float *__restrict__ weight,
    float *__restrict__ out, int H, float eps)
{
    __shared__ float s_red[kGlueBlock / CBQ_WAVE];
    float *hr = h + (size_t)blockIdx.x * H;
    float *orow = out + (size_t)blockIdx.x * H;
    float ss = 0.f;
    if (delta) {
        const float *dr = delta + (size_t)blockIdx.x * H;
        for (int i = threadIdx.x; i < H; i += kGlueBlock) {
            const float v = __fadd_rn(hr[i], dr[i]);
            hr[i] = v;
            ss = __fadd_rn(ss, __fmul_rn(v, v));
        }
    } else {
        for (int i = threadIdx.x; i < H; i += kGlueBlock) {
            const float v = hr[i];
            ss = __fadd_rn(ss, __fmul_rn(v, v));
        }
    }
    const float r = rsqrtf(block_sum(ss, s_red) / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += kGlueBlock) {
        float o = __fmul_rn(hr[i], r);
        if (weight) o = __fmul_rn(weight[i], o);
        orow[i] = o;
    }
}

// grid (n_q + n_kv, T), one wave per head.
__global__ __launch_bounds__(CBQ_WAVE) void head_norm_rope_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ qw, const float *__restrict__ kw, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, const int64_t *__restrict__ pos, float *__restrict__ q_out,
    float *__restrict__ kc, float *__restrict__ vc, int n_q, int n_kv, int hd, int max_len,
    float eps)
{
    __shared__ float s_x[256];
    const int hidx = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const bool is_q = hidx < n_q;
    const int kvh = hidx - n_q;
    const float *src = is_q ? q + ((size_t)t * n_q + hidx) * hd : k + ((size_t)t * n_kv + kvh) * hd;
    const float *w = is_q ? qw : kw;
    const int64_t p = pos[0] + t;
    const bool in_cache = p >= 0 && p < max_len;
    const int64_t row = in_cache ? p : 0;

    float ss = 0.f;
    for (int d = lane; d < hd; d += CBQ_WAVE) {
        const float x = src[d];
        s_x[d] = x;
        ss = __fadd_rn(ss, __fmul_rn(x, x));
    }
    const float r = rsqrtf(wave_sum(ss) / (float)hd + eps);
    __syncthreads();
    const int half = hd >> 1;
    for (int d = lane; d < hd; d += CBQ_WAVE) {
        const int dp = d < half ? d + half : d - half;
        float xn = __fmul_rn(s_x[d], r), xp = __fmul_rn(s_x[dp], r);
        if (w) { xn = __fmul_rn(w[d], xn); xp = __fmul_rn(w[dp], xp); }
        const float rot = d < half ? -xp : xp;
        const float o = __fadd_rn(__fmul_rn(xn, cos_t[row * hd + d]), __fmul_rn(rot, sin_t[row * hd + d]));
        if (is_q)
            q_out[((size_t)t * n_q + hidx) * hd + d] = o;
        else if (in_cache)
            kc[((size_t)kvh * max_len + p) * hd + d] = o;
    }
    if (!is_q && in_cache)
        for (int d = lane; d < hd; d += CBQ_WAVE)
            vc[((size_t)kvh * max_len + p) * hd + d] = v[((size_t)t * n_kv + kvh) * hd + d];
}

// One block per query head; scores and then probabilities in LDS.
template <int HD>
__global__ __launch_bounds__(kGlueBlock) void attn_decode_kernel(
    const float *__restrict__ q, const float *__restrict__ kc, const float *__restrict__ vc,
    const int64_t *__restrict__ pos, float *__restrict__ out, int group, int max_len, float scale)
{
    extern __shared__ float s_att[];                              // [max_len]
    __shared__ float s_q[HD];
    __shared__ float s_part[kGlueBlock];
    __shared__ float s_red[kGlueBlock / CBQ_WAVE];
    const int h = blockIdx.x, kvh = h / group, tid = threadIdx.x;
    const int64_t p = pos[0];
    const int L = (int)(p + 1 < 1 ? 1 : (p + 1 > max_len ? max_len : p + 1));
    for (int d = tid; d < HD; d += kGlueBlock) s_q[d] = q[(size_t)h * HD + d];
    __syncthreads();

    const float *K = kc + (size_t)kvh * max_len * HD;
    const float *V = vc + (size_t)kvh * max_len * HD;
    typedef float f4 __attribute__((ext_vector_type(4)));
    float mx = -INFINITY;
    for (int j = tid; j < L; j += kGlueBlock) {
        const f4 *kr = (const f4 *)(K + (size_t)j * HD);
        float acc = 0.f;
#pragma unroll 8
        for (int d4 = 0; d4 < HD / 4; d4++) {
            const f4 kv = kr[d4];
            acc = fmaf(s_q[4 * d4 + 0], kv.x, acc);
            acc = fmaf(s_q[4 * d4 + 1], kv.y, acc);
            acc = fmaf(s_q[4 * d4 + 2], kv.z, acc);
            acc = fmaf(s_q[4 * d4 + 3], kv.w, acc);
        }
        const float s = __fmul_rn(acc, scale);
        s_att[j] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_max(mx, s_red);
    float sum = 0.f;
    for (int j = tid; j < L; j += kGlueBlock) {
        const float e = expf(__fsub_rn(s_att[j], mx));
        s_att[j] = e;
        sum = __fadd_rn(sum, e);
    }
    sum = block_sum(sum, s_red);                                  // ends with a barrier
    for (int j = tid; j < L; j += kGlueBlock) s_att[j] = __fdiv_rn(s_att[j], sum);
    __syncthreads();

    constexpr int G = kGlueBlock / HD;                            // position groups
    const int g = tid / HD, d = tid % HD;
    float acc = 0.f;
    int j = g;
    for (; j + 3 * G < L; j += 4 * G) {
        const float v0 = V[(size_t)j * HD + d], v1 = V[(size_t)(j + G) * HD + d];
        const float v2 = V[(size_t)(j + 2 * G) * HD + d], v3 = V[(size_t)(j + 3 * G) * HD + d];
        acc = fmaf(s_att[j], v0, acc);
        acc = fmaf(s_att[j + G], v1, acc);
        acc = fmaf(s_att[j + 2 * G], v2, acc);
        acc = fmaf(s_att[j + 3 * G], v3, acc);
    }
    for (; j < L; j += G) acc = fmaf(s_att[j], V[(size_t)j * HD + d], acc);
    s_part[tid] = acc;
    __syncthreads();
    if (tid < HD) {
        float t = 0.f;
        for (int gg = 0; gg < G; gg++) t += s_part[gg * HD + tid];
        out[(size_t)h * HD + tid] = t;
    }
}

__global__ __launch_bounds__(kGlueBlock) void silu_mul_kernel(const float *__restrict__ g,
                                                             const float *__restrict__ u,
                                                             float *__restrict__ out, int64_t n)
{
    const int64_t stride = (int64_t)gridDim.x * kGlueBlock;
    for (int64_t i = (int64_t)blockIdx.x * kGlueBlock + threadIdx.x; i < n; i += stride) {
        const float x = g[i];
        out[i] = __fmul_rn(__fdiv_rn(x, __fadd_rn(1.0f, expf(-x))), u[i]);
    }
}

}  // namespace

extern "C" {

int cbq_add_rmsnorm_f32(float *h, const float *delta, const float *weight, float *out, int T,
                        int H, float eps, hipStream_t stream)
{
    if (!h || !out || out == h || T <= 0 || H <= 0 || T > 65535) return CK_ERR_ARG;
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(T), dim3(kGlueBlock), 0, stream, h, delta, weight,
                       out, H, eps);
    return cbq_launch_status("add_rmsnorm_kernel");
}

int cbq_head_norm_rope_f32(const float *q, const float *k, const float *v, const float *q_weight,
                           const float *k_weight, const float *cos_table, const float *sin_table,
                           const int64_t *pos, float *q_out, float *k_cache, float *v_cache, int T,
                           int n_q, int n_kv, int hd, int max_len, float eps, hipStream_t stream)
{
    if (!q || !k || !v || !cos_table || !sin_table || !pos || !q_out || !k_cache || !v_cache)
        return CK_ERR_ARG;
    if (T <= 0 || T > 65535 || n_q <= 0 || n_kv <= 0 || hd < 2 || hd > 256 || (hd & 1) ||
        max_len <= 0)
        return CK_ERR_ARG;
    hipLaunchKernelGGL(head_norm_rope_kernel, dim3(n_q + n_kv, T), dim3(CBQ_WAVE), 0, stream, q, k,
                       v, q_weight, k_weight, cos_table, sin_table, pos, q_out, k_cache, v_cache,
                       n_q, n_kv, hd, max_len, eps);
    return cbq_launch_status("head_norm_rope_kernel");
}

int cbq_attn_decode_f32(const float *q, const float *k_cache, const float *v_cache,
                        const int64_t *pos, float *out, int n_q, int n_kv, int hd, int max_len,
                        float scale, hipStream_t stream)
{
    if (!q || !k_cache || !v_cache || !pos || !out) return CK_ERR_ARG;
    if (n_q <= 0 || n_kv <= 0 || n_q % n_kv || max_len <= 0 || max_len > kAttnMaxLen)
        return CK_ERR_ARG;
    if (((uintptr_t)k_cache & 15) != 0) return CK_ERR_ARG;       // 16-byte key rows
    const size_t lds = (size_t)max_len * sizeof(float);
    const int group = n_q / n_kv;
    switch (hd) {
    case 64:
        hipLaunchKernelGGL(attn_decode_kernel<64>, dim3(n_q), dim3(kGlueBlock), lds, stream, q,
                           k_cache, v_cache, pos, out, group, max_len, scale);
        break;
    case 128:
        hipLaunchKernelGGL(attn_decode_kernel<128>, dim3(n_q), dim3(kGlueBlock), lds, stream, q,
                           k_cache, v_cache, pos, out, group, max_len, scale);
        break;
    case 256:
        hipLaunchKernelGGL(attn_decode_kernel<256>, dim3(n_q), dim3(kGlueBlock), lds, stream, q,
                           k_cache, v_cache, pos, out, group, max_len, scale);
        break;
    default:
        return CK_ERR_ARG;
    }
    return cbq_launch_status("attn_decode_kernel");
}

int cbq_silu_mul_f32(const float *g, const float *u, float *out, int64_t n, hipStream_t stream)
{
    if (!g || !u || !out || n <= 0) return CK_ERR_ARG;
    const int64_t want = (n + kGlueBlock - 1) / kGlueBlock;
    const int blocks = (int)(want < 4096 ? want : 4096);
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks), dim3(kGlueBlock), 0, stream, g, u, out, n);
    return cbq_launch_status("silu_mul_kernel");
}

}  // extern "C"
