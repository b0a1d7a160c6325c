// Fused fp32 decoder glue for gfx950: residual add + RMSNorm, per-head
// RMSNorm + rotary embedding + KV-cache write, single-token grouped-query
// attention (alone or with the head norm, rope and cache write folded in),
// the SiLU-gated product and the greedy pick.  HF Qwen3 semantics (the modelling
// code the reference's compressed modules plug into,
// src/model_loader.py:213-277); products and sums that PyTorch rounds one at
// a time are rounded one at a time here too (no contraction into FMAs),
// reductions run in a different order.
#include "cbq_device.h"
#include "../../include/cbq_decode.h"

#include <math.h>
#include <stdio.h>

#include <mutex>

// hipcc contracts a * b + c into an fma by default; the glue rounds each
// product and sum on its own (explicit fmaf calls stay fused).
#pragma clang fp contract(off)

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

// One block per row, the row held in registers (H <= kNormThreads * kNormPer):
// every load is issued before the reduction, so a row costs one memory
// round trip rather than one per loop iteration.
constexpr int kNormThreads = 1024;
constexpr int kNormPer = 16;

__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(
    float *__restrict__ h, const float *__restrict__ delta, const float *__restrict__ weight,
    float *__restrict__ out, int H, float eps)
{
    __shared__ float s_red[kNormThreads / CBQ_WAVE];
    float *hr = h + (size_t)blockIdx.x * H;
    float *orow = out + (size_t)blockIdx.x * H;
    const float *dr = delta ? delta + (size_t)blockIdx.x * H : nullptr;
    float v[kNormPer];
#pragma unroll
    for (int j = 0; j < kNormPer; j++) {
        const int i = threadIdx.x + j * kNormThreads;
        v[j] = i < H ? hr[i] : 0.f;
    }
    if (dr) {
#pragma unroll
        for (int j = 0; j < kNormPer; j++) {
            const int i = threadIdx.x + j * kNormThreads;
            if (i < H) {
                v[j] = __fadd_rn(v[j], dr[i]);
                hr[i] = v[j];
            }
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kNormPer; j++) ss = add_square(ss, v[j]);
    const float r = rsqrtf(block_sum(ss, s_red) / (float)H + eps);
#pragma unroll
    for (int j = 0; j < kNormPer; j++) {
        const int i = threadIdx.x + j * kNormThreads;
        if (i < H) orow[i] = weight ? __fmul_rn(weight[i], __fmul_rn(v[j], r)) : __fmul_rn(v[j], r);
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
    extern __shared__ __attribute__((aligned(16))) float s_att[];                              // [max_len]
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

// Single-token attention with the q/k head norm + rope and the KV-cache write
// folded in.  One block per query head: waves 0 and 1 normalise and rotate
// the query head and its group's new key, wave 2 stages the new value; the
// group's first block stores key and value at row pos.  Cached rows [0, pos)
// come from memory, the new row from LDS, so no block waits on another.
constexpr int kAttnThreads = 512;

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_rope_decode_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ qw, const float *__restrict__ kw, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, const int64_t *__restrict__ pos, float *__restrict__ kc,
    float *__restrict__ vc, float *__restrict__ out, int group, int max_len, float scale,
    float eps)
{
    extern __shared__ __attribute__((aligned(16))) float s_att[];                              // [max_len + 1]
    __shared__ float s_raw[2][HD];
    __shared__ __attribute__((aligned(16))) float s_q[HD];       // read as float4
    __shared__ __attribute__((aligned(16))) float s_k[HD];
    __shared__ float s_v[HD], s_cs[2][HD];
    __shared__ __attribute__((aligned(16))) float s_part[4 * kAttnThreads];
    __shared__ float s_red[kAttnThreads / CBQ_WAVE];
    const int h = blockIdx.x, g = h / group, tid = threadIdx.x;
    const int wave = tid / CBQ_WAVE, lane = tid & (CBQ_WAVE - 1);
    const int64_t p = pos[0];
    const bool store = p >= 0 && p < max_len;
    const int64_t trow = store ? p : 0;                           // cos/sin row
    const int n_old = (int)(p < 0 ? 0 : (p > max_len ? max_len : p));

    float r = 0.f;
    if (wave < 2) {
        const float *src = wave == 0 ? q + (size_t)h * HD : k + (size_t)g * HD;
        float ss = 0.f;
        for (int d = lane; d < HD; d += CBQ_WAVE) {
            const float x = src[d];
            s_raw[wave][d] = x;
            ss = __fadd_rn(ss, __fmul_rn(x, x));
        }
        r = rsqrtf(wave_sum(ss) / (float)HD + eps);
    } else if (wave == 2) {
        for (int d = lane; d < HD; d += CBQ_WAVE) s_v[d] = v[(size_t)g * HD + d];
    } else if (wave < 5) {
        const float *src = (wave == 3 ? cos_t : sin_t) + trow * HD;
        for (int d = lane; d < HD; d += CBQ_WAVE) s_cs[wave - 3][d] = src[d];
    }
    // Warm L2 with the cached K and V rows [0, min(n_old, 512)) (one dword
    // per 128-byte line) while the head vectors are normalised; the values
    // are only kept until the end of the kernel.
    constexpr int kLines = 8 * HD / 256;                          // lines of one K + one V row, / 4
    uint32_t warm[2 * kLines];
    {
        const int rows = n_old < kAttnThreads ? n_old : kAttnThreads;
        const uint32_t *kb = (const uint32_t *)(kc + (size_t)g * max_len * HD);
        const uint32_t *vb = (const uint32_t *)(vc + (size_t)g * max_len * HD);
#pragma unroll
        for (int i = 0; i < kLines; i++) {
            const int line = i * kAttnThreads + tid;             // line of the [rows, HD] block
            const bool in = line < rows * (HD / 32);
            warm[2 * i] = in ? kb[line * 32] : 0u;
            warm[2 * i + 1] = in ? vb[line * 32] : 0u;
        }
    }
    __syncthreads();
    if (wave < 2) {
        const float *w = wave == 0 ? qw : kw;
        float *dst = wave == 0 ? s_q : s_k;
        constexpr int half = HD / 2;
        for (int d = lane; d < HD; d += CBQ_WAVE) {
            const int dp = d < half ? d + half : d - half;
            float xn = __fmul_rn(s_raw[wave][d], r), xp = __fmul_rn(s_raw[wave][dp], r);
            if (w) { xn = __fmul_rn(w[d], xn); xp = __fmul_rn(w[dp], xp); }
            const float rot = d < half ? -xp : xp;
            dst[d] = __fadd_rn(__fmul_rn(xn, s_cs[0][d]), __fmul_rn(rot, s_cs[1][d]));
        }
    }
    __syncthreads();
    if (store && h % group == 0)
        for (int d = tid; d < HD; d += kAttnThreads) {
            kc[((size_t)g * max_len + p) * HD + d] = s_k[d];
            vc[((size_t)g * max_len + p) * HD + d] = s_v[d];
        }

    const float *K = kc + (size_t)g * max_len * HD;
    const float *V = vc + (size_t)g * max_len * HD;
    typedef float f4 __attribute__((ext_vector_type(4)));
    float mx = -INFINITY;
    // q . k_j: 8 lanes per row, lane s of a row taking float4 s, s + 8, ...,
    // so the 8 lanes of a row read 128 contiguous bytes per load (a lane per
    // row reads one line per lane and is bound by the address path); the 8
    // partial sums add by shuffles.  Row n_old is the new key, from LDS.
    static_assert(HD % 32 == 0, "whole float4 per lane of a row");
    constexpr int NQ = HD / 32;                                   // float4 per lane
    const int sub = lane & 7;
    f4 qv[NQ];
#pragma unroll
    for (int m = 0; m < NQ; m++) qv[m] = ((const f4 *)s_q)[sub + 8 * m];
    for (int j0 = 0; j0 <= n_old; j0 += kAttnThreads / 8) {
        const int j = j0 + tid / 8;
        float acc = 0.f;
        if (j <= n_old) {
            const f4 *kr = j < n_old ? (const f4 *)(K + (size_t)j * HD) : (const f4 *)s_k;
#pragma unroll
            for (int m = 0; m < NQ; m++) {
                const f4 kv = kr[sub + 8 * m];
                acc = fmaf(qv[m].x, kv.x, acc);
                acc = fmaf(qv[m].y, kv.y, acc);
                acc = fmaf(qv[m].z, kv.z, acc);
                acc = fmaf(qv[m].w, kv.w, acc);
            }
        }
        acc = group_sum(acc, 8);
        if (j <= n_old) {
            const float sc = __fmul_rn(acc, scale);
            if (sub == 0) s_att[j] = sc;
            mx = fmaxf(mx, sc);
        }
    }
    mx = block_max(mx, s_red);
    float sum = 0.f;
    for (int j = tid; j <= n_old; j += kAttnThreads) {
        const float e = expf(__fsub_rn(s_att[j], mx));
        s_att[j] = e;
        sum = __fadd_rn(sum, e);
    }
    sum = block_sum(sum, s_red);                                  // ends with a barrier
    for (int j = tid; j <= n_old; j += kAttnThreads) s_att[j] = __fdiv_rn(s_att[j], sum);
    __syncthreads();

    // out = sum_j p_j v_j: thread (gg, d4) owns dims [4 d4, 4 d4 + 4) of rows gg, gg + G, ...
    constexpr int Q = HD / 4, G = kAttnThreads / Q;
    const int gg = tid / Q, d4 = tid % Q;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    int j = gg;
    for (; j + 3 * G < n_old; j += 4 * G) {
        const f4 v0 = ((const f4 *)(V + (size_t)j * HD))[d4];
        const f4 v1 = ((const f4 *)(V + (size_t)(j + G) * HD))[d4];
        const f4 v2 = ((const f4 *)(V + (size_t)(j + 2 * G) * HD))[d4];
        const f4 v3 = ((const f4 *)(V + (size_t)(j + 3 * G) * HD))[d4];
        acc = __builtin_elementwise_fma((f4)s_att[j], v0, acc);
        acc = __builtin_elementwise_fma((f4)s_att[j + G], v1, acc);
        acc = __builtin_elementwise_fma((f4)s_att[j + 2 * G], v2, acc);
        acc = __builtin_elementwise_fma((f4)s_att[j + 3 * G], v3, acc);
    }
    for (; j < n_old; j += G)
        acc = __builtin_elementwise_fma((f4)s_att[j], ((const f4 *)(V + (size_t)j * HD))[d4], acc);
    ((f4 *)s_part)[tid] = acc;
    __syncthreads();
    if (tid < HD) {
        float t = 0.f;
        for (int i = 0; i < G; i++) t += s_part[i * HD + tid];
        out[(size_t)h * HD + tid] = fmaf(s_att[n_old], s_v[tid], t);
    }
    uint32_t sink = 0;
#pragma unroll
    for (int i = 0; i < 2 * kLines; i++) sink ^= warm[i];
    asm volatile("" ::"v"(sink));                                 // keeps the warming loads
}

// The same one-token step with the cached rows split over S blocks per query
// head (grid n_q x S, flash decoding): a lone block per head is held to one
// CU's load bandwidth, S blocks per head spread the key/value reads over the
// chip.  Block (h, s) takes rows [s R, (s + 1) R) of the n_old + 1 rows
// (R = ceil((n_old + 1) / S)) in chunks of CH rows: scores, a running max and
// sum of exponentials, and the exp-weighted sum of value rows.  It writes the
// partial (max, sum, vector) to the workspace; attn_combine_kernel, the next
// launch, merges the S partials of each head in order s = 0 .. S-1.  The
// first chunk's key and value rows are requested before the head norm, so
// their latency overlaps it.
constexpr int kSplitThreads = 256;
constexpr int kSplitChunk = 64;
constexpr int kMaxSplits = 16;

__host__ __device__ constexpr int attn_split_count(int max_len)
{
    return max_len <= kSplitChunk ? 1
         : ((max_len + kSplitChunk - 1) / kSplitChunk > kMaxSplits
                ? kMaxSplits : (max_len + kSplitChunk - 1) / kSplitChunk);
}

template <int HD>
__global__ __launch_bounds__(kSplitThreads) void attn_rope_split_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v,
    const float *__restrict__ qw, const float *__restrict__ kw, const float *__restrict__ cos_t,
    const float *__restrict__ sin_t, const int64_t *__restrict__ pos, float *__restrict__ kc,
    float *__restrict__ vc, float *__restrict__ part, int group, int max_len, float scale,
    float eps)
{
    typedef float f4 __attribute__((ext_vector_type(4)));
    constexpr int LPR = HD / 32;                       // lanes per key row, 32 dims each
    constexpr int RPP = kSplitThreads / LPR;           // key rows per score pass
    constexpr int CH = RPP < kSplitChunk ? RPP : kSplitChunk;
    constexpr int Q4 = HD / 4;                         // float4 columns of a row
    constexpr int NG = kSplitThreads / Q4;             // row groups of the value pass
    constexpr int VPT = CH / NG;                       // value rows per thread per chunk
    static_assert(CH <= CBQ_WAVE && CH % NG == 0, "chunk layout");

    __shared__ float s_raw[2][HD];
    __shared__ __attribute__((aligned(16))) float s_q[HD];
    __shared__ float s_k[HD], s_cs[2][HD];
    __shared__ __attribute__((aligned(16))) float s_v[HD];
    __shared__ float s_sc[CH], s_p[CH];
    __shared__ __attribute__((aligned(16))) float s_part[NG * HD];
    __shared__ float s_ml[3];                          // running max, sum, chunk rescale

    const int h = blockIdx.x, sp = blockIdx.y, S = gridDim.y, g = h / group;
    const int tid = threadIdx.x, wave = tid / CBQ_WAVE, lane = tid & (CBQ_WAVE - 1);
    const int64_t p = pos[0];
    const bool store = p >= 0 && p < max_len;
    const int64_t trow = store ? p : 0;
    const int n_old = (int)(p < 0 ? 0 : (p > max_len ? max_len : p));
    const int n_all = n_old + 1;
    const int R = (n_all + S - 1) / S;
    const int j0 = sp * R < n_all ? sp * R : n_all;
    const int j1 = j0 + R < n_all ? j0 + R : n_all;

    const float *K = kc + (size_t)g * max_len * HD;
    const float *V = vc + (size_t)g * max_len * HD;
    const int srow = tid / LPR, spart = tid % LPR;     // score pass: row, 32-dim part
    const int d4 = tid % Q4, rg = tid / Q4;            // value pass: column, row group
    f4 kreg[8], vreg[VPT];
    auto load_chunk = [&](int c0) {
        const int j = c0 + srow;
        if (srow < CH && j < j1 && j < n_old) {
            const f4 *kr = (const f4 *)(K + (size_t)j * HD + spart * 32);
#pragma unroll
            for (int i = 0; i < 8; i++) kreg[i] = kr[i];
        }
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const int jv = c0 + rg + i * NG;
            if (jv < j1 && jv < n_old) vreg[i] = ((const f4 *)(V + (size_t)jv * HD))[d4];
        }
    };
    if (j0 < j1) load_chunk(j0);

    // head norm + rope of the query head and the group's new key (as
    // attn_rope_decode_kernel), the new value row
    float r = 0.f;
    if (wave < 2) {
        const float *src = wave == 0 ? q + (size_t)h * HD : k + (size_t)g * HD;
        float ss = 0.f;
        for (int d = lane; d < HD; d += CBQ_WAVE) {
            const float x = src[d];
            s_raw[wave][d] = x;
            ss = __fadd_rn(ss, __fmul_rn(x, x));
        }
        r = rsqrtf(wave_sum(ss) / (float)HD + eps);
    } else if (wave == 2) {
        for (int d = lane; d < HD; d += CBQ_WAVE) s_v[d] = v[(size_t)g * HD + d];
    } else {
        for (int d = lane; d < HD; d += CBQ_WAVE) {
            s_cs[0][d] = cos_t[trow * HD + d];
            s_cs[1][d] = sin_t[trow * HD + d];
        }
    }
    __syncthreads();
    if (wave < 2) {
        const float *w = wave == 0 ? qw : kw;
        float *dst = wave == 0 ? s_q : s_k;
        constexpr int half = HD / 2;
        for (int d = lane; d < HD; d += CBQ_WAVE) {
            const int dp = d < half ? d + half : d - half;
            float xn = __fmul_rn(s_raw[wave][d], r), xp = __fmul_rn(s_raw[wave][dp], r);
            if (w) { xn = __fmul_rn(w[d], xn); xp = __fmul_rn(w[dp], xp); }
            const float rot = d < half ? -xp : xp;
            dst[d] = __fadd_rn(__fmul_rn(xn, s_cs[0][d]), __fmul_rn(rot, s_cs[1][d]));
        }
    }
    __syncthreads();
    if (store && sp == 0 && h % group == 0)
        for (int d = tid; d < HD; d += kSplitThreads) {
            kc[((size_t)g * max_len + p) * HD + d] = s_k[d];
            vc[((size_t)g * max_len + p) * HD + d] = s_v[d];
        }

    float m_run = -INFINITY, l_run = 0.f;              // wave 0's copies are the live ones
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = j0; c0 < j1; c0 += CH) {
        if (c0 != j0) load_chunk(c0);
        const int n = j1 - c0 < CH ? j1 - c0 : CH;
        if (srow < n) {
            const int j = c0 + srow;
            const float *qp = s_q + spart * 32;
            float dot = 0.f;
            if (j < n_old) {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    dot = fmaf(qp[4 * i + 0], kreg[i].x, dot);
                    dot = fmaf(qp[4 * i + 1], kreg[i].y, dot);
                    dot = fmaf(qp[4 * i + 2], kreg[i].z, dot);
                    dot = fmaf(qp[4 * i + 3], kreg[i].w, dot);
                }
            } else {
                for (int d = 0; d < 32; d++) dot = fmaf(qp[d], s_k[spart * 32 + d], dot);
            }
#pragma unroll
            for (int o = LPR >> 1; o > 0; o >>= 1) dot = __fadd_rn(dot, __shfl_xor(dot, o, CBQ_WAVE));
            if (spart == 0) s_sc[srow] = __fmul_rn(dot, scale);
        }
        __syncthreads();
        if (wave == 0) {
            const float sc = lane < n ? s_sc[lane] : -INFINITY;
            const float mn = fmaxf(m_run, wave_max(sc));
            const float alpha = expf(__fsub_rn(m_run, mn));
            const float pj = lane < n ? expf(__fsub_rn(sc, mn)) : 0.f;
            if (lane < CH) s_p[lane] = pj;
            l_run = __fadd_rn(__fmul_rn(l_run, alpha), wave_sum(pj));
            m_run = mn;
            if (lane == 0) s_ml[2] = alpha;
        }
        __syncthreads();
        const float alpha = s_ml[2];
        acc.x = __fmul_rn(acc.x, alpha);
        acc.y = __fmul_rn(acc.y, alpha);
        acc.z = __fmul_rn(acc.z, alpha);
        acc.w = __fmul_rn(acc.w, alpha);
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const int rr = rg + i * NG;
            if (rr < n) {
                const f4 vv = c0 + rr < n_old ? vreg[i] : ((const f4 *)s_v)[d4];
                acc = __builtin_elementwise_fma((f4)s_p[rr], vv, acc);
            }
        }
    }
    ((f4 *)s_part)[tid] = acc;
    if (tid == 0) {
        s_ml[0] = m_run;
        s_ml[1] = l_run;
    }
    __syncthreads();

    // this block's partial: [max, sum, vector[HD]]
    float *rec = part + ((size_t)h * S + sp) * (HD + 2);
    for (int d = tid; d < HD; d += kSplitThreads) {
        float t = 0.f;
        for (int i = 0; i < NG; i++) t = __fadd_rn(t, s_part[i * HD + d]);
        rec[2 + d] = t;
    }
    if (tid == 0) {
        rec[0] = s_ml[0];
        rec[1] = s_ml[1];
    }
}

// out[h] = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s over the S partials
// of head h, in order s = 0 .. S-1 (M = max_s m_s; an empty split has
// m = -inf, l = 0, acc = 0 and adds nothing).  One block per head, one
// thread per dimension.
template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(const float *__restrict__ part, int S,
                                                          float *__restrict__ out)
{
    const int h = blockIdx.x, d = threadIdx.x;
    const float *base = part + (size_t)h * S * (HD + 2);
    float M = -INFINITY;
    for (int t = 0; t < S; t++) M = fmaxf(M, base[(size_t)t * (HD + 2)]);
    float L = 0.f, o = 0.f;
    for (int t = 0; t < S; t++) {
        const float *rt = base + (size_t)t * (HD + 2);
        const float e = expf(__fsub_rn(rt[0], M));
        L = __fadd_rn(L, __fmul_rn(rt[1], e));
        o = __fadd_rn(o, __fmul_rn(rt[2 + d], e));
    }
    out[(size_t)h * HD + d] = __fdiv_rn(o, L);
}

// Greedy pick of a decode step in two launches: kArgBlocks blocks reduce
// slices of the logits to (value, index) partials in the caller's workspace,
// one block reduces those and does the step bookkeeping.  Order: first
// maximum; NaN ranks highest (first NaN wins), as torch.argmax.
constexpr int kArgThreads = 512;
constexpr int kArgBlocks = 128;

__device__ __forceinline__ void arg_block_reduce(float &best, int &bi, float *s_v, int *s_i)
{
    for (int o = CBQ_WAVE >> 1; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, CBQ_WAVE);
        const int oi = __shfl_xor(bi, o, CBQ_WAVE);
        if (arg_better(ov, oi, best, bi)) { best = ov; bi = oi; }
    }
    if ((threadIdx.x & (CBQ_WAVE - 1)) == 0) {
        s_v[threadIdx.x / CBQ_WAVE] = best;
        s_i[threadIdx.x / CBQ_WAVE] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < (int)(blockDim.x / CBQ_WAVE); w++)
            if (arg_better(s_v[w], s_i[w], best, bi)) { best = s_v[w]; bi = s_i[w]; }
}

__global__ __launch_bounds__(kArgThreads) void argmax_partial_kernel(
    const float *__restrict__ x, int n, float *__restrict__ part_v, int *__restrict__ part_i)
{
    __shared__ float s_v[kArgThreads / CBQ_WAVE];
    __shared__ int s_i[kArgThreads / CBQ_WAVE];
    float best = -INFINITY;
    int bi = n;                                    // "none": loses to any real index
    for (int i = blockIdx.x * kArgThreads + threadIdx.x; i < n; i += kArgBlocks * kArgThreads) {
        const float xv = x[i];
        if (arg_better(xv, i, best, bi)) { best = xv; bi = i; }
    }
    arg_block_reduce(best, bi, s_v, s_i);
    if (threadIdx.x == 0) { part_v[blockIdx.x] = best; part_i[blockIdx.x] = bi; }
}

__global__ __launch_bounds__(kArgBlocks) void argmax_final_kernel(
    const float *__restrict__ part_v, const int *__restrict__ part_i, int n,
    int32_t *__restrict__ ids32, int64_t *__restrict__ toks, int64_t *__restrict__ pos,
    int64_t first, int64_t n_toks)
{
    __shared__ float s_v[kArgBlocks / CBQ_WAVE];
    __shared__ int s_i[kArgBlocks / CBQ_WAVE];
    float best = part_v[threadIdx.x];
    int bi = part_i[threadIdx.x];
    arg_block_reduce(best, bi, s_v, s_i);
    if (threadIdx.x == 0) {
        const int tok = bi < n ? bi : 0;
        ids32[0] = tok;
        const int64_t p = pos[0];
        const int64_t kk = p - first;
        if (kk >= 0 && kk < n_toks) toks[kk] = tok;
        pos[0] = p + 1;
    }
}

// Merge of the (value, index) pairs a fused GEMV + pick wrote (one per
// block), then the step bookkeeping of argmax_final_kernel.
constexpr int kMergeThreads = 1024;

__global__ __launch_bounds__(kMergeThreads) void argmax_merge_kernel(
    const float *__restrict__ part_v, const int *__restrict__ part_i, int n_part, int n,
    int32_t *__restrict__ ids32, int64_t *__restrict__ toks, int64_t *__restrict__ pos,
    int64_t first, int64_t n_toks)
{
    __shared__ float s_v[kMergeThreads / CBQ_WAVE];
    __shared__ int s_i[kMergeThreads / CBQ_WAVE];
    float best = -INFINITY;
    int bi = kArgNone;
    for (int i = threadIdx.x; i < n_part; i += kMergeThreads)
        if (arg_better(part_v[i], part_i[i], best, bi)) { best = part_v[i]; bi = part_i[i]; }
    arg_block_reduce(best, bi, s_v, s_i);
    if (threadIdx.x == 0) {
        const int tok = bi < n ? bi : 0;
        ids32[0] = tok;
        const int64_t p = pos[0];
        const int64_t kk = p - first;
        if (kk >= 0 && kk < n_toks) toks[kk] = tok;
        pos[0] = p + 1;
    }
}

__global__ __launch_bounds__(kGlueBlock) void silu_mul_kernel(const float *__restrict__ g,
                                                             const float *__restrict__ u,
                                                             float *__restrict__ out, int64_t n)
{
    const int64_t stride = (int64_t)gridDim.x * kGlueBlock;
    for (int64_t i = (int64_t)blockIdx.x * kGlueBlock + threadIdx.x; i < n; i += stride) {
        const float x = g[i];
        out[i] = silu_mul_value(x, u[i]);
    }
}

}  // namespace

int cbq_argmax_merge(const float *part_v, const int *part_i, int n_part, int n, int32_t *ids32,
                     int64_t *toks, int64_t *pos, int64_t first, int64_t n_toks,
                     hipStream_t stream)
{
    hipLaunchKernelGGL(argmax_merge_kernel, dim3(1), dim3(kMergeThreads), 0, stream, part_v,
                       part_i, n_part, n, ids32, toks, pos, first, n_toks);
    return cbq_launch_status("argmax_merge_kernel");
}

// Static split-partials scratch of cbq_attn_rope_decode_noalloc_f32, one
// copy per device, held for the life of the process.  Host code never passes
// the array's name to a kernel (in host code it names a host-side stand-in):
// scratch_address() resolves the device's own copy once per device with
// hipGetSymbolAddress and every launch uses that pointer.
constexpr size_t kAttnScratchBytes = CBQ_ATTN_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kAttnScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_ptr[kMaxDevices];

// The current device's copy of `scratch`.
int scratch_address(float **out)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        fprintf(stderr, "[cbq_hip] scratch: no usable current device (%d)\n", dev);
        return CK_ERR_HIP;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            fprintf(stderr, "[cbq_hip] scratch: hipGetSymbolAddress failed on device %d: %s\n",
                    dev, hipGetErrorString(e));
            return CK_ERR_HIP;
        }
        g_scratch_ptr[dev] = (float *)p;
    }
    *out = g_scratch_ptr[dev];
    return CK_SUCCESS;
}

// Argument checks shared by the split one-token attention entry points.
int attn_split_check(const float *q, const float *k, const float *v, const float *cos_table,
                     const float *sin_table, const int64_t *pos, const float *k_cache,
                     const float *v_cache, const float *out, int n_q, int n_kv, int hd,
                     int max_len)
{
    if (!q || !k || !v || !cos_table || !sin_table || !pos || !k_cache || !v_cache || !out)
        return CK_ERR_ARG;
    if (n_q <= 0 || n_kv <= 0 || n_q % n_kv || max_len <= 0 || max_len > kAttnMaxLen)
        return CK_ERR_ARG;
    if (((uintptr_t)k_cache & 15) != 0 || ((uintptr_t)v_cache & 15) != 0) return CK_ERR_ARG;
    if (hd != 64 && hd != 128 && hd != 256) return CK_ERR_ARG;
    return CK_SUCCESS;
}

// Split launch + merge launch with the partials at `part`
// (attn_split_count(max_len) * n_q * (hd + 2) floats).
int attn_split_launch(const float *q, const float *k, const float *v, const float *q_weight,
                      const float *k_weight, const float *cos_table, const float *sin_table,
                      const int64_t *pos, float *k_cache, float *v_cache, float *out, int n_q,
                      int n_kv, int hd, int max_len, float scale, float eps, float *part,
                      hipStream_t stream)
{
    const int S = attn_split_count(max_len);
    const int group = n_q / n_kv;
#define CBQ_ATTN_SPLIT(HD)                                                                      \
    hipLaunchKernelGGL(attn_rope_split_kernel<HD>, dim3(n_q, S), dim3(kSplitThreads), 0, stream, \
                       q, k, v, q_weight, k_weight, cos_table, sin_table, pos, k_cache, v_cache,  \
                       part, group, max_len, scale, eps);                                          \
    hipLaunchKernelGGL(attn_combine_kernel<HD>, dim3(n_q), dim3(HD), 0, stream, part, S, out)
    switch (hd) {
    case 64: CBQ_ATTN_SPLIT(64); break;
    case 128: CBQ_ATTN_SPLIT(128); break;
    default: CBQ_ATTN_SPLIT(256); break;
    }
#undef CBQ_ATTN_SPLIT
    return cbq_launch_status("attn_combine_kernel");
}

}  // namespace

extern "C" {

int cbq_add_rmsnorm_f32(float *h, const float *delta, const float *weight, float *out, int T,
                        int H, float eps, hipStream_t stream)
{
    if (!h || !out || out == h || T <= 0 || H <= 0 || T > 65535 || H > kNormThreads * kNormPer)
        return CK_ERR_ARG;
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(T), dim3(kNormThreads), 0, stream, h, delta,
                       weight, out, H, eps);
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

int cbq_attn_rope_decode_f32(const float *q, const float *k, const float *v,
                             const float *q_weight, const float *k_weight,
                             const float *cos_table, const float *sin_table, const int64_t *pos,
                             float *k_cache, float *v_cache, float *out, int n_q, int n_kv,
                             int hd, int max_len, float scale, float eps, hipStream_t stream)
{
    if (!q || !k || !v || !cos_table || !sin_table || !pos || !k_cache || !v_cache || !out)
        return CK_ERR_ARG;
    if (n_q <= 0 || n_kv <= 0 || n_q % n_kv || max_len <= 0 || max_len > kAttnMaxLen)
        return CK_ERR_ARG;
    if (((uintptr_t)k_cache & 15) != 0) return CK_ERR_ARG;       // 16-byte key rows
    const size_t lds = (size_t)(max_len + 1) * sizeof(float);
    const int group = n_q / n_kv;
#define CBQ_ATTN_ROPE(HD)                                                                     \
    hipLaunchKernelGGL(attn_rope_decode_kernel<HD>, dim3(n_q), dim3(kAttnThreads), lds, stream, \
                       q, k, v, q_weight, k_weight, cos_table, sin_table, pos, k_cache, v_cache, \
                       out, group, max_len, scale, eps)
    switch (hd) {
    case 64: CBQ_ATTN_ROPE(64); break;
    case 128: CBQ_ATTN_ROPE(128); break;
    case 256: CBQ_ATTN_ROPE(256); break;
    default: return CK_ERR_ARG;
    }
#undef CBQ_ATTN_ROPE
    return cbq_launch_status("attn_rope_decode_kernel");
}

size_t cbq_attn_rope_decode_workspace(int n_q, int hd, int max_len)
{
    if (n_q <= 0 || hd <= 0 || max_len <= 0) return 0;
    return (size_t)n_q * attn_split_count(max_len) * (hd + 2) * sizeof(float);
}

int cbq_attn_rope_decode_ws_f32(const float *q, const float *k, const float *v,
                                const float *q_weight, const float *k_weight,
                                const float *cos_table, const float *sin_table,
                                const int64_t *pos, float *k_cache, float *v_cache, float *out,
                                int n_q, int n_kv, int hd, int max_len, float scale, float eps,
                                void *workspace, size_t workspace_bytes, hipStream_t stream)
{
    if (!workspace || ((uintptr_t)workspace & 3) != 0) return CK_ERR_ARG;
    const int rc = attn_split_check(q, k, v, cos_table, sin_table, pos, k_cache, v_cache, out,
                                    n_q, n_kv, hd, max_len);
    if (rc) return rc;
    if (workspace_bytes < cbq_attn_rope_decode_workspace(n_q, hd, max_len)) return CK_ERR_ARG;
    return attn_split_launch(q, k, v, q_weight, k_weight, cos_table, sin_table, pos, k_cache,
                             v_cache, out, n_q, n_kv, hd, max_len, scale, eps,
                             (float *)workspace, stream);
}

int cbq_attn_rope_decode_noalloc_f32(const float *q, const float *k, const float *v,
                                     const float *q_weight, const float *k_weight,
                                     const float *cos_table, const float *sin_table,
                                     const int64_t *pos, float *k_cache, float *v_cache,
                                     float *out, int n_q, int n_kv, int hd, int max_len,
                                     float scale, float eps, hipStream_t stream)
{
    int rc = attn_split_check(q, k, v, cos_table, sin_table, pos, k_cache, v_cache, out, n_q,
                              n_kv, hd, max_len);
    if (rc) return rc;
    const size_t need = cbq_attn_rope_decode_workspace(n_q, hd, max_len);
    if (need > sizeof(scratch)) {
        fprintf(stderr,
                "[cbq_hip] cbq_attn_rope_decode_noalloc_f32: n_q=%d hd=%d max_len=%d needs %zu "
                "bytes of split partials, above the %zu-byte static scratch; use "
                "cbq_attn_rope_decode_ws_f32 with a workspace\n",
                n_q, hd, max_len, need, sizeof(scratch));
        return CK_ERR_ARG;
    }
    float *part = nullptr;
    rc = scratch_address(&part);
    if (rc) return rc;
    return attn_split_launch(q, k, v, q_weight, k_weight, cos_table, sin_table, pos, k_cache,
                             v_cache, out, n_q, n_kv, hd, max_len, scale, eps, part, stream);
}

int cbq_argmax_step(const float *logits, int n, void *workspace, int32_t *ids32, int64_t *toks,
                    int64_t *pos, int64_t first, int64_t n_toks, hipStream_t stream)
{
    if (!logits || n <= 0 || !workspace || !ids32 || !toks || !pos || n_toks <= 0)
        return CK_ERR_ARG;
    float *part_v = (float *)workspace;
    int *part_i = (int *)(part_v + kArgBlocks);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks), dim3(kArgThreads), 0, stream,
                       logits, n, part_v, part_i);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgBlocks), 0, stream, part_v, part_i,
                       n, ids32, toks, pos, first, n_toks);
    return cbq_launch_status("argmax_final_kernel");
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
