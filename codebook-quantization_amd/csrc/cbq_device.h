// Device-side helpers shared by the gfx950 kernels: wave64 reductions and
// scans, bf16 conversion, error plumbing for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/cbq_hip.h"

#define CBQ_WAVE 64

// Launch-error check shared by every C entry point.
static inline int cbq_launch_status(const char *what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fprintf(stderr, "[cbq_hip] %s: %s\n", what, hipGetErrorString(e));
        return CK_ERR_HIP;
    }
    return CK_SUCCESS;
}

// Number of compute units of the current device (cached per device id).
int cbq_num_cus();

// ---- greedy pick (argmax) ----------------------------------------------------
// Order of (value, index) candidates: the larger value, then the smaller
// index; NaN ranks highest (the first NaN wins), as torch.argmax.  An empty
// candidate is (-inf, kArgNone): it loses to every real index.
constexpr int kArgNone = 0x7fffffff;

__device__ __forceinline__ bool arg_better(float a, int ia, float b, int ib)
{
    const bool na = a != a, nb = b != b;
    if (na || nb) return na && (!nb || ia < ib);
    return a > b || (a == b && ia < ib);
}

__device__ __forceinline__ void arg_wave_reduce(float &best, int &bi)
{
    for (int o = CBQ_WAVE >> 1; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, CBQ_WAVE);
        const int oi = __shfl_xor(bi, o, CBQ_WAVE);
        if (arg_better(ov, oi, best, bi)) { best = ov; bi = oi; }
    }
}

// The block's best candidate into part_v / part_i [blockIdx.x]; every thread
// of the block calls it.  s_v / s_i: one slot per wave.
__device__ __forceinline__ void arg_block_store(float best, int bi, float *s_v, int *s_i,
                                                float *part_v, int *part_i)
{
    arg_wave_reduce(best, bi);
    if ((threadIdx.x & (CBQ_WAVE - 1)) == 0) {
        s_v[threadIdx.x / CBQ_WAVE] = best;
        s_i[threadIdx.x / CBQ_WAVE] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x / CBQ_WAVE); w++)
            if (arg_better(s_v[w], s_i[w], best, bi)) { best = s_v[w]; bi = s_i[w]; }
        part_v[blockIdx.x] = best;
        part_i[blockIdx.x] = bi;
    }
}

// Second launch of a fused greedy pick (cbq_decode.hip): merges n_part
// (value, index) pairs, then ids32[0] = tok; toks[pos[0] - first] = tok when
// that index lies in [0, n_toks); pos[0] += 1 (tok = 0 when no candidate
// is below n).
int cbq_argmax_merge(const float *part_v, const int *part_i, int n_part, int n, int32_t *ids32,
                     int64_t *toks, int64_t *pos, int64_t first, int64_t n_toks,
                     hipStream_t stream);
// Bytes of the pairs a fused GEMV + pick writes: one per block, at most 1024.
constexpr int kArgMaxParts = 1024;

__device__ __forceinline__ float bf16_to_f32(uint16_t h)
{
    return __uint_as_float((uint32_t)h << 16);
}

// Round-to-nearest-even float -> bf16 bit pattern; NaN stays quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

template <typename XT> __device__ __forceinline__ float to_f32(XT v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

template <typename OT> __device__ __forceinline__ OT from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) { return f32_to_bf16(v); }

// ---- exact products on the bf16 matrix cores --------------------------------
typedef __bf16 cbq_bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t cbq_u32x4 __attribute__((ext_vector_type(4)));
typedef float cbq_f32x4 __attribute__((ext_vector_type(4)));

// bf16 bits of a (low half) and of b (high half), both truncated: v_perm
// picks the upper two bytes of each
__device__ __forceinline__ uint32_t cbq_hi_pair(uint32_t a, uint32_t b)
{
    return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// v = h + m + l exactly, each a bf16 number (8 values, packed two to a
// dword): h keeps the top 8 significand bits of v (its low 16 bits
// cleared), m the same of r = v - h, l = r - m; both differences are exact
// in fp32 and l has at most 8 significant bits
__device__ __forceinline__ void cbq_split3(const float (&v)[8], cbq_u32x4 &h, cbq_u32x4 &m,
                                           cbq_u32x4 &l)
{
    uint32_t hp[4], mp[4], lp[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const uint32_t a = __float_as_uint(v[e]), b = __float_as_uint(v[e + 1]);
        const float ra = v[e] - __uint_as_float(a & 0xffff0000u);
        const float rb = v[e + 1] - __uint_as_float(b & 0xffff0000u);
        const uint32_t ua = __float_as_uint(ra), ub = __float_as_uint(rb);
        const float la = ra - __uint_as_float(ua & 0xffff0000u);
        const float lb = rb - __uint_as_float(ub & 0xffff0000u);
        hp[e >> 1] = cbq_hi_pair(a, b);
        mp[e >> 1] = cbq_hi_pair(ua, ub);
        lp[e >> 1] = cbq_hi_pair(__float_as_uint(la), __float_as_uint(lb));
    }
    h = cbq_u32x4{hp[0], hp[1], hp[2], hp[3]};
    m = cbq_u32x4{mp[0], mp[1], mp[2], mp[3]};
    l = cbq_u32x4{lp[0], lp[1], lp[2], lp[3]};
}

// c + A * B on v_mfma_f32_16x16x32_bf16: lane l holds A row l % 16 and B
// column l % 16, k = 8 (l / 16) .. +7 of both; D lane l: rows 4 (l / 16) + v,
// column l % 16
__device__ __forceinline__ cbq_f32x4 cbq_mfma_bf16(cbq_u32x4 a, cbq_u32x4 b, cbq_f32x4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(cbq_bf16x8, a),
                                                   __builtin_bit_cast(cbq_bf16x8, b), c, 0, 0, 0);
}

// dst[i] = src[min(i, n_src - 1)] for i < n_dst (0 < n_src <= n_dst), global
// to LDS by the whole block, with a thread's loads (up to 8 pieces) in flight
// before its first store: one round trip per 8 pieces rather than one per
// element.  16-byte pieces over the aligned whole pieces of src; indices past
// the end repeat the last one (the same value to the same place), so nothing
// is conditional and no wait is needed between batches.
__device__ __forceinline__ void stage_clamped(float *dst, const float *__restrict__ src,
                                              int n_src, int n_dst)
{
    typedef float v4 __attribute__((ext_vector_type(4)));
    const int nt = (int)blockDim.x, t = (int)threadIdx.x;
    int done = 0;
    const int n4 = n_src >> 2;
    if ((((uintptr_t)src | (uintptr_t)dst) & 15) == 0 && n4 > 0) {
        const v4 *s4 = (const v4 *)src;
        v4 *d4 = (v4 *)dst;
        for (int b = 0; b < n4; b += 8 * nt) {
            v4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = s4[min(b + u * nt + t, n4 - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) d4[min(b + u * nt + t, n4 - 1)] = v[u];
        }
        done = n4 << 2;
    }
    for (int b = done; b < n_dst; b += 8 * nt) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = src[min(min(b + u * nt + t, n_dst - 1), n_src - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) dst[min(b + u * nt + t, n_dst - 1)] = v[u];
    }
}

// Butterfly sum over aligned groups of `width` lanes (power of two <= 64);
// every lane of a group ends with the group total.
__device__ __forceinline__ float group_sum(float v, int width)
{
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, CBQ_WAVE);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum(v, CBQ_WAVE); }

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v)
{
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    for (int o = 1; o < CBQ_WAVE; o <<= 1) {
        uint32_t u = __shfl_up(v, o, CBQ_WAVE);
        if (lane >= o) v += u;
    }
    return v;
}

// The decoder's glue arithmetic, shared by the standalone glue kernels and
// the GEMVs that fold the glue into their x staging, so that both paths
// round alike.  hipcc contracts a * b + c into one fma by default, and
// whether it does depends on the surrounding code; these helpers switch
// contraction off, so every operation rounds on its own (as torch's
// elementwise ops do) wherever they are inlined.

// ss + v * v, two roundings.
__device__ __forceinline__ float add_square(float ss, float v)
{
#pragma clang fp contract(off)
    return ss + v * v;
}

// silu(g) * u = g / (1 + exp(-g)) * u on the hardware exp2 and reciprocal
// (v_exp_f32 of -g log2(e), v_rcp_f32; each about 1 ulp): 6 instructions
// where expf and an IEEE divide take ~22, which matters for a GEMV that
// stages silu(gate) * up for all 12 288 columns in every block.  Relative
// error below 1e-6 for |g| < 16, and the limits hold: g -> -inf gives -0
// (exp overflows, rcp(inf) = 0), g -> +inf gives g * u.
__device__ __forceinline__ float silu_mul_value(float g, float u)
{
#pragma clang fp contract(off)
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504f);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// The activation transforms a GEMV can apply while it stages x (T = 1):
// 1: silu(x0) * x1; 2: rmsnorm(x0 + x1) (x0 + x1 also stored to h_out by
// one block); 3: rmsnorm(x0).  Rounded as the separate decoder kernels
// round, so fused and unfused paths give identical x.
enum { XF_NONE = 0, XF_SILU = CBQ_XF_SILU, XF_ADD_RMS = CBQ_XF_ADD_RMS, XF_RMS = CBQ_XF_RMS };

// The same transform of element i from values already loaded (v0 = x0[i],
// v1 = x1[i] where the mode reads x1).
__device__ __forceinline__ float xform_of(int mode, float v0, float v1, float *h_out,
                                          bool store_h, int i, float r)
{
#pragma clang fp contract(off)
    if (mode == XF_SILU) return silu_mul_value(v0, v1);
    float v = v0;
    if (mode == XF_ADD_RMS) {
        v = v + v1;
        if (store_h) h_out[i] = v;
    }
    return v * r;
}

__device__ __forceinline__ float xform_value(int mode, const float *__restrict__ x0,
                                             const float *__restrict__ x1, float *h_out,
                                             bool store_h, int i, float r)
{
    const bool two = mode == XF_SILU || mode == XF_ADD_RMS;
    return xform_of(mode, x0[i], two ? x1[i] : 0.f, h_out, store_h, i, r);
}

// Workgroup barrier for LDS hand-off only: waits for this wave's LDS
// operations, then s_barrier.  Unlike __syncthreads() it does not wait for
// outstanding global loads, so prefetched weight data stays in flight.
__device__ __forceinline__ void lds_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The glue-transformed x of a one-token GEMV, held in registers (K <= 16384).
// Thread tid of an NTHR-thread block owns the elements i = vt + 1024 j
// (i < K) of its virtual threads vt = tid + k NTHR, k < 1024 / NTHR,
// j < 16.  load() only issues the global loads, so a kernel can start its
// weight stream before finish() consumes them.  The RMSNorm sum runs in
// exactly the order of a 1024-thread block whose thread vt adds the
// squares of v[vt + 1024 j] for j = 0..15 (terms past K are +0), whose
// waves reduce by wave_sum and whose 16 wave sums add in wave order: the
// decoder's standalone RMSNorm kernel.  NJ < 16 holds only j < NJ, for
// K <= 1024 NJ (the terms it drops are +0 and leave the sums unchanged).
template <int NTHR, int XMODE, int NJ = 16>
struct GlueTile {
    static_assert(1024 % NTHR == 0 && NTHR >= CBQ_WAVE, "block size divides 1024");
    static_assert(NJ >= 1 && NJ <= 16, "16 terms per virtual thread at most");
    static constexpr int VPT = 1024 / NTHR;
    static constexpr int kJ = NJ;
    static constexpr bool TWO = XMODE == XF_SILU || XMODE == XF_ADD_RMS;
    float a[VPT][NJ];
    float b[TWO ? VPT : 1][NJ];

    __device__ __forceinline__ void load(const float *__restrict__ x0,
                                         const float *__restrict__ x1, int K)
    {
        // unconditional loads (past K: element K - 1 again, zeroed in
        // finish), so the wait for them leaves later weight loads in flight
#pragma unroll
        for (int k = 0; k < VPT; k++)
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int i = (int)threadIdx.x + k * NTHR + j * 1024;
                const int ic = i < K ? i : K - 1;
                a[k][j] = x0[ic];
                if constexpr (TWO) b[k][j] = x1[ic];
            }
    }

    // Applies the transform in place; returns the RMSNorm scale (1 for
    // SiLU).  Norm modes contain one block barrier (LDS only, global loads stay
    // in flight) and use s_red16 (16
    // floats of LDS, not written again before the next barrier).
    __device__ __forceinline__ float finish(int K, float eps, float *s_red16)
    {
#pragma clang fp contract(off)
#pragma unroll
        for (int k = 0; k < VPT; k++)
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                if ((int)threadIdx.x + k * NTHR + j * 1024 >= K) {   // terms past K are +0
                    a[k][j] = 0.f;
                    if constexpr (TWO) b[k][j] = 0.f;
                }
                if constexpr (XMODE == XF_SILU) a[k][j] = silu_mul_value(a[k][j], b[k][j]);
                if constexpr (XMODE == XF_ADD_RMS) a[k][j] = a[k][j] + b[k][j];
            }
        if constexpr (XMODE == XF_SILU) return 1.f;
#pragma unroll
        for (int k = 0; k < VPT; k++) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < NJ; j++) ss = add_square(ss, a[k][j]);
            ss = wave_sum(ss);
            if ((threadIdx.x & (CBQ_WAVE - 1)) == 0)
                s_red16[((int)threadIdx.x + k * NTHR) / CBQ_WAVE] = ss;
        }
        lds_barrier();
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < 16; w++) t += s_red16[w];
        return rsqrtf(t / (float)K + eps);
    }

    // Element i of the staged x (v * r for the norms, v for SiLU).
    __device__ __forceinline__ float value(int k, int j, float r) const
    {
#pragma clang fp contract(off)
        return XMODE == XF_SILU ? a[k][j] : a[k][j] * r;
    }

    // x0 + x1 (ADD_RMS) to h_out.
    __device__ __forceinline__ void store_sum(float *h_out, int K) const
    {
        if constexpr (XMODE == XF_ADD_RMS)
#pragma unroll
            for (int k = 0; k < VPT; k++)
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    const int i = (int)threadIdx.x + k * NTHR + j * 1024;
                    if (i < K) h_out[i] = a[k][j];
                }
    }
};

// b-bit field starting at bit `s` of the little-endian pair (hi:lo).
__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t s)
{
    return __builtin_amdgcn_alignbit(hi, lo, s);
}

// Byte offsets into the LDS codebook of the 32 indices of one group: each
// field is extracted already shifted left by 2 (alignbit/shift + and).  A
// PADDED codebook has 2^BITS entries (entries >= C repeat cb[C-1]), so the
// index clamp of the reference (idx >= C -> C-1) costs nothing; otherwise the
// offset is clamped to 4*(C-1).
template <int BITS, bool PADDED>
__device__ __forceinline__ void group_offsets(const uint32_t (&w)[BITS], uint32_t cmax4,
                                              uint32_t off[32])
{
    constexpr uint32_t m4 = ((1u << BITS) - 1u) << 2;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const int o = j * BITS, q = o >> 5, s = o & 31;
        uint32_t a;
        if (s >= 2)
            a = (s + BITS <= 32) ? ((w[q] >> (s - 2)) & m4)
                                 : (funnel(w[q + 1], w[q], (uint32_t)(s - 2)) & m4);
        else
            a = (w[q] << (2 - s)) & m4;
        if (!PADDED) a = a < cmax4 ? a : cmax4;
        off[j] = a;
    }
}
