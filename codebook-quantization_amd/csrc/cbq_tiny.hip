// Fixed-width GEMM for a few tokens (2 <= T <= 16; ck_linear_f32 and
// ck_linear_bf16 send it tiles of 5..16) on the fp32 matrix cores of gfx950
// (v_mfma_f32_16x16x4_f32)
// (rocm/compressed_kernel.hip:607-627 is the reference entry point; its
// kernel runs one block per output scalar).
//
// Same arithmetic as the reference's loop (src/compressed_matmul.c:416-450):
// out[t, r] = sum_k x[t, k] * cb[min(idx[r, k], C - 1)], fp32 products
// (exact in the fp32 MFMA) and fp32 sums in a different order.
//
// A wave owns a tile of 16 rows and a quarter of the 32-index groups of K.
// Per group, lane l decodes indices 8j .. 8j+7 (j = l / 16) of row l % 16:
// one 4-dword window of the packed row holds them for every width here (the
// 16 rows' groups arrive with one 16-byte load per lane and are rearranged
// through LDS).  The
// group then takes 8 MFMAs; in step s the k slot j stands for column
// 32 g + 8 j + s, for the weights (A: row l % 16, slot l / 16) and for x
// (B: slot l / 16, token l % 16) alike, so the 16 x 16 product is exact for
// any T <= 16.  x rows are read straight from memory (two float4 per lane and
// group, shared by the 16 rows).  The four quarters of a row tile are summed
// through LDS in order.  Tokens past T compute on token 0's x and are not
// written.
#include "cbq_device.h"

#include <algorithm>

namespace {

constexpr int kTinyWaves = 8;                 // 2 row tiles x 4 column quarters
constexpr int kTinyThreads = kTinyWaves * CBQ_WAVE;
constexpr int kTinyRing = 4;                  // groups in flight per wave
constexpr int kTinyMaxCodebook = 16384;

typedef float f4 __attribute__((ext_vector_type(4)));

// LDS written by some lanes of a wave, then read by others: keep the
// compiler from moving the accesses across (the hardware runs a wave's LDS
// operations in order).
__device__ __forceinline__ void wave_sync_lds()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// x in XT (fp32, or bf16 widened exactly); out in OT (one rounding for bf16).
template <int BITS, typename XT, typename OT>
__global__ __launch_bounds__(kTinyThreads) void fixed_tiny_mfma_kernel(
    const XT *__restrict__ x, const uint32_t *__restrict__ words,
    const float *__restrict__ cb, OT *__restrict__ out, int T, int M, int K, int C)
{
    static_assert(BITS >= 8 && BITS <= 16, "widths with a 4-dword 8-index window");
    // codebook [cs], partials [8][64][4], then per wave kTinyRing slots of
    // 16 rows x 16 words of packed groups
    extern __shared__ __attribute__((aligned(16))) float s_dyn[];
    const int G = K >> 5;
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = threadIdx.x / CBQ_WAVE;
    const int tile = wave & 1, quarter = wave >> 1;
    const int r0 = (blockIdx.x * 2 + tile) * 16;
    const int j = lane >> 4, tok = lane & 15;
    const int Gq = (G + 3) >> 2;
    const int ga = quarter * Gq < G ? quarter * Gq : G;
    const int gb = ga + Gq < G ? ga + Gq : G;
    const int cs = (C + 63) & ~63;
    f4 *s_part = (f4 *)(s_dyn + cs);
    uint32_t *s_w = (uint32_t *)(s_dyn + cs + kTinyWaves * CBQ_WAVE * 4) +
                    wave * (kTinyRing * 16 * 16);

    stage_clamped(s_dyn, cb, C, cs);

    // this lane's 8 indices of a group: bits [8 j BITS, 8 j BITS + 8 BITS)
    constexpr uint32_t mask = (1u << BITS) - 1u;
    const int wbit = j * 8 * BITS;
    const int w0 = wbit >> 5;
    const int boff = wbit & 31;
    const int lastq = ((wbit + 8 * BITS - 1) >> 5) - w0;     // last word of the window, <= 3
    const XT *xrow = x + (size_t)(tok < T ? tok : 0) * K + 8 * j;
    // loads: lane l fetches 4 words of row l / 4's group, at word
    // min(4 (l % 4), BITS - 4), so one 16-byte load per lane covers the 16
    // rows' groups and never leaves a group; they pass through LDS to the
    // MFMA layout (lane l: row l % 16, words w0 .. w0+3 of its window)
    const int lr = lane >> 2;
    const int loff = (4 * (lane & 3)) < BITS - 4 ? 4 * (lane & 3) : BITS - 4;
    const int lrow = r0 + lr < M ? r0 + lr : M - 1;
    const uint32_t *lsrc = words + (size_t)lrow * G * BITS + loff;

    uint32_t wr[kTinyRing][4];
    f4 xa[kTinyRing], xb[kTinyRing];
    auto load = [&](int d, int g) {
        const int gg = g < gb ? g : (gb > 0 ? gb - 1 : 0);
        __builtin_memcpy(wr[d], lsrc + (size_t)gg * BITS, sizeof(wr[d]));
        if constexpr (sizeof(XT) == 4) {
            const f4 *xp = (const f4 *)(xrow + (size_t)gg * 32);
            xa[d] = xp[0];
            xb[d] = xp[1];
        } else {                                // 8 bf16 values: 16 bytes
            uint32_t h[4];
            __builtin_memcpy(h, xrow + (size_t)gg * 32, sizeof(h));
            xa[d] = (f4){__uint_as_float(h[0] << 16), __uint_as_float(h[0] & 0xffff0000u),
                         __uint_as_float(h[1] << 16), __uint_as_float(h[1] & 0xffff0000u)};
            xb[d] = (f4){__uint_as_float(h[2] << 16), __uint_as_float(h[2] & 0xffff0000u),
                         __uint_as_float(h[3] << 16), __uint_as_float(h[3] & 0xffff0000u)};
        }
    };
#pragma unroll
    for (int d = 0; d < kTinyRing; d++) load(d, ga + d);
    __syncthreads();                           // codebook staged

    // four accumulators (step s goes to acc[s % 4]) keep four MFMAs in
    // flight; every ring slot is reloaded unconditionally (clamped group) so
    // the wait counts stay exact
    f4 acc[4];
#pragma unroll
    for (int a = 0; a < 4; a++) acc[a] = (f4){0.f, 0.f, 0.f, 0.f};
    for (int g = ga; g < gb; g += kTinyRing) {
#pragma unroll
        for (int d = 0; d < kTinyRing; d++) {
            const bool live = g + d < gb;
            uint32_t *sw = s_w + d * 256;
#pragma unroll
            for (int k = 0; k < 4; k++) sw[lr * 16 + loff + k] = wr[d][k];
            wave_sync_lds();
            uint32_t wb[4];
#pragma unroll
            for (int k = 0; k < 4; k++) wb[k] = sw[tok * 16 + w0 + (k < lastq ? k : lastq)];
            wave_sync_lds();
            const unsigned __int128 win =
                ((unsigned __int128)(((uint64_t)wb[3] << 32) | wb[2]) << 64 |
                 (((uint64_t)wb[1] << 32) | wb[0])) >> boff;
            const uint64_t lo = (uint64_t)win, hi = (uint64_t)(win >> 64);
            const float xs[8] = {xa[d].x, xa[d].y, xa[d].z, xa[d].w,
                                 xb[d].x, xb[d].y, xb[d].z, xb[d].w};
            float wv[8];
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const int sh = s * BITS;
                uint32_t idx;
                if (sh + BITS <= 64) idx = (uint32_t)(lo >> sh) & mask;
                else if (sh >= 64) idx = (uint32_t)(hi >> (sh - 64)) & mask;
                else idx = (uint32_t)((lo >> sh) | (hi << (64 - sh))) & mask;
                wv[s] = s_dyn[idx < (uint32_t)C ? idx : (uint32_t)(C - 1)];
            }
            load(d, g + d + kTinyRing);
            if (live) {
#pragma unroll
                for (int s = 0; s < 8; s++)
                    acc[s & 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[s], xs[s], acc[s & 3], 0, 0, 0);
            }
        }
    }
    f4 sum4;
    sum4.x = (acc[0].x + acc[1].x) + (acc[2].x + acc[3].x);
    sum4.y = (acc[0].y + acc[1].y) + (acc[2].y + acc[3].y);
    sum4.z = (acc[0].z + acc[1].z) + (acc[2].z + acc[3].z);
    sum4.w = (acc[0].w + acc[1].w) + (acc[2].w + acc[3].w);

    s_part[wave * CBQ_WAVE + lane] = sum4;
    __syncthreads();
    if (quarter == 0) {
        f4 sum = s_part[tile * CBQ_WAVE + lane];
#pragma unroll
        for (int q = 1; q < 4; q++) {
            const f4 v = s_part[(q * 2 + tile) * CBQ_WAVE + lane];
            sum.x += v.x;
            sum.y += v.y;
            sum.z += v.z;
            sum.w += v.w;
        }
        // D[m][n]: lane l, element v holds row m = 4 (l / 16) + v, token n = l % 16
        const float vals[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int m = r0 + 4 * j + v;
            if (m < M && tok < T) out[(size_t)tok * M + m] = from_f32<OT>(vals[v]);
        }
    }
}

template <typename XT, typename OT>
int tiny_launch(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T, int M,
                int K, int C, int bits, hipStream_t st)
{
    if (T < 2 || T > 16 || M <= 0 || K <= 0 || K % 32 || C <= 0 || C > kTinyMaxCodebook)
        return -1;
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)packed & 3) != 0) return -1;
    const int cs = (C + 63) & ~63;
    const size_t lds = (size_t)cs * 4 + (size_t)kTinyWaves * CBQ_WAVE * 16 +
                       (size_t)kTinyWaves * kTinyRing * 16 * 16 * 4;
    const int blocks = (M + 31) / 32;
#define CBQ_TINY(B)                                                                            \
    hipLaunchKernelGGL((fixed_tiny_mfma_kernel<B, XT, OT>), dim3(blocks), dim3(kTinyThreads),  \
                       lds, st, x, (const uint32_t *)packed, cb, out, T, M, K, C)
    switch (bits) {
    case 8: CBQ_TINY(8); break;
    case 10: CBQ_TINY(10); break;
    case 11: CBQ_TINY(11); break;
    case 12: CBQ_TINY(12); break;
    case 13: CBQ_TINY(13); break;
    case 14: CBQ_TINY(14); break;
    case 16: CBQ_TINY(16); break;
    default: return -1;
    }
#undef CBQ_TINY
    return cbq_launch_status("fixed_tiny_mfma_kernel");
}

}  // namespace

// 2 <= T <= 16 tokens (fp32, or bf16 x and out), K % 32 == 0, widths 8,
// 10-14 and 16: the kernel above; returns -1 for shapes it does not take
// (the caller then uses its other paths).
int cbq_fixed_tiny_t(const float *x, const uint8_t *packed, const float *cb, float *out, int T,
                     int M, int K, int C, int bits, hipStream_t st)
{
    return tiny_launch<float, float>(x, packed, cb, out, T, M, K, C, bits, st);
}

int cbq_fixed_tiny_t_bf16(const uint16_t *x, const uint8_t *packed, const float *cb,
                          uint16_t *out, int T, int M, int K, int C, int bits, hipStream_t st)
{
    return tiny_launch<uint16_t, uint16_t>(x, packed, cb, out, T, M, K, C, bits, st);
}
