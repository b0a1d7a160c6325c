// Fixed-width GEMM for a few tokens (2 <= T <= 16; ck_linear_f32 and
// ck_linear_bf16 send it tiles of 2..16) on the matrix cores of gfx950
// (rocm/compressed_kernel.hip:607-627 is the reference entry point; its
// kernel runs one block per output scalar).
//
// Same arithmetic as the reference's loop (src/compressed_matmul.c:416-450):
// out[t, r] = sum_k x[t, k] * cb[min(idx[r, k], C - 1)], exact products and
// fp32 sums in a different order.
//
// fixed_fewtok_kernel (K % 128 == 0): bf16 matrix cores
// (v_mfma_f32_16x16x32_bf16).  The codebook values are bf16 numbers (the
// lossless codebooks are bf16 weights), and an fp32 x is split exactly into
// three bf16 parts, x = h + m + l (truncations: h keeps the top 8 significand
// bits, m the next 8 of x - h, l = x - h - m the rest, at most 8 bits), so
// every product w * part is exact and the three MFMAs sum them in fp32.  A
// codebook with any entry that is not a bf16 number (found while staging
// it) is split the same way and six MFMAs of the nine part products run
// (the three left out are below 2^-24 of the product).  bf16 x is one part.
//   - Block: 8 waves over R tiles of 16 rows; wave w takes the 128-column
//     steps w, w + 8, w + 16, ... (the block's waves read neighbouring spans
//     of each row at the same time).
//   - A tile-step (16 rows x 4 groups of 32 indices) is loaded with 16-byte
//     chunks, consecutive lanes on consecutive bytes of a row, Q tile-steps
//     ahead into registers; a wave-private LDS buffer re-lays it so that
//     lane l holds group l / 16 of row l % 16 (BITS words).
//   - MFMA c of a tile-step takes chunk c (indices 8c .. 8c+7) of each of the
//     step's four groups, for the weights (A: row l % 16) and for x (B: token
//     l % 16) alike.  x of a step is split once and serves the R tiles.
//   - The 8 waves' partial tiles are summed through LDS in wave order.
// Measured against the per-lane loads of one 52-byte group each (16 rows x
// 4 groups per instruction): 44.6 us for the 163.6 MB stacked gate+up read
// alone against 30.9 us for these chunk loads.
//
// fixed_tiny_mfma_kernel (K % 32 == 0 otherwise): fp32 matrix cores
// (v_mfma_f32_16x16x4_f32).  A wave owns a tile of 16 rows and a quarter of
// the 32-index groups of K.  Per group, lane l decodes indices 8j .. 8j+7
// (j = l / 16) of row l % 16: one 4-dword window of the packed row holds
// them for every width here (the 16 rows' groups arrive with one 16-byte
// load per lane and are rearranged through LDS).  The group then takes 8
// MFMAs; in step s the k slot j stands for column 32 g + 8 j + s, for the
// weights (A: row l % 16, slot l / 16) and for x (B: slot l / 16, token
// l % 16) alike, so the 16 x 16 product is exact for any T <= 16.  x rows are
// read straight from memory (two float4 per lane and group, shared by the 16
// rows).  The four quarters of a row tile are summed through LDS in order.
// Tokens past T compute on token 0's x and are not written.
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

// ---- fixed_fewtok_kernel ------------------------------------------------------

constexpr int kFtWaves = 8;
constexpr int kFtThreads = kFtWaves * CBQ_WAVE;

typedef cbq_u32x4 u32x4;

// x of one lane and step: 32 values of token l % 16, group l / 16 of the step
template <typename XT> struct FtX;
template <> struct FtX<float> {
    static constexpr int kWords = 32;
    static constexpr int kParts = 3;
    __device__ static void parts(const uint32_t (&xw)[kWords], u32x4 (&b)[4][3])
    {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float q[8];
#pragma unroll
            for (int e = 0; e < 8; e++) q[e] = __uint_as_float(xw[8 * c + e]);
            cbq_split3(q, b[c][0], b[c][1], b[c][2]);
        }
    }
};
template <> struct FtX<uint16_t> {
    static constexpr int kWords = 16;
    static constexpr int kParts = 1;
    __device__ static void parts(const uint32_t (&xw)[kWords], u32x4 (&b)[4][3])
    {
#pragma unroll
        for (int c = 0; c < 4; c++)
            b[c][0] = u32x4{xw[4 * c], xw[4 * c + 1], xw[4 * c + 2], xw[4 * c + 3]};
    }
};

// R row tiles per block, Q tile-steps of weights in flight per wave (Q
// divides R, so every ring slot is a compile-time register array).
template <int BITS, int R, int Q, typename XT, typename OT>
__global__ __launch_bounds__(kFtThreads) void fixed_fewtok_kernel(
    const XT *__restrict__ x, const uint32_t *__restrict__ words,
    const float *__restrict__ cb, OT *__restrict__ out, int T, int M, int K, int C)
{
    static_assert(R % Q == 0, "ring slots are static: Q divides R");
    static_assert(BITS >= 4 && BITS <= 16, "a group's words per lane");
    constexpr bool PADDED = BITS <= 14;           // 2^BITS-entry table: the clamp is free
    constexpr int NI = (BITS + 3) / 4;            // 16-byte loads per lane and tile-step
    constexpr int CH = 16 * BITS;                 // 16-byte chunks of a tile-step
    constexpr int XW = FtX<XT>::kWords;
    __shared__ __attribute__((aligned(16))) float s_cb[PADDED ? (1 << BITS) : kTinyMaxCodebook];
    __shared__ __attribute__((aligned(16))) uint32_t s_tr[kFtWaves][64 * BITS];
    __shared__ int s_flag[kFtWaves];
    extern __shared__ __attribute__((aligned(16))) f4 s_part[];     // [8][R][64]

    const int tid = threadIdx.x;
    const int lane = tid & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / CBQ_WAVE);
    const int rsub = lane & 15, j = lane >> 4;
    const int G = K >> 5;
    const int NS = G >> 2;                        // 128-column steps of a row
    const int Sw = NS > wave ? (NS - wave + kFtWaves - 1) / kFtWaves : 0;
    const int tile0 = blockIdx.x * R;
    const size_t rowstride = (size_t)G * BITS;    // words of a packed row
    const int C_eff = C < (1 << BITS) ? C : (1 << BITS);
    const int NT = PADDED ? (1 << BITS) : ((C_eff + 63) & ~63);

    // codebook loads first, so that waiting for them leaves the weight and
    // x loads below in flight
    constexpr int kMaxNE = ((PADDED ? (1 << BITS) : kTinyMaxCodebook) + kFtThreads - 1) / kFtThreads;
    const int NE = (NT + kFtThreads - 1) / kFtThreads;
    float cv[kMaxNE];
#pragma unroll
    for (int e = 0; e < kMaxNE; e++) {
        const int i = e * kFtThreads + tid;
        if (e < NE) cv[e] = cb[i < C_eff ? i : C_eff - 1];
    }
    __builtin_amdgcn_sched_barrier(0);

    // this lane's chunks of a tile-step: c = 64 k + lane -> row c / BITS,
    // 16-byte piece c % BITS of the row's 4 BITS words (lanes past CH re-read
    // the last chunk and store nothing)
    int crow[NI], cpiece[NI];
#pragma unroll
    for (int k = 0; k < NI; k++) {
        int c = 64 * k + lane;
        c = c < CH ? c : CH - 1;
        crow[k] = c / BITS;
        cpiece[k] = c % BITS;
    }
    // global step of local step s; steps past the wave's last re-read it (an L2 hit)
    auto gstep = [&](int s) {
        const int sl = s < Sw ? s : (Sw > 0 ? Sw - 1 : 0);
        const int g = kFtWaves * sl + wave;
        return g < NS ? g : NS - 1;
    };
    auto load_item = [&](int s, int t, u32x4 (&dst)[NI]) {
        const size_t col = (size_t)gstep(s) * 4 * BITS;
#pragma unroll
        for (int k = 0; k < NI; k++) {
            int row = (tile0 + t) * 16 + crow[k];
            row = row < M ? row : M - 1;
            __builtin_memcpy(&dst[k], words + (size_t)row * rowstride + col + 4 * cpiece[k], 16);
        }
    };
    auto load_x = [&](int s, uint32_t (&xw)[XW]) {
        if (rsub < T) {
            __builtin_memcpy(xw, x + (size_t)rsub * K + (size_t)(4 * gstep(s) + j) * 32,
                             sizeof(xw));
        } else {
#pragma unroll
            for (int i = 0; i < XW; i++) xw[i] = 0u;
        }
    };
    u32x4 wr[Q][NI];
#pragma unroll
    for (int q = 0; q < Q; q++) load_item(0, q, wr[q]);
    uint32_t xn[XW];
    load_x(0, xn);
    __builtin_amdgcn_sched_barrier(0);

    int inexact = 0;
#pragma unroll
    for (int e = 0; e < kMaxNE; e++) {
        const int i = e * kFtThreads + tid;
        if (e < NE && i < NT) {
            s_cb[i] = cv[e];
            inexact |= (__float_as_uint(cv[e]) & 0xffffu) != 0;
        }
    }
    {
        const bool any = __ballot(inexact) != 0;
        if (lane == 0) s_flag[wave] = any;
    }
    __syncthreads();                               // codebook and flags staged
    bool wsplit = false;
#pragma unroll
    for (int w = 0; w < kFtWaves; w++) wsplit |= s_flag[w] != 0;
    const uint32_t cmax4 = (uint32_t)(C_eff - 1) << 2;

    f4 acc[R];
#pragma unroll
    for (int t = 0; t < R; t++) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    uint32_t *tr = s_tr[wave];

    for (int s = 0; s < Sw; s++) {
        u32x4 xb[4][3];
        FtX<XT>::parts(xn, xb);
        load_x(s + 1, xn);                         // next step's x, one step ahead
#pragma unroll
        for (int t = 0; t < R; t++) {
            u32x4 (&slot)[NI] = wr[t % Q];
#pragma unroll
            for (int k = 0; k < NI; k++)
                if (64 * k + lane < CH) *(u32x4 *)(tr + 4 * (64 * k + lane)) = slot[k];
            wave_sync_lds();
            uint32_t w[BITS];
#pragma unroll
            for (int q = 0; q < BITS; q++) w[q] = tr[(rsub * 4 + j) * BITS + q];
            wave_sync_lds();
            // this slot's next tile-step, Q ahead in (step, tile) order
            if (t + Q < R) load_item(s, t + Q, slot);
            else load_item(s + 1, t + Q - R, slot);

            uint32_t off[32];
            group_offsets<BITS, PADDED>(w, cmax4, off);
            float wv[32];
#pragma unroll
            for (int q = 0; q < 32; q++) wv[q] = *(const float *)((const char *)s_cb + off[q]);
            u32x4 a[4];
#pragma unroll
            for (int c = 0; c < 4; c++)
                a[c] = u32x4{cbq_hi_pair(__float_as_uint(wv[8 * c]), __float_as_uint(wv[8 * c + 1])),
                             cbq_hi_pair(__float_as_uint(wv[8 * c + 2]), __float_as_uint(wv[8 * c + 3])),
                             cbq_hi_pair(__float_as_uint(wv[8 * c + 4]), __float_as_uint(wv[8 * c + 5])),
                             cbq_hi_pair(__float_as_uint(wv[8 * c + 6]), __float_as_uint(wv[8 * c + 7]))};
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int p = 0; p < FtX<XT>::kParts; p++) acc[t] = cbq_mfma_bf16(a[c], xb[c][p], acc[t]);
            if (wsplit) {                          // codebook not bf16: w = wh + wm + wl
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    float q8[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) q8[e] = wv[8 * c + e];
                    u32x4 wh, wm, wl;
                    cbq_split3(q8, wh, wm, wl);
                    acc[t] = cbq_mfma_bf16(wm, xb[c][0], acc[t]);
                    acc[t] = cbq_mfma_bf16(wl, xb[c][0], acc[t]);
                    if (FtX<XT>::kParts > 1) acc[t] = cbq_mfma_bf16(wm, xb[c][1], acc[t]);
                }
            }
        }
    }

    // the 8 waves' partial tiles, summed in wave order
#pragma unroll
    for (int t = 0; t < R; t++) s_part[(wave * R + t) * CBQ_WAVE + lane] = acc[t];
    __syncthreads();
    if (wave < R) {
        const int t = wave;
        f4 sum = s_part[t * CBQ_WAVE + lane];
#pragma unroll
        for (int w = 1; w < kFtWaves; w++) {
            const f4 v = s_part[(w * R + t) * CBQ_WAVE + lane];
            sum.x += v.x;
            sum.y += v.y;
            sum.z += v.z;
            sum.w += v.w;
        }
        // D[m][n]: lane l, element v holds row m = 4 (l / 16) + v, token n = l % 16
        const int n = lane & 15;
        const float vals[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int row = (tile0 + t) * 16 + 4 * j + v;
            if (row < M && n < T) out[(size_t)n * M + row] = from_f32<OT>(vals[v]);
        }
    }
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

template <int R, int Q, typename XT, typename OT>
int fewtok_launch_r(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T, int M,
                    int K, int C, int bits, int blocks, hipStream_t st)
{
    const size_t lds = (size_t)kFtWaves * R * CBQ_WAVE * sizeof(f4);
#define CBQ_FT(B)                                                                              \
    hipLaunchKernelGGL((fixed_fewtok_kernel<B, R, Q, XT, OT>), dim3(blocks), dim3(kFtThreads),  \
                       lds, st, x, (const uint32_t *)packed, cb, out, T, M, K, C)
    switch (bits) {
    case 8: CBQ_FT(8); break;
    case 10: CBQ_FT(10); break;
    case 11: CBQ_FT(11); break;
    case 12: CBQ_FT(12); break;
    case 13: CBQ_FT(13); break;
    case 14: CBQ_FT(14); break;
    case 16: CBQ_FT(16); break;
    default: return -1;
    }
#undef CBQ_FT
    return cbq_launch_status("fixed_fewtok_kernel");
}

// Row tiles per block R (6, 3, 2 or 1; a block holds one CU: 8 waves, up to
// 141 KiB of LDS): the R of least rounds x (R + 1), rounds =
// ceil(ceil(tiles / R) / CUs) and the + 1 a block's fixed cost in tiles
// (codebook staging, the first loads, the partial-tile sums), larger R on a
// tie.  E.g. 384 tiles on 256 CUs take R = 2 (one round of 192 blocks, 16
// us for the 9B stacked q/k/v at 2 tokens) rather than two rounds of R = 1
// (20 us); 1536 tiles take R = 6.
template <typename XT, typename OT>
int fewtok_launch(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T, int M,
                  int K, int C, int bits, hipStream_t st)
{
    if (T < 2 || T > 16 || M <= 0 || K <= 0 || K % 128 || C <= 0 || C > kTinyMaxCodebook)
        return -1;
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)packed & 15) != 0) return -1;
    if (bits != 8 && (bits < 10 || bits > 14) && bits != 16) return -1;
    const long tiles = (M + 15) / 16;
    const long ncu = cbq_num_cus();
    int R = 1;
    long best = -1;
    for (const int r : {1, 2, 3, 6}) {
        const long cost = ((tiles + r - 1) / r + ncu - 1) / ncu * (r + 1);
        if (best < 0 || cost <= best) {
            best = cost;
            R = r;
        }
    }
    const long blocks = (tiles + R - 1) / R;
    if (blocks > 0x7fffffffL) return -1;
    switch (R) {
    case 6: return fewtok_launch_r<6, 2>(x, packed, cb, out, T, M, K, C, bits, (int)blocks, st);
    case 3: return fewtok_launch_r<3, 3>(x, packed, cb, out, T, M, K, C, bits, (int)blocks, st);
    case 2: return fewtok_launch_r<2, 2>(x, packed, cb, out, T, M, K, C, bits, (int)blocks, st);
    default: return fewtok_launch_r<1, 1>(x, packed, cb, out, T, M, K, C, bits, (int)blocks, st);
    }
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

// 2 <= T <= 16 tokens (fp32, or bf16 x and out), K % 128 == 0, 16-byte
// aligned x and stream, widths 8, 10-14 and 16, C <= 16384: the bf16
// matrix-core kernel above; returns -1 for shapes it does not take.
int cbq_fixed_fewtok_t(const float *x, const uint8_t *packed, const float *cb, float *out, int T,
                       int M, int K, int C, int bits, hipStream_t st)
{
    return fewtok_launch<float, float>(x, packed, cb, out, T, M, K, C, bits, st);
}

int cbq_fixed_fewtok_t_bf16(const uint16_t *x, const uint8_t *packed, const float *cb,
                            uint16_t *out, int T, int M, int K, int C, int bits, hipStream_t st)
{
    return fewtok_launch<uint16_t, uint16_t>(x, packed, cb, out, T, M, K, C, bits, st);
}
