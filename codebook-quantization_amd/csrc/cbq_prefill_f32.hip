// fp32-activation prefill GEMM over fixed-width codebook indices, on the fp32
// matrix cores of gfx950 (v_mfma_f32_32x32x2_f32).
//
// out[t, m] = sum_k x[t, k] * codebook[min(idx[m*K + k], C-1)] with fp32 x,
// the fp32 codebook and fp32 accumulation, for T >= 64 tokens: the batched
// case of ck_linear_f32 (rocm/compressed_kernel.h:52-64), where one K-tile of
// weights serves 256 tokens instead of being re-read per token tile.  Every
// product is exact in fp32; only the summation order differs from a GEMV.
// Index layout is the reference's LSB-first stream (src/bitpack.py:32-95);
// K % 32 == 0, so each row's 32-index groups are BITS whole 32-bit words.
//
// Block = 8 waves, output tile 256 tokens x 128 features, K step 32.  Per K
// step the block copies the x tile [256][32] and decodes the W tile
// [128][32] (4 threads per row, 8 indices each, gathered from an LDS fp32
// codebook padded to 2^BITS, which is the reference's clamp) into LDS; each
// wave then runs 2 x 2 x 16 MFMAs on its 64 x 64 sub-tile.  x and index
// words of the next two K steps are held in registers.  With split K (a
// caller workspace), block z sums only its share of the K steps and writes an
// fp32 partial tile; a second kernel adds the partials in order.
#include "cbq_device.h"

#include <algorithm>

namespace {

constexpr int kFT = 256;          // tokens per block tile
constexpr int kFM = 128;          // features per block tile
constexpr int kFK = 32;           // K step (one index group)
constexpr int kFBlock = 512;      // 8 waves: 4 along T x 2 along M, 64 x 64 each

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f4 __attribute__((ext_vector_type(4)));

// A tile row holds one K step's 32 values with k permuted to (k & 1) * 16 +
// (k >> 1): MFMA j of a step takes k = 2j + h in lane half h, so a lane's 16
// operands are 4 contiguous 16-byte chunks.  Chunk c of row r sits at chunk
// c ^ (r & 7): the 8 lanes of a ds_read_b128 pass (8 consecutive rows) hit
// distinct bank groups.
__device__ __forceinline__ float *frow_chunk(float *tile, int r, int c)
{
    return tile + r * kFK + ((c ^ (r & 7)) << 2);
}

// The 8 fp32 codebook values of indices 8*WP .. 8*WP+7 of a 32-index group,
// from the words loaded from word 8*WP*BITS/32 on.  All offsets compile-time.
template <int BITS, int WP, int NW>
__device__ __forceinline__ void decode_part_f32(const uint32_t (&wv)[NW], const float *s_cb,
                                                float (&v)[8])
{
    constexpr uint32_t mask = (1u << BITS) - 1u;
    constexpr int sh0 = (WP * 8 * BITS) & 31;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int o = sh0 + j * BITS;
        const int q = o >> 5, sh = o & 31;
        uint32_t f;
        if (sh + BITS <= 32) f = (wv[q] >> sh) & mask;
        else f = __builtin_amdgcn_alignbit(wv[q + 1], wv[q], (uint32_t)sh) & mask;
        v[j] = s_cb[f];
    }
}

template <int BITS, int WP>
__device__ __forceinline__ void prefill_f32_loop(
    const float *__restrict__ xrow, const uint32_t *__restrict__ wrow, int G, int q0,
    const float *s_cb, float *s_x, float *s_w, int xr, int hx, int wr, int lane, int wt, int wmo,
    bool active, f32x16 (&acc)[2][2])
{
    constexpr int NW = (8 * BITS + 31 + 31) / 32;             // words covering 8 fields
    auto load_step = [&](int g, f4 (&xv)[4], uint32_t (&wv)[NW]) {
        const f4 *xs = (const f4 *)(xrow + (size_t)g * kFK);
#pragma unroll
        for (int i = 0; i < 4; i++) xv[i] = xs[i];
        const uint32_t *ws = wrow + (size_t)g * BITS;
        // words past the group's last one are never used: clamp them in
#pragma unroll
        for (int i = 0; i < NW; i++) wv[i] = ws[q0 + i < BITS ? i : BITS - 1 - q0];
    };
    // Two K steps in flight (each step is ~4k cycles of matrix core per
    // wave, longer than a global load); the loop is unrolled by the ring
    // depth so ring slots are fixed registers.
    constexpr int PD = 2;
    f4 xv[PD][4];
    uint32_t wv[PD][NW];
#pragma unroll
    for (int d = 0; d < PD; d++) load_step(d < G ? d : G - 1, xv[d], wv[d]);

    // Steps past G (G odd) run on zeroed x, adding nothing.
    for (int g0 = 0; g0 < G; g0 += PD) {
#pragma unroll
        for (int d = 0; d < PD; d++) {
            const int g = g0 + d;
            const bool live = g < G;
            lds_barrier();                    // previous step's operands fully read
            {
                // x: this thread's 16 values k = 16 hx + i; evens go to chunks
                // 2 hx, 2 hx + 1, odds to chunks 4 + 2 hx, 5 + 2 hx
                const f4 z = {0.f, 0.f, 0.f, 0.f};
                const f4 a = live ? xv[d][0] : z, b = live ? xv[d][1] : z;
                const f4 c = live ? xv[d][2] : z, e = live ? xv[d][3] : z;
                *(f4 *)frow_chunk(s_x, xr, 2 * hx) = f4{a.x, a.z, b.x, b.z};
                *(f4 *)frow_chunk(s_x, xr, 2 * hx + 1) = f4{c.x, c.z, e.x, e.z};
                *(f4 *)frow_chunk(s_x, xr, 4 + 2 * hx) = f4{a.y, a.w, b.y, b.w};
                *(f4 *)frow_chunk(s_x, xr, 5 + 2 * hx) = f4{c.y, c.w, e.y, e.w};
                // W: indices k = 8 WP + i; evens to chunk WP, odds to chunk 4 + WP
                float v[8];
                decode_part_f32<BITS, WP>(wv[d], s_cb, v);
                *(f4 *)frow_chunk(s_w, wr, WP) = f4{v[0], v[2], v[4], v[6]};
                *(f4 *)frow_chunk(s_w, wr, 4 + WP) = f4{v[1], v[3], v[5], v[7]};
            }
            __builtin_amdgcn_sched_barrier(0);
            load_step(g + PD < G ? g + PD : G - 1, xv[d], wv[d]);
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();
            // waves whose 64 tokens all lie past T (a short batch) only stage
            if (!active) continue;

            const int h = lane >> 5;
            float af[2][16], bf[2][16];
#pragma unroll
            for (int a = 0; a < 2; a++) {
                const int r = wt + a * 32 + (lane & 31);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f4 t = *(const f4 *)frow_chunk(s_x, r, 4 * h + q);
                    af[a][4 * q] = t.x;
                    af[a][4 * q + 1] = t.y;
                    af[a][4 * q + 2] = t.z;
                    af[a][4 * q + 3] = t.w;
                }
            }
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const int r = wmo + b * 32 + (lane & 31);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f4 t = *(const f4 *)frow_chunk(s_w, r, 4 * h + q);
                    bf[b][4 * q] = t.x;
                    bf[b][4 * q + 1] = t.y;
                    bf[b][4 * q + 2] = t.z;
                    bf[b][4 * q + 3] = t.w;
                }
            }
#pragma unroll
            for (int j = 0; j < 16; j++)
#pragma unroll
                for (int a = 0; a < 2; a++)
#pragma unroll
                    for (int b = 0; b < 2; b++)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a][j], bf[b][j],
                                                                         acc[a][b], 0, 0, 0);
        }
    }
}

// SPLIT: block z sums only K groups [z * gs, z * gs + gs) and writes its fp32
// partial tile to ws + z * T * M; prefill_f32_reduce_kernel adds the partials.
template <int BITS, bool SPLIT>
__global__ __launch_bounds__(kFBlock) void fixed_prefill_f32_kernel(
    const float *__restrict__ x, const uint32_t *__restrict__ words,
    const float *__restrict__ cb, float *__restrict__ out, int T, int M, int K, int C,
    float *__restrict__ ws, int gs)
{
    __shared__ __attribute__((aligned(16))) float s_cb[1 << BITS];       // padded codebook
    __shared__ __attribute__((aligned(16))) float s_x[kFT * kFK];      // [256][32]
    __shared__ __attribute__((aligned(16))) float s_w[kFM * kFK];      // [128][32]

    const int tid = threadIdx.x;
    const int lane = tid & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / CBQ_WAVE);
    const int t0 = blockIdx.x * kFT, m0 = blockIdx.y * kFM;
    const int G_all = K / kFK;
    const int g_lo = SPLIT ? (int)blockIdx.z * gs : 0;
    const int G = SPLIT ? min(G_all, g_lo + gs) - g_lo : G_all;

    stage_clamped(s_cb, cb, C < (1 << BITS) ? C : (1 << BITS), 1 << BITS);
    // (the loop's first barrier publishes the codebook)

    // x staging: thread -> tile row tid/2, k half tid%2 (clamped row)
    const int xr = tid >> 1, hx = tid & 1;
    const int xt = min(t0 + xr, T - 1);
    const float *xrow = x + (size_t)xt * K + (size_t)g_lo * kFK + hx * 16;
    // W decode: wave w takes part w % 4 (indices 8*part .. +7 of each group)
    // of tile rows 64*(w / 4) + lane, so the part is wave-uniform
    const int wr = ((wave >> 2) << 6) + lane, wp = wave & 3;
    const int wm = min(m0 + wr, M - 1);
    const int q0 = (wp * 8 * BITS) >> 5;
    const uint32_t *wrow = words + ((size_t)wm * G_all + g_lo) * BITS + q0;

    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) acc[a][b] = f32x16{};
    const int wt = (wave >> 1) * 64;      // wave's token offset in the tile
    const int wmo = (wave & 1) * 64;      // wave's feature offset in the tile
    const bool active = t0 + wt < T;      // wave-uniform
#define CBQ_PF32_LOOP(P)                                                                          \
    prefill_f32_loop<BITS, P>(xrow, wrow, G, q0, s_cb, s_x, s_w, xr, hx, wr, lane, wt, wmo,      \
                              active, acc)
    switch (wp) {
    case 0: CBQ_PF32_LOOP(0); break;
    case 1: CBQ_PF32_LOOP(1); break;
    case 2: CBQ_PF32_LOOP(2); break;
    default: CBQ_PF32_LOOP(3); break;
    }
#undef CBQ_PF32_LOOP

    // acc[a][b][i*4+j] = C[tok = wt + a*32 + i*8 + (lane/32)*4 + j][feat = wmo + b*32 + lane%32]
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int m = m0 + wmo + b * 32 + (lane & 31);
            if (m >= M) continue;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int t = t0 + wt + a * 32 + i * 8 + (lane >> 5) * 4 + j;
                    if (t >= T) continue;
                    if (SPLIT)
                        ws[((size_t)blockIdx.z * T + t) * M + m] = acc[a][b][i * 4 + j];
                    else
                        out[(size_t)t * M + m] = acc[a][b][i * 4 + j];
                }
        }
}

// out = sum over s of ws[s], s in order.
__global__ void prefill_f32_reduce_kernel(const float *__restrict__ ws, int S, int64_t n,
                                          float *__restrict__ out)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float t = ws[i];
        for (int s = 1; s < S; s++) t += ws[s * n + i];
        out[i] = t;
    }
}

template <int BITS>
int launch_prefill_f32(const float *x, const uint8_t *packed, const float *cb, float *out, int T,
                       int M, int K, int C, int S, float *ws, hipStream_t st)
{
    const int G = K / kFK;
    if (S <= 1) {
        dim3 grid((unsigned)((T + kFT - 1) / kFT), (unsigned)((M + kFM - 1) / kFM));
        hipLaunchKernelGGL((fixed_prefill_f32_kernel<BITS, false>), grid, dim3(kFBlock), 0, st,
                           x, (const uint32_t *)packed, cb, out, T, M, K, C, (float *)nullptr, G);
        return cbq_launch_status("fixed_prefill_f32_kernel");
    }
    const int gs = (G + S - 1) / S;
    S = (G + gs - 1) / gs;                                   // no empty split
    dim3 grid((unsigned)((T + kFT - 1) / kFT), (unsigned)((M + kFM - 1) / kFM), (unsigned)S);
    hipLaunchKernelGGL((fixed_prefill_f32_kernel<BITS, true>), grid, dim3(kFBlock), 0, st, x,
                       (const uint32_t *)packed, cb, out, T, M, K, C, ws, gs);
    int rc = cbq_launch_status("fixed_prefill_f32_kernel");
    if (rc) return rc;
    const int64_t n = (int64_t)T * M;
    const int blocks = (int)std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(prefill_f32_reduce_kernel, dim3(blocks), dim3(256), 0, st, ws, S, n, out);
    return cbq_launch_status("prefill_f32_reduce_kernel");
}

}  // namespace

// K splits for a T x M x K fp32 prefill: the matrix cores are the bound here,
// so every grid under two blocks per CU splits, into enough blocks to cover
// the CUs twice, with at least 8 K groups per split and at most 16 splits.
int cbq_prefill_f32_splits(int T, int M, int K)
{
    if (T < 64 || K % kFK != 0) return 1;
    const int64_t tiles = (int64_t)((T + kFT - 1) / kFT) * ((M + kFM - 1) / kFM);
    const int64_t want = 2 * (int64_t)cbq_num_cus();
    if (tiles >= want) return 1;
    int S = (int)std::min<int64_t>((want + tiles - 1) / tiles, 16);
    S = std::min(S, (K / kFK) / 8);
    return S < 2 ? 1 : S;
}

// fp32 MFMA prefill used by ck_linear_f32; -1 = shape not handled here.  S > 1
// splits K, with S * T * M floats of workspace.
int cbq_prefill_f32(const float *x, const uint8_t *packed, const float *cb, float *out, int T,
                    int M, int K, int C, int bits, hipStream_t st, int S, float *ws)
{
    if (T < 64 || K % kFK != 0 || (((uintptr_t)packed | (uintptr_t)x) & 15) != 0 ||
        (size_t)T > 65535ull * kFT || M > 65535 * kFM)
        return -1;
    if (S > 1 && !ws) return -1;
    switch (bits) {
    case 8: return launch_prefill_f32<8>(x, packed, cb, out, T, M, K, C, S, ws, st);
    case 10: return launch_prefill_f32<10>(x, packed, cb, out, T, M, K, C, S, ws, st);
    case 11: return launch_prefill_f32<11>(x, packed, cb, out, T, M, K, C, S, ws, st);
    case 12: return launch_prefill_f32<12>(x, packed, cb, out, T, M, K, C, S, ws, st);
    case 13: return launch_prefill_f32<13>(x, packed, cb, out, T, M, K, C, S, ws, st);
    default: return -1;
    }
}
