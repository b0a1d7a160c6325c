// Prefill GEMM over fixed-width codebook indices on bf16 MFMA (gfx950).
//
// out[t, m] = sum_k x[t, k] * codebook[min(idx[m*K + k], C-1)] with bf16 x,
// fp32 accumulation and bf16 out, for T >= 64 tokens (the GEMM regime of
// ck_linear_bf16, rocm/compressed_kernel.h:66-73).  Index layout is the
// reference's LSB-first stream (src/bitpack.py:32-95); K % 32 == 0, so each
// row's 32-index groups are BITS whole 32-bit words.
//
// Block = 8 waves, output tile 256 tokens x 128 features, K step 32.  Per K
// step the block (tiles double-buffered in LDS, one barrier per step)
//   - copies the x tile [256][32] bf16 to LDS,
//   - decodes the W tile [128][32]: 4 threads per row, 8 indices each,
//     gathering bf16 values from an LDS codebook padded to 2^BITS entries
//     (entries >= C repeat codebook[C-1], which is the reference's clamp),
//   - runs v_mfma_f32_32x32x16_bf16: each wave owns a 64 x 64 sub-tile
//     (2 x 2 MFMA blocks), A = x rows, B = W rows (both K-contiguous).
// A codebook that is not exactly bf16 (found while staging it) is split
// into bf16 hi + lo halves, each run through the MFMA.
// x and index words of the next four K steps are held in registers, so
// global latency hides behind the MFMAs.  LDS rows are 4 chunks of 16
// bytes stored at chunk ^ ((row >> 1) & 3): the ds_read_b128 of 8
// neighbouring rows then hit distinct bank groups.
#include "cbq_device.h"

#include <algorithm>

namespace {

constexpr int kPT = 256;          // tokens per block tile
constexpr int kPM = 128;          // features per block tile
constexpr int kPK = 32;           // K step (one index group)
constexpr int kPBlock = 512;      // 8 waves: 4 along T x 2 along M, 64 x 64 each

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 3); }

// 16-byte chunk `c` of tile row `r` (rows of 32 bf16 = 64 bytes).
__device__ __forceinline__ uint32_t *tile_chunk(uint32_t *tile, int r, int c)
{
    return tile + r * 16 + (swz(r, c) << 2);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Decode the 8 indices of part WP (indices 8*WP .. 8*WP+7 of a 32-index
// group) from the words loaded from word 8*WP*BITS/32 on, into 8 bf16 (and
// their lo halves when TWO).  All offsets are compile-time.
template <int BITS, int WP, bool TWO, int NW>
__device__ __forceinline__ void decode_part(const uint32_t (&wv)[NW], const uint16_t *s_cb,
                                            const uint16_t *s_cblo, uint32_t (&pk)[4],
                                            uint32_t (&pl)[4])
{
    constexpr uint32_t mask = (1u << BITS) - 1u;
    constexpr int sh0 = (WP * 8 * BITS) & 31;
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        uint32_t v[2], vl[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int o = sh0 + (j + h) * BITS;
            const int q = o >> 5, sh = o & 31;
            uint32_t f;
            if (sh + BITS <= 32) f = (wv[q] >> sh) & mask;
            else f = __builtin_amdgcn_alignbit(wv[q + 1], wv[q], (uint32_t)sh) & mask;
            v[h] = s_cb[f];
            if (TWO) vl[h] = s_cblo[f];
        }
        pk[j >> 1] = v[0] | (v[1] << 16);
        if (TWO) pl[j >> 1] = vl[0] | (vl[1] << 16);
    }
}

// Main K loop.  TWO: the codebook is not bf16-exact, so each weight is
// split as hi + lo (both bf16, lo = bf16(w - hi)) and both halves go through
// the MFMA, which keeps ~16 mantissa bits of the fp32 codebook.
template <int BITS, bool TWO, int WP>
__device__ __forceinline__ void prefill_loop(
    const uint16_t *__restrict__ xrow, const uint32_t *__restrict__ wrow, int G, int q0,
    int sh0, const uint16_t *s_cb, const uint16_t *s_cblo, uint32_t *s_x, uint32_t *s_w,
    uint32_t *s_wlo, int xr, int xc, int wr, int wp, int lane, int wt, int wmo, bool active,
    f32x16 (&acc)[2][2])
{
    constexpr int NW = (8 * BITS + 31 + 31) / 32;             // words covering 8 fields
    auto load_step = [&](int g, u32x4 (&xv)[2], uint32_t (&wv)[NW]) {
        const u32x4 *xs = (const u32x4 *)(xrow + (size_t)g * kPK);
        xv[0] = xs[0];
        xv[1] = xs[1];
        const uint32_t *ws = wrow + (size_t)g * BITS;
        // words past the group's last one are never used: clamp them in
#pragma unroll
        for (int i = 0; i < NW; i++) wv[i] = ws[q0 + i < BITS ? i : BITS - 1 - q0];
    };
    // Four K steps in flight: a register ring of x and index words.  The LDS
    // tiles are double-buffered: step g's MFMAs read buffer g & 1 while the
    // waves decode and write step g + 1 into the other buffer, so each step
    // needs one barrier, and the decode overlaps the matrix core.  The loop
    // is unrolled by the ring depth (even) so ring slots and buffers are
    // fixed registers and addresses; barriers wait on LDS only.
    constexpr int PD = 4;
    u32x4 xv[PD][2];
    uint32_t wv[PD][NW];
#pragma unroll
    for (int d = 0; d < PD; d++) load_step(d < G ? d : G - 1, xv[d], wv[d]);

    auto stage = [&](int d, int g, int buf) {
        const bool live = g < G;
        uint32_t *bx = s_x + buf * (kPT * 16);
        uint32_t *bw = s_w + buf * (kPM * 16);
        uint32_t *bl = s_wlo + buf * (kPM * 16);
        *(u32x4 *)tile_chunk(bx, xr, xc) = live ? xv[d][0] : u32x4{0, 0, 0, 0};
        *(u32x4 *)tile_chunk(bx, xr, xc + 1) = live ? xv[d][1] : u32x4{0, 0, 0, 0};
        uint32_t pk[4], pl[4];
        decode_part<BITS, WP, TWO>(wv[d], s_cb, s_cblo, pk, pl);
        *(u32x4 *)tile_chunk(bw, wr, wp) = u32x4{pk[0], pk[1], pk[2], pk[3]};
        if (TWO) *(u32x4 *)tile_chunk(bl, wr, wp) = u32x4{pl[0], pl[1], pl[2], pl[3]};
    };
    auto mfma_step = [&](int buf) {
        const uint32_t *bx = s_x + buf * (kPT * 16);
        const uint32_t *bw = s_w + buf * (kPM * 16);
        const uint32_t *bl = s_wlo + buf * (kPM * 16);
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {   // two k16 halves of the 32-wide step
            bf16x8 af[2], bfr[2], bfl[2];
            const int c = kk * 2 + (lane >> 5);        // 16-byte chunk of the row
#pragma unroll
            for (int a = 0; a < 2; a++) {
                const int r = wt + a * 32 + (lane & 31);
                const u32x4 v = *(const u32x4 *)tile_chunk((uint32_t *)bx, r, c);
                __builtin_memcpy(&af[a], &v, 16);
            }
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const int r = wmo + b * 32 + (lane & 31);
                const u32x4 v = *(const u32x4 *)tile_chunk((uint32_t *)bw, r, c);
                __builtin_memcpy(&bfr[b], &v, 16);
                if (TWO) {
                    const u32x4 vl = *(const u32x4 *)tile_chunk((uint32_t *)bl, r, c);
                    __builtin_memcpy(&bfl[b], &vl, 16);
                }
            }
#pragma unroll
            for (int a = 0; a < 2; a++)
#pragma unroll
                for (int b = 0; b < 2; b++) {
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bfr[b], acc[a][b],
                                                                         0, 0, 0);
                    if (TWO)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bfl[b],
                                                                             acc[a][b], 0, 0, 0);
                }
        }
    };

    stage(0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    load_step(PD < G ? PD : G - 1, xv[0], wv[0]);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    // Steps past G (G not a multiple of PD) run on zeroed x, adding nothing;
    // keeping them unconditional keeps the loop body branch-free.
    for (int g0 = 0; g0 < G; g0 += PD) {
#pragma unroll
        for (int d = 0; d < PD; d++) {
            const int g = g0 + d;
            const int dn = (d + 1) % PD;
            // waves whose 64 tokens all lie past T (a short batch) only stage
            if (active) mfma_step(d & 1);
            stage(dn, g + 1, (d + 1) & 1);
            // refill the staged slot (a clamped repeat past the end: never
            // written); the scheduling barriers keep the loads PD steps ahead
            __builtin_amdgcn_sched_barrier(0);
            load_step(g + 1 + PD < G ? g + 1 + PD : G - 1, xv[dn], wv[dn]);
            __builtin_amdgcn_sched_barrier(0);
            lds_barrier();
        }
    }
}

// SPLIT: block z sums only K groups [z * gs, z * gs + gs) and writes its fp32
// partial tile to ws + z * T * M; prefill_reduce_kernel adds the partials.
template <int BITS, bool SPLIT>
__global__ __launch_bounds__(kPBlock) void fixed_prefill_kernel(
    const uint16_t *__restrict__ x, const uint32_t *__restrict__ words,
    const float *__restrict__ cb, uint16_t *__restrict__ out, int T, int M, int K, int C,
    float *__restrict__ ws, int gs)
{
    __shared__ uint16_t s_cb[1 << BITS];                       // bf16 codebook (hi), padded
    __shared__ uint16_t s_cblo[1 << BITS];                     // bf16(cb - hi)
    __shared__ __attribute__((aligned(16))) uint32_t s_x[2 * kPT * 16];   // 2 x [256][32] bf16
    __shared__ __attribute__((aligned(16))) uint32_t s_w[2 * kPM * 16];   // 2 x [128][32] bf16
    __shared__ __attribute__((aligned(16))) uint32_t s_wlo[2 * kPM * 16];

    const int tid = threadIdx.x;
    const int lane = tid & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / CBQ_WAVE);
    const int t0 = blockIdx.x * kPT, m0 = blockIdx.y * kPM;
    const int G_all = K / kPK;
    const int g_lo = SPLIT ? (int)blockIdx.z * gs : 0;
    const int G = SPLIT ? min(G_all, g_lo + gs) - g_lo : G_all;

    // bf16 codebook, padded to 2^BITS (clamp semantics), split hi + lo
    int inexact = 0;
    for (int i = tid; i < (1 << BITS); i += kPBlock) {
        const float v = cb[i < C ? i : C - 1];
        const uint16_t hi = f32_to_bf16_rne(v);
        const uint16_t lo = f32_to_bf16_rne(v - __uint_as_float((uint32_t)hi << 16));
        s_cb[i] = hi;
        s_cblo[i] = lo;
        inexact |= (lo & 0x7fffu) != 0;
    }
    const bool two = __syncthreads_or(inexact);        // also publishes the codebook

    // x staging: thread -> tile row tid/2, chunks 2*(tid%2) and +1 (clamped row)
    const int xr = tid >> 1, xc = (tid & 1) * 2;
    const int xt = min(t0 + xr, T - 1);
    const uint16_t *xrow = x + (size_t)xt * K + (size_t)g_lo * kPK + xc * 8;
    // W decode: wave w takes part w % 4 (indices 8*part .. +7 of each group)
    // of tile rows 64*(w / 4) + lane, so the part is wave-uniform
    const int wr = ((wave >> 2) << 6) + lane, wp = wave & 3;
    const int wm = min(m0 + wr, M - 1);
    const int bit0 = wp * 8 * BITS;                            // within the 32-index group
    const int q0 = bit0 >> 5, sh0 = bit0 & 31;
    const uint32_t *wrow = words + ((size_t)wm * G_all + g_lo) * BITS + q0;

    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) acc[a][b] = f32x16{};
    const int wt = (wave >> 1) * 64;      // wave's token offset in the tile
    const int wmo = (wave & 1) * 64;      // wave's feature offset in the tile
    // one loop instance per (split, part): the loop body itself has no branch
    const bool active = t0 + wt < T;      // wave-uniform
#define CBQ_PREFILL_LOOP(TW, P)                                                                  \
    prefill_loop<BITS, TW, P>(xrow, wrow, G, q0, sh0, s_cb, s_cblo, s_x, s_w, s_wlo, xr, xc, wr, \
                              wp, lane, wt, wmo, active, acc)
    if (two) {
        switch (wp) {
        case 0: CBQ_PREFILL_LOOP(true, 0); break;
        case 1: CBQ_PREFILL_LOOP(true, 1); break;
        case 2: CBQ_PREFILL_LOOP(true, 2); break;
        default: CBQ_PREFILL_LOOP(true, 3); break;
        }
    } else {
        switch (wp) {
        case 0: CBQ_PREFILL_LOOP(false, 0); break;
        case 1: CBQ_PREFILL_LOOP(false, 1); break;
        case 2: CBQ_PREFILL_LOOP(false, 2); break;
        default: CBQ_PREFILL_LOOP(false, 3); break;
        }
    }
#undef CBQ_PREFILL_LOOP

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
                        out[(size_t)t * M + m] = f32_to_bf16_rne(acc[a][b][i * 4 + j]);
                }
        }
}

// out = bf16(sum over s of ws[s]), s in order.
__global__ void prefill_reduce_kernel(const float *__restrict__ ws, int S, int64_t n,
                                      uint16_t *__restrict__ out)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float t = ws[i];
        for (int s = 1; s < S; s++) t += ws[s * n + i];
        out[i] = f32_to_bf16_rne(t);
    }
}

template <int BITS>
int launch_prefill(const uint16_t *x, const uint8_t *packed, const float *cb, uint16_t *out,
                   int T, int M, int K, int C, int S, float *ws, hipStream_t st)
{
    const int G = K / kPK;
    if (S <= 1) {
        dim3 grid((unsigned)((T + kPT - 1) / kPT), (unsigned)((M + kPM - 1) / kPM));
        hipLaunchKernelGGL((fixed_prefill_kernel<BITS, false>), grid, dim3(kPBlock), 0, st, x,
                           (const uint32_t *)packed, cb, out, T, M, K, C, (float *)nullptr, G);
        return cbq_launch_status("fixed_prefill_kernel");
    }
    const int gs = (G + S - 1) / S;
    S = (G + gs - 1) / gs;                                   // no empty split
    dim3 grid((unsigned)((T + kPT - 1) / kPT), (unsigned)((M + kPM - 1) / kPM), (unsigned)S);
    hipLaunchKernelGGL((fixed_prefill_kernel<BITS, true>), grid, dim3(kPBlock), 0, st, x,
                       (const uint32_t *)packed, cb, out, T, M, K, C, ws, gs);
    int rc = cbq_launch_status("fixed_prefill_kernel");
    if (rc) return rc;
    const int64_t n = (int64_t)T * M;
    const int blocks = (int)std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(prefill_reduce_kernel, dim3(blocks), dim3(256), 0, st, ws, S, n, out);
    return cbq_launch_status("prefill_reduce_kernel");
}

}  // namespace

// K splits for a T x M x K prefill.  Only grids of fewer tiles than half the
// CUs split (past that the partials' extra traffic costs more than the idle
// CUs): into enough blocks to cover the CUs once, with at least 8 K groups
// (256 inputs) per split and at most 16 splits.
int cbq_prefill_splits(int T, int M, int K)
{
    if (T < 64 || K % kPK != 0) return 1;
    const int64_t tiles = (int64_t)((T + kPT - 1) / kPT) * ((M + kPM - 1) / kPM);
    const int64_t cus = cbq_num_cus();
    if (2 * tiles >= cus) return 1;
    int S = (int)std::min<int64_t>((cus + tiles - 1) / tiles, 16);
    S = std::min(S, (K / kPK) / 8);
    return S < 2 ? 1 : S;
}

// Prefill dispatch used by ck_linear_bf16 (cbq_fixed.hip).  Returns -1 when
// the shape is not handled here (the caller keeps its token-tile path).
// S > 1 needs ws of S * T * M floats.
int cbq_prefill_bf16(const uint16_t *x, const uint8_t *packed, const float *cb, uint16_t *out,
                     int T, int M, int K, int C, int bits, hipStream_t st, int S, float *ws)
{
    if (T < 64 || K % kPK != 0 || (((uintptr_t)packed | (uintptr_t)x) & 15) != 0 ||
        (K * 2) % 16 != 0 || (size_t)T > 65535ull * kPT || M > 65535 * kPM)
        return -1;
    if (S > 1 && !ws) return -1;
    switch (bits) {
    case 8: return launch_prefill<8>(x, packed, cb, out, T, M, K, C, S, ws, st);
    case 10: return launch_prefill<10>(x, packed, cb, out, T, M, K, C, S, ws, st);
    case 11: return launch_prefill<11>(x, packed, cb, out, T, M, K, C, S, ws, st);
    case 12: return launch_prefill<12>(x, packed, cb, out, T, M, K, C, S, ws, st);
    case 13: return launch_prefill<13>(x, packed, cb, out, T, M, K, C, S, ws, st);
    case 14: return launch_prefill<14>(x, packed, cb, out, T, M, K, C, S, ws, st);
    default: return -1;
    }
}
