// Prefill GEMM over fixed-width codebook indices on bf16 MFMA (gfx950).
//
// out[t, m] = sum_k x[t, k] * codebook[min(idx[m*K + k], C-1)] with bf16 x,
// fp32 accumulation and bf16 out, for T >= 64 tokens (the GEMM regime of
// ck_linear_bf16, rocm/compressed_kernel.h:66-73).  Index layout is the
// reference's LSB-first stream (src/bitpack.py:32-95); K % 32 == 0, so each
// row's 32-index groups are BITS whole 32-bit words.
//
// Block = 8 waves (two per SIMD), output tile 512 tokens x 128 features, K
// step 32 (one index group per row).  Wave w owns tokens 64 w .. 64 w + 63
// and all 128 features: 4 x 8 blocks of v_mfma_f32_16x16x32_bf16, 32 MFMAs a
// step.
//   - x does not pass through LDS.  The A operand of a 16-token block is lane
//     l's 8 bf16 at row l % 16, k 8 (l / 16) .. +7.  With a caller workspace
//     (cbq_linear_bf16_ws) x is first copied to that fragment order
//     (prefill_x_frag_kernel), so every operand load is 1 KiB contiguous;
//     without one (ck_linear_bf16) each lane reads its own row, which the L2
//     serves at about a third of the rate.
//   - The W tile's index words (128 rows x BITS words per step) are loaded by
//     dword loads, consecutive lanes on consecutive words of a row, three
//     steps ahead into registers, then stored to a double-buffered LDS slot.
//   - Each step the 512 threads decode the W tile of step + 2 once for the
//     block: thread -> (row, 8 indices), bf16 values gathered from an LDS
//     codebook padded to 2^BITS entries (entries >= C repeat codebook[C-1],
//     which is the reference's clamp), into a triple-buffered bf16 tile whose
//     fragments the MFMAs read as their B operand.  One barrier per step.
// A weight is decoded once per 512 tokens: the random codebook gathers
// (about 8 per clock per CU on gfx950) stay below the matrix core's time.
// A codebook that is not exactly bf16 (found while staging it) is split into
// bf16 hi + lo halves, each run through the MFMA.  The output leaves through
// LDS: each wave transposes 16 tokens at a time into a padded row-major tile
// and stores whole rows, 16 bytes a lane.
#include "cbq_device.h"

#include <algorithm>

namespace {

constexpr int kPT = 512;               // tokens per block tile
constexpr int kPM = 128;               // features per block tile
constexpr int kPK = 32;                // K step (one index group)
constexpr int kPWaves = 8;            // two per SIMD: one hides the other's waits
constexpr int kPBlock = kPWaves * CBQ_WAVE;
constexpr int kWT = kPT / kPWaves;     // tokens per wave (64)
constexpr int kTB = kWT / 16;          // 16-token MFMA blocks per wave
constexpr int kNB = kPM / 16;          // 16-feature MFMA blocks
constexpr int kXD = 2;                 // x register ring (steps)
constexpr int kRD = 3;                 // index-word register ring (steps)
constexpr int kUnroll = 6;             // K loop unroll: every ring index compile-time
constexpr int kWBuf = kPM * 4;         // 16-byte chunks per W tile buffer
// Index words of one step: kPM rows x BITS words, moved by kRawLoads dword
// loads per thread (load j of thread t: slot dword j * 512 + t = word s % BITS
// of tile row s / BITS; dwords past kPM * BITS are loaded and stored but
// never read).
template <int BITS> constexpr int kRawLoads = (kPM * BITS + kPBlock - 1) / kPBlock;
template <int BITS> constexpr int kRawSlot = kRawLoads<BITS> * kPBlock;
// The W tiles (hi and lo, three buffers each) share one LDS array with the
// epilogue, which reuses it after the K loop: per wave kEpiRows rows of kPM
// fp32 or bf16 outputs, rows padded by 16 bytes.
template <bool SPLIT> constexpr int kEpiRow = kPM * (SPLIT ? 4 : 2) + 16;
constexpr int kEpiRows = 16;
constexpr int kLdsEpi = kPWaves * kEpiRows * kEpiRow<true>;
constexpr int kWtChunks = (6 * kWBuf * 16 > kLdsEpi ? 6 * kWBuf * 16 : kLdsEpi) / 16;

// Diagnostic build (-DCBQ_TIMELINE): wave w of block b (grid index
// z * gridDim.x + b) records the 100 MHz s_memrealtime clock at entry, after
// the codebook staging, after the loop's prologue (ring filled, first two
// W tiles decoded), after the K loop and at exit, plus its K steps, into
// cbq_pf_timeline (read by cbq_prefill_timeline_read).  The product build
// has none of it.
constexpr int kPfTimelineWaves = 4096;
constexpr int kPfTimelineFields = 6;
#ifdef CBQ_TIMELINE
__device__ unsigned long long cbq_pf_timeline[kPfTimelineWaves * kPfTimelineFields];
#endif

// Word 3 of a raw buffer resource on gfx9 (32-bit data format; no swizzle,
// no stride): loads past num_records bytes return 0.
constexpr int kBufRsrcWord3 = 0x00020000;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// W tile row r (32 bf16) is four 16-byte chunks; chunk c sits at 16-byte
// slot r * 4 + (c ^ ((r >> 2) & 3)).  The 16 lanes of a B-fragment read that
// share a chunk take 16 consecutive rows and so 16 distinct bank groups; so
// do 16 consecutive decode threads writing one chunk.
__device__ __forceinline__ int wslot(int r, int c) { return (r << 2) + (c ^ ((r >> 2) & 3)); }

// fp32 -> bf16 bits by the hardware conversion (v_cvt_pk_bf16_f32: round to
// nearest even), for outputs.
__device__ __forceinline__ uint16_t bf16_out(float f)
{
    const __bf16 h = (__bf16)f;
    uint16_t u;
    __builtin_memcpy(&u, &h, 2);
    return u;
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// lo | hi << 16 of two 16-bit values (one v_perm; built as a two-element
// vector, so no mask of the loaded halves is emitted first).
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(uint32_t lo, uint32_t hi)
{
    u16x2 p;
    p.x = (unsigned short)lo;
    p.y = (unsigned short)hi;
    return __builtin_bit_cast(uint32_t, p);
}

// Main K loop of one wave; HP = which part (of kPWaves / 2) of each
// 32-index group this thread decodes (wave-uniform).  Steps past G clamp their loads to the last
// group and skip their MFMAs.
//
// Per step g (one barrier), in issue order:
//   - the words of step g + 3 (in registers since step g - 3) go to LDS
//     slot (g + 1) & 1, whose words (step g + 1) were decoded during step
//     g - 1, and the words of step g + 6 are loaded in their place;
//   - the 32 MFMAs of step g run on B fragments already in registers; after
//     the last MFMA of each 16-feature block its fragment of step g + 1 is
//     read from W buffer (g + 1) % 3 (decoded during step g - 1);
//   - between the MFMA blocks the threads decode step g + 2 (slot g & 1)
//     into W buffer (g + 2) % 3, whose fragments were read during step g - 2:
//     index words, then the codebook gathers, then the tile store;
//   - x of step g + 2 is loaded.
// So the MFMAs wait on no LDS read of their own step: the fragment reads,
// gathers and stores run while the matrix core works.
template <int BITS, bool TWO, int HP, bool XF>
__device__ __forceinline__ void prefill_loop(
    __amdgpu_buffer_rsrc_t xb, const uint32_t (&xoff)[kTB], __amdgpu_buffer_rsrc_t wb,
    const uint32_t (&doff)[kRawLoads<BITS>], int G, const uint16_t *s_cb, const uint16_t *s_cblo,
    u32x4 *s_w, u32x4 *s_wlo, uint32_t *s_raw, int wave, int lane, bool active,
    f32x4 (&acc)[kTB][kNB], unsigned long long &ts_pro)
{
    constexpr int NF = 64 / kPWaves;                     // indices a thread decodes
    constexpr int NW = (NF * BITS + 31 + 31) / 32;       // words covering them
    constexpr int q0 = (HP * NF * BITS) >> 5;
    constexpr int sh0 = (HP * NF * BITS) & 31;
    constexpr uint32_t mask = (1u << BITS) - 1u;
    constexpr int ND = kRawLoads<BITS>;
    constexpr int kSlot = kRawSlot<BITS>;
    const int tid = wave * CBQ_WAVE + lane;
    const int wr = ((wave / (kPWaves / 2)) << 6) + lane;  // decoded tile row
    const int fo = wslot(lane & 15, lane >> 4);          // this lane's B-fragment chunk
    // (row nb * 16 + lane % 16 has slot fo + nb * 64: (r >> 2) & 3 is unchanged by + 16)

    auto load_raw = [&](int g, uint32_t (&rr)[ND]) {     // step g's index words
        const int gc = g < G ? g : G - 1;
#pragma unroll
        for (int j = 0; j < ND; j++)
            rr[j] = __builtin_amdgcn_raw_buffer_load_b32(wb, (int)(doff[j] * 4u), gc * BITS * 4, 0);
    };
    auto store_raw = [&](int slot_i, const uint32_t (&rr)[ND]) {
        uint32_t *slot = s_raw + slot_i * kSlot + tid;
#pragma unroll
        for (int j = 0; j < ND; j++) slot[j * kPBlock] = rr[j];
    };
    auto load_x = [&](int g, bf16x8 (&xr)[kTB]) {
        const int gc = g < G ? g : G - 1;
#pragma unroll
        for (int tb = 0; tb < kTB; tb++)
            xr[tb] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                                    xb, (int)(xoff[tb] * 2u), gc * (XF ? 1024 : 2 * kPK), 0));
    };
    auto read_words = [&](int slot_i, uint32_t (&wv)[NW]) {
        const uint32_t *rw = s_raw + slot_i * kSlot + wr * BITS;
#pragma unroll
        for (int i = 0; i < NW; i++) wv[i] = rw[q0 + i < BITS ? q0 + i : BITS - 1];
    };
    // Each index is extracted already doubled (the byte offset of its bf16
    // entry): shift by one bit less, mask with mask << 1.  The tables sit at
    // the bottom of LDS, so the offset goes to ds_read_u16 as it is.
    auto gather = [&](const uint32_t (&wv)[NW], uint32_t (&v)[NF], uint32_t (&vl)[NF]) {
        constexpr uint32_t mask2 = mask << 1;
#pragma unroll
        for (int j = 0; j < NF; j++) {
            const int o = sh0 + j * BITS;
            const int q = o >> 5, sh = o & 31;
            uint32_t f2;
            if (sh == 0) f2 = (wv[q] << 1) & mask2;
            else if (sh + BITS <= 32) f2 = (wv[q] >> (sh - 1)) & mask2;
            else f2 = __builtin_amdgcn_alignbit(wv[q + 1], wv[q], (uint32_t)(sh - 1)) & mask2;
            v[j] = *(const uint16_t *)((const char *)s_cb + f2);
            if (TWO) vl[j] = *(const uint16_t *)((const char *)s_cblo + f2);
        }
    };
    auto store_w = [&](int buf, const uint32_t (&v)[NF], const uint32_t (&vl)[NF]) {
#pragma unroll
        for (int h = 0; h < NF / 8; h++) {
            const int o = buf * kWBuf + wslot(wr, (NF / 8) * HP + h);
            const int e = 8 * h;
            s_w[o] = u32x4{pack_bf16x2(v[e], v[e + 1]), pack_bf16x2(v[e + 2], v[e + 3]),
                           pack_bf16x2(v[e + 4], v[e + 5]), pack_bf16x2(v[e + 6], v[e + 7])};
            if (TWO)
                s_wlo[o] = u32x4{pack_bf16x2(vl[e], vl[e + 1]), pack_bf16x2(vl[e + 2], vl[e + 3]),
                                 pack_bf16x2(vl[e + 4], vl[e + 5]), pack_bf16x2(vl[e + 6], vl[e + 7])};
        }
    };
    auto read_frag = [&](int buf, int nb, bf16x8 &b, bf16x8 &bl) {
        const u32x4 v = s_w[buf * kWBuf + fo + nb * 64];
        __builtin_memcpy(&b, &v, 16);
        if (TWO) {
            const u32x4 vl = s_wlo[buf * kWBuf + fo + nb * 64];
            __builtin_memcpy(&bl, &vl, 16);
        }
    };
    // MFMAs of feature blocks [n0, n1) of step g.  bf16 codebook: each block
    // is followed by the read of its fragment for step g + 1 (buffer nbuf)
    // into the same registers.  hi + lo codebook (twice the fragments): the
    // step's own fragments are read from buffer cbuf just before their MFMAs.
    auto mfma_blocks = [&](int n0, int n1, bool on, const bf16x8 (&xr)[kTB], bf16x8 (&bf)[kNB],
                           int cbuf, int nbuf) {
#pragma unroll
        for (int nb = n0; nb < n1; nb++) {
            bf16x8 b = bf[nb], bl;
            if (TWO) read_frag(cbuf, nb, b, bl);
            if (on) {
#pragma unroll
                for (int tb = 0; tb < kTB; tb++) {
                    acc[tb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xr[tb], b, acc[tb][nb],
                                                                          0, 0, 0);
                    if (TWO)
                        acc[tb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xr[tb], bl,
                                                                              acc[tb][nb], 0, 0, 0);
                }
            }
            if (!TWO) read_frag(nbuf, nb, bf[nb], bl);
        }
    };

    bf16x8 xr[kXD][kTB];
    uint32_t rr[kRD][ND];
    bf16x8 bf[kNB];
    {
        uint32_t r0[ND], r1[ND], r2[ND];
        load_raw(0, r0);
        load_raw(1, r1);
        load_raw(2, r2);
#pragma unroll
        for (int d = 0; d < kRD; d++) load_raw(d + 3, rr[d]);
#pragma unroll
        for (int d = 0; d < kXD; d++) load_x(d, xr[d]);
        store_raw(0, r0);
        store_raw(1, r1);
        lds_barrier();
        uint32_t wv[NW], v[NF], vl[NF];
        read_words(0, wv);
        gather(wv, v, vl);
        store_w(0, v, vl);
        lds_barrier();                                   // slot 0 free again
        store_raw(0, r2);
        read_words(1, wv);
        gather(wv, v, vl);
        store_w(1, v, vl);
        lds_barrier();
        if (!TWO) {
            bf16x8 bl;
#pragma unroll
            for (int nb = 0; nb < kNB; nb++) read_frag(0, nb, bf[nb], bl);
        }
    }
#ifdef CBQ_TIMELINE
    ts_pro = __builtin_amdgcn_s_memrealtime();
#else
    (void)ts_pro;
#endif
    for (int g0 = 0; g0 < G; g0 += kUnroll) {
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int g = g0 + u;                        // g % kUnroll == u
            const bool on = active && g < G;
            store_raw((u + 1) & 1, rr[u % kRD]);         // words of step g + 3
            load_raw(g + 3 + kRD, rr[u % kRD]);
            uint32_t wv[NW], v[NF], vl[NF];
            __builtin_amdgcn_sched_barrier(0);
            mfma_blocks(0, 2, on, xr[u % kXD], bf, u % 3, (u + 1) % 3);
            __builtin_amdgcn_sched_barrier(0);
            read_words(u & 1, wv);                       // step g + 2's words
            __builtin_amdgcn_sched_barrier(0);
            mfma_blocks(2, 4, on, xr[u % kXD], bf, u % 3, (u + 1) % 3);
            __builtin_amdgcn_sched_barrier(0);
            gather(wv, v, vl);
            __builtin_amdgcn_sched_barrier(0);
            mfma_blocks(4, 6, on, xr[u % kXD], bf, u % 3, (u + 1) % 3);
            __builtin_amdgcn_sched_barrier(0);
            store_w((u + 2) % 3, v, vl);
            __builtin_amdgcn_sched_barrier(0);
            mfma_blocks(6, kNB, on, xr[u % kXD], bf, u % 3, (u + 1) % 3);
            __builtin_amdgcn_sched_barrier(0);
            load_x(g + kXD, xr[u % kXD]);
            lds_barrier();
        }
    }
}

// Block b takes tile tix = tile0 + b: token tile tix % nT of feature tile
// tix / nT.  SPLIT: block (b, z) sums only K groups [z * gs, z * gs + gs) and
// writes its fp32 partial tile, row-major [512][128], to partial tile
// z * gridDim.x + b of ws; prefill_reduce_tiles_kernel adds the partials.
template <int BITS, bool SPLIT, bool XF>
__global__ __launch_bounds__(kPBlock) void fixed_prefill_kernel(
    const uint16_t *__restrict__ x, const uint32_t *__restrict__ words,
    const float *__restrict__ cb, uint16_t *__restrict__ out, int T, int M, int K, int C,
    float *__restrict__ ws, int gs, int nT, int tile0)
{
    // bf16 codebook (hi), padded, and bf16(cb - hi).  The 64-byte alignment
    // places them first in LDS (the allocator orders by alignment), below
    // the 64 KiB that a ds_read offset field reaches.
    __shared__ __attribute__((aligned(64))) uint16_t s_cb[1 << BITS];
    __shared__ __attribute__((aligned(64))) uint16_t s_cblo[1 << BITS];
    __shared__ __attribute__((aligned(16))) u32x4 s_wt[kWtChunks];   // W tiles, then the epilogue's
    __shared__ uint32_t s_raw[2 * kRawSlot<BITS>];
    u32x4 *s_w = s_wt;                                         // 3 x [128][32] bf16
    u32x4 *s_wlo = s_wt + 3 * kWBuf;

    const int tid = threadIdx.x;
    const int lane = tid & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / CBQ_WAVE);
    unsigned long long ts_pro = 0;
#ifdef CBQ_TIMELINE
    const unsigned long long ts_entry = __builtin_amdgcn_s_memrealtime();
#endif
    const int tix = tile0 + (int)blockIdx.x;
    const int t0 = (tix % nT) * kPT;
    const int m0 = (tix / nT) * kPM;
    const int G_all = K / kPK;
    const int g_lo = SPLIT ? (int)blockIdx.z * gs : 0;
    const int G = SPLIT ? min(G_all, g_lo + gs) - g_lo : G_all;

    // bf16 codebook, padded to 2^BITS (clamp semantics), split hi + lo; every
    // load of a thread is issued before the first is used (one latency, not
    // one per entry)
    int inexact = 0;
    {
        constexpr int NE = ((1 << BITS) + kPBlock - 1) / kPBlock;
        float v[NE];
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const int i = e * kPBlock + tid;
            v[e] = cb[i < C ? i : C - 1];
        }
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const int i = e * kPBlock + tid;
            if (i >= (1 << BITS)) break;
            const uint16_t hi = f32_to_bf16_rne(v[e]);
            const uint16_t lo = f32_to_bf16_rne(v[e] - __uint_as_float((uint32_t)hi << 16));
            s_cb[i] = hi;
            s_cblo[i] = lo;
            inexact |= (lo & 0x7fffu) != 0;
        }
    }
    const bool two = __syncthreads_or(inexact);        // also publishes the codebook
#ifdef CBQ_TIMELINE
    const unsigned long long ts_staged = __builtin_amdgcn_s_memrealtime();
#endif

    // x fragments: token block tb, lane -> row lane % 16, k chunk lane / 16.
    // XF: x is in fragment order (prefill_x_frag_kernel), the wave's 1 KiB
    // fragment of each step is contiguous; else row-major with rows clamped.
    uint32_t xoff[kTB];
#pragma unroll
    for (int tb = 0; tb < kTB; tb++) {
        if (XF) {
            const int b = min(t0 + wave * kWT + tb * 16, ((T + 15) & ~15) - 16) >> 4;
            xoff[tb] = ((uint32_t)b * (uint32_t)G_all + (uint32_t)g_lo) * 512u + (uint32_t)lane * 8u;
        } else {
            xoff[tb] = (uint32_t)min(t0 + wave * kWT + tb * 16 + (lane & 15), T - 1) * (uint32_t)K +
                       (uint32_t)(g_lo * kPK + (lane >> 4) * 8);
        }
    }
    // index words: load j of thread tid is dword s = j * 512 + tid of the
    // step's slot = word s % BITS of tile row s / BITS (rows clamped)
    const uint32_t RW = (uint32_t)G_all * BITS;
    uint32_t doff[kRawLoads<BITS>];
#pragma unroll
    for (int j = 0; j < kRawLoads<BITS>; j++) {
        const int s = j * kPBlock + tid;
        const int row = s / BITS, w = s - row * BITS;
        doff[j] = (uint32_t)min(m0 + row, M - 1) * RW + (uint32_t)(g_lo * BITS + w);
    }

    // global operands as buffer resources: a load's per-step advance is a
    // scalar offset, so the K loop spends no VALU on addresses
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)x, (short)0, (int)(XF ? (uint32_t)((T + 15) & ~15) * (uint32_t)K * 2u
                                       : (uint32_t)T * (uint32_t)K * 2u), kBufRsrcWord3);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)words, (short)0, (int)((uint32_t)M * RW * 4u), kBufRsrcWord3);

    f32x4 acc[kTB][kNB];
#pragma unroll
    for (int a = 0; a < kTB; a++)
#pragma unroll
        for (int b = 0; b < kNB; b++) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    // waves whose 64 tokens all lie past T decode their share but skip the MFMAs
    const bool active = t0 + wave * kWT < T;
#define CBQ_PREFILL_LOOP(TW, H)                                                                 \
    prefill_loop<BITS, TW, H, XF>(xrs, xoff, wrs, doff, G, s_cb, s_cblo, s_w, s_wlo, s_raw, wave, \
                                  lane, active, acc, ts_pro)
    static_assert(kPWaves == 8, "the part switch below has kPWaves / 2 cases");
    if (two) {
        switch (wave & 3) {
        case 0: CBQ_PREFILL_LOOP(true, 0); break;
        case 1: CBQ_PREFILL_LOOP(true, 1); break;
        case 2: CBQ_PREFILL_LOOP(true, 2); break;
        default: CBQ_PREFILL_LOOP(true, 3); break;
        }
    } else {
        switch (wave & 3) {
        case 0: CBQ_PREFILL_LOOP(false, 0); break;
        case 1: CBQ_PREFILL_LOOP(false, 1); break;
        case 2: CBQ_PREFILL_LOOP(false, 2); break;
        default: CBQ_PREFILL_LOOP(false, 3); break;
        }
    }
#undef CBQ_PREFILL_LOOP
#ifdef CBQ_TIMELINE
    const unsigned long long ts_loop = __builtin_amdgcn_s_memrealtime();
#endif

    // acc[tb][nb][r] = out[token t0 + 64 wave + 16 tb + 4 (lane / 16) + r]
    //                     [feature m0 + 16 nb + lane % 16]
    // Through LDS, kEpiRows tokens per pass: each wave writes its values into
    // a padded row-major tile of its own and stores whole rows.
    lds_barrier();                                    // every wave is done with the LDS above
    constexpr int ES = SPLIT ? 4 : 2;                 // bytes per output value
    constexpr int RS = kEpiRow<SPLIT>;
    constexpr int LPR = kPM * ES / 16;                // lanes per row (16 bytes each)
    constexpr int HB = kEpiRows / 16;                 // token blocks per pass
    uint8_t *tile = (uint8_t *)s_wt + wave * kEpiRows * RS;
#pragma unroll
    for (int p = 0; p < kTB / HB; p++) {
#pragma unroll
        for (int h = 0; h < HB; h++)
#pragma unroll
            for (int nb = 0; nb < kNB; nb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = h * 16 + (lane >> 4) * 4 + r, col = nb * 16 + (lane & 15);
                    if (SPLIT)
                        *(float *)(tile + row * RS + col * 4) = acc[HB * p + h][nb][r];
                    else
                        *(uint16_t *)(tile + row * RS + col * 2) = bf16_out(acc[HB * p + h][nb][r]);
                }
#pragma unroll
        for (int i = 0; i < kEpiRows * LPR / CBQ_WAVE; i++) {
            const int row = i * (CBQ_WAVE / LPR) + lane / LPR, c = lane % LPR;
            const u32x4 v = *(const u32x4 *)(tile + row * RS + c * 16);
            const int t = t0 + wave * kWT + p * kEpiRows + row;
            const int m = m0 + c * (16 / ES);
            if (t >= T || m >= M) continue;
            uint8_t *dst = SPLIT ? (uint8_t *)(ws + (((size_t)blockIdx.z * gridDim.x + blockIdx.x) *
                                                         kPT + (t - t0)) * kPM + (m - m0))
                                 : (uint8_t *)(out + (size_t)t * M + m);
            if (m + 16 / ES <= M && ((uintptr_t)dst & 15) == 0) {
                *(u32x4 *)dst = v;
            } else {
                const uint8_t *src = (const uint8_t *)&v;
                for (int e = 0; e < 16 / ES && m + e < M; e++)
                    __builtin_memcpy(dst + e * ES, src + e * ES, ES);
            }
        }
    }
#ifdef CBQ_TIMELINE
    const unsigned long long ts_exit = __builtin_amdgcn_s_memrealtime();
    const int twid = ((int)(blockIdx.z * gridDim.x + blockIdx.x)) * kPWaves + wave;
    if (lane == 0 && twid < kPfTimelineWaves) {
        unsigned long long *tl = cbq_pf_timeline + (size_t)twid * kPfTimelineFields;
        tl[0] = ts_entry;
        tl[1] = ts_staged;
        tl[2] = ts_pro;
        tl[3] = ts_loop;
        tl[4] = ts_exit;
        tl[5] = (unsigned long long)G;
    }
#endif
}

// x [T][K] bf16 row-major -> fragment order: piece i (16 bytes) of chunk
// c = b * (K / 32) + g holds x[16 b + i % 16][32 g + 8 (i / 16) .. +7], i.e.
// lane i's MFMA A operand for token block b at K step g; rows >= T are 0.
// Block (b, s) moves token block b over K steps [8 s, 8 s + 8): row-contiguous
// reads into a padded LDS tile, then fragment-order reads and contiguous
// writes (both global sides coalesced).
constexpr int kXfSteps = 8;
constexpr int kXfRow = kXfSteps * kPK * 2 + 16;        // LDS bytes per token row (padded)
__global__ __launch_bounds__(256) void prefill_x_frag_kernel(const uint16_t *__restrict__ x,
                                                             uint16_t *__restrict__ xf, int T,
                                                             int K)
{
    __shared__ __attribute__((aligned(16))) uint8_t tile[16 * kXfRow];
    const int G = K / kPK;
    const int b = blockIdx.x, g0 = blockIdx.y * kXfSteps;
    const int ns = min(kXfSteps, G - g0);                // K steps in this block
    constexpr int kRowPieces = kXfSteps * 4;            // 16-byte pieces per row
    for (int i = threadIdx.x; i < 16 * kRowPieces; i += blockDim.x) {
        const int r = i / kRowPieces, c = i % kRowPieces;
        const int t = b * 16 + r;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (t < T && c < ns * 4) v = *(const u32x4 *)(x + (size_t)t * K + (size_t)g0 * kPK + c * 8);
        *(u32x4 *)(tile + r * kXfRow + c * 16) = v;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < ns * CBQ_WAVE; i += blockDim.x) {
        const int gl = i / CBQ_WAVE, l = i % CBQ_WAVE;
        const u32x4 v = *(const u32x4 *)(tile + (l & 15) * kXfRow + (gl * 4 + (l >> 4)) * 16);
        *(u32x4 *)(xf + (((size_t)b * G + g0 + gl) * CBQ_WAVE + l) * 8) = v;
    }
}

// Output tiles tile0 .. tile0 + ntile - 1 = bf16 of the sum of their S
// partial tiles (ws partial tile z * ntile + i, row-major [512][128]), added
// in split order; entries past T or M are skipped.  Four columns a thread.
__global__ void prefill_reduce_tiles_kernel(const float *__restrict__ ws, int S, int ntile,
                                            int tile0, int nT, int T, int M,
                                            uint16_t *__restrict__ out)
{
    constexpr int64_t kTile = (int64_t)kPT * kPM;
    const int64_t n4 = (int64_t)ntile * kTile / 4;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
        const int64_t e = i * 4;
        const int tl = (int)(e / kTile);
        const int r = (int)(e % kTile) / kPM, c = (int)(e % kPM);
        const int tix = tile0 + tl;
        const int t = (tix % nT) * kPT + r, m = (tix / nT) * kPM + c;
        if (t >= T || m >= M) continue;
        const float *p = ws + (int64_t)tl * kTile + r * kPM + c;
        f32x4 a = *(const f32x4 *)p;
        for (int z = 1; z < S; z++) {
            const f32x4 v = *(const f32x4 *)(p + (int64_t)z * ntile * kTile);
            a[0] += v[0];
            a[1] += v[1];
            a[2] += v[2];
            a[3] += v[3];
        }
        uint16_t *o = out + (size_t)t * M + m;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (m + k < M) o[k] = bf16_out(a[k]);
    }
}

// How a T x M x K prefill is launched: tiles [0, full) run whole, tiles
// [full, tiles) split K S ways (S = 1: none).  One 512-thread block per CU.
// A grid of at most half the CUs splits every tile floor(CUs / tiles) ways;
// tiles that leave at most half of a last round of the CUs split
// floor(CUs / leftover) ways, so that round is as short as the others' share
// of K.  At most 16 splits, each of at least 8 K groups.
struct PrefillPlan {
    int nT, tiles, full, S;
};

PrefillPlan prefill_plan(int T, int M, int K)
{
    PrefillPlan p;
    p.nT = (T + kPT - 1) / kPT;
    p.tiles = p.nT * ((M + kPM - 1) / kPM);
    p.full = p.tiles;
    p.S = 1;
    const int cus = cbq_num_cus();
    const int max_s = std::min(16, (K / kPK) / 8);
    const int r = p.tiles % cus;
    int left = 0;
    if (2 * p.tiles <= cus) left = p.tiles;
    else if (p.tiles > cus && r > 0 && 2 * r <= cus) left = r;
    if (left > 0) {
        const int S = std::min(cus / left, max_s);
        if (S >= 2) {
            p.full = p.tiles - left;
            p.S = S;
        }
    }
    return p;
}

size_t prefill_partial_bytes(const PrefillPlan &p)
{
    return p.S > 1 ? (size_t)(p.tiles - p.full) * p.S * kPT * kPM * sizeof(float) : 0;
}

template <int BITS, bool XF>
int launch_prefill_x(const uint16_t *x, const uint8_t *packed, const float *cb, uint16_t *out,
                     int T, int M, int K, int C, const PrefillPlan &p, float *ws, hipStream_t st)
{
    const int G = K / kPK;
    if (p.full > 0) {
        hipLaunchKernelGGL((fixed_prefill_kernel<BITS, false, XF>), dim3((unsigned)p.full),
                           dim3(kPBlock), 0, st, x, (const uint32_t *)packed, cb, out, T, M, K, C,
                           (float *)nullptr, G, p.nT, 0);
        const int rc = cbq_launch_status("fixed_prefill_kernel");
        if (rc) return rc;
    }
    if (p.full == p.tiles) return CK_SUCCESS;
    const int n = p.tiles - p.full;
    const int gs = (G + p.S - 1) / p.S;
    const int S = (G + gs - 1) / gs;                         // no empty split (<= p.S)
    hipLaunchKernelGGL((fixed_prefill_kernel<BITS, true, XF>), dim3((unsigned)n, 1, (unsigned)S),
                       dim3(kPBlock), 0, st, x, (const uint32_t *)packed, cb, out, T, M, K, C, ws,
                       gs, p.nT, p.full);
    int rc = cbq_launch_status("fixed_prefill_kernel");
    if (rc) return rc;
    const int64_t n4 = (int64_t)n * kPT * kPM / 4;
    const int blocks = (int)std::min<int64_t>((n4 + 255) / 256, 4096);
    hipLaunchKernelGGL(prefill_reduce_tiles_kernel, dim3(blocks), dim3(256), 0, st, ws, S, n,
                       p.full, p.nT, T, M, out);
    return cbq_launch_status("prefill_reduce_tiles_kernel");
}

// xf != nullptr: x is first copied to fragment order there (prefill_x_frag_kernel)
template <int BITS>
int launch_prefill(const uint16_t *x, const uint8_t *packed, const float *cb, uint16_t *out,
                   int T, int M, int K, int C, const PrefillPlan &p, float *ws, uint16_t *xf,
                   hipStream_t st)
{
    if (!xf) return launch_prefill_x<BITS, false>(x, packed, cb, out, T, M, K, C, p, ws, st);
    const dim3 grid((unsigned)((T + 15) >> 4), (unsigned)((K / kPK + kXfSteps - 1) / kXfSteps));
    hipLaunchKernelGGL(prefill_x_frag_kernel, grid, dim3(256), 0, st, x, xf, T, K);
    const int rc = cbq_launch_status("prefill_x_frag_kernel");
    if (rc) return rc;
    return launch_prefill_x<BITS, true>(xf, packed, cb, out, T, M, K, C, p, ws, st);
}

}  // namespace

// Bytes of the fragment-order copy of x a T x K prefill uses.
static size_t xf_bytes(int T, int K)
{
    return ((size_t)((T + 15) & ~15) * K * sizeof(uint16_t) + 255) & ~(size_t)255;
}

static bool prefill_shape(int T, int M, int K)
{
    return T >= 64 && M > 0 && K > 0 && K % kPK == 0 &&
           (uint64_t)((T + 15) & ~15) * K < (1ull << 31);    // x within one 4 GiB buffer
}

static bool prefill_takes(int T, int M, int K, int bits)
{
    return prefill_shape(T, M, K) && (bits == 8 || (bits >= 10 && bits <= 14)) &&
           (uint64_t)M * (K / kPK) * bits < (1ull << 30);   // index words within one 4 GiB buffer
}

// Workspace bytes of the MFMA prefill with a caller workspace: x in fragment
// order, then the split partials (0: the shape does not take this path).
size_t cbq_prefill_ws_bytes(int T, int M, int K)
{
    if (!prefill_shape(T, M, K)) return 0;
    return xf_bytes(T, K) + prefill_partial_bytes(prefill_plan(T, M, K));
}

// Prefill dispatch used by ck_linear_bf16 / cbq_linear_bf16_ws (cbq_fixed.hip).
// Returns -1 when the shape is not handled here (the caller keeps its
// token-tile path).  With a workspace of cbq_prefill_ws_bytes (256-byte
// aligned) x is copied to fragment order there and K may be split; without
// one, x is read row-major (a lane per row, more slowly) and K is never split.
int cbq_prefill_bf16(const uint16_t *x, const uint8_t *packed, const float *cb, uint16_t *out,
                     int T, int M, int K, int C, int bits, hipStream_t st, void *ws,
                     size_t ws_bytes)
{
    if (!prefill_takes(T, M, K, bits) || (((uintptr_t)packed | (uintptr_t)x) & 15) != 0)
        return -1;
    PrefillPlan p = prefill_plan(T, M, K);
    uint16_t *xf = nullptr;
    float *part = nullptr;
    if (ws && ((uintptr_t)ws & 255) == 0 && ws_bytes >= cbq_prefill_ws_bytes(T, M, K)) {
        xf = (uint16_t *)ws;
        part = (float *)((char *)ws + xf_bytes(T, K));
    } else {
        p.full = p.tiles;
        p.S = 1;
    }
    switch (bits) {
    case 8: return launch_prefill<8>(x, packed, cb, out, T, M, K, C, p, part, xf, st);
    case 10: return launch_prefill<10>(x, packed, cb, out, T, M, K, C, p, part, xf, st);
    case 11: return launch_prefill<11>(x, packed, cb, out, T, M, K, C, p, part, xf, st);
    case 12: return launch_prefill<12>(x, packed, cb, out, T, M, K, C, p, part, xf, st);
    case 13: return launch_prefill<13>(x, packed, cb, out, T, M, K, C, p, part, xf, st);
    case 14: return launch_prefill<14>(x, packed, cb, out, T, M, K, C, p, part, xf, st);
    default: return -1;
    }
}

// Per-wave timeline of the last bf16 prefill launch (every launch of a call
// writes it; the last one's waves win), in a -DCBQ_TIMELINE build:
// kPfTimelineWaves x 6 uint64 (entry, codebook staged, prologue done, loop
// done, exit in 10 ns ticks; K steps).  CK_ERR_ARG in the product build or
// when dst_bytes is short.
extern "C" int cbq_prefill_timeline_read(void *dst, size_t dst_bytes)
{
#ifdef CBQ_TIMELINE
    const size_t n = sizeof(unsigned long long) * kPfTimelineWaves * kPfTimelineFields;
    if (!dst || dst_bytes < n) return CK_ERR_ARG;
    if (hipMemcpyFromSymbol(dst, HIP_SYMBOL(cbq_pf_timeline), n, 0, hipMemcpyDeviceToHost) !=
        hipSuccess)
        return CK_ERR_HIP;
    return CK_SUCCESS;
#else
    (void)dst;
    (void)dst_bytes;
    return CK_ERR_ARG;
#endif
}
