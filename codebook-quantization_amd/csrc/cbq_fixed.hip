// Fixed-width codebook GEMV / skinny GEMM and embedding gather for gfx950.
//
// Index stream: b-bit indices, LSB-first; index i occupies stream bits
// [i*b, (i+1)*b) (src/bitpack.py:32-95, src/compressed_matmul.c:334-347).
// When K % 32 == 0 every run of 32 consecutive indices of a row starts on a
// 32-bit word boundary and fills exactly b words, so one lane loads b words
// with wide loads and unpacks its 32 indices with compile-time shifts
// (v_alignbit for the fields that straddle words).  The codebook sits in LDS,
// padded reads never leave the row's own words, and each wave owns whole
// rows, reducing its lanes' partial dots with a butterfly.
//
// Output semantics follow ck_linear_f32 / ck_embedding_f32
// (rocm/compressed_kernel.hip:58-120): fp32 accumulate, index clamped to C-1,
// output written.
#include "cbq_device.h"


#include <algorithm>
#include <type_traits>

// Matrix-core paths for 2..16 tokens (cbq_tiny.hip); -1 = shape not handled
// there.  fewtok: bf16 matrix cores, K % 128 == 0; tiny: fp32 matrix cores.
int cbq_fixed_fewtok_t(const float *x, const uint8_t *packed, const float *cb, float *out, int T,
                       int M, int K, int C, int bits, hipStream_t st);
int cbq_fixed_fewtok_t_bf16(const uint16_t *x, const uint8_t *packed, const float *cb,
                            uint16_t *out, int T, int M, int K, int C, int bits, hipStream_t st);
int cbq_fixed_tiny_t(const float *x, const uint8_t *packed, const float *cb, float *out, int T,
                     int M, int K, int C, int bits, hipStream_t st);
int cbq_fixed_tiny_t_bf16(const uint16_t *x, const uint8_t *packed, const float *cb,
                          uint16_t *out, int T, int M, int K, int C, int bits, hipStream_t st);

namespace {

constexpr int kBlock = 1024;                // 16 waves share one LDS codebook
constexpr int kWavesPerBlock = kBlock / CBQ_WAVE;
constexpr int kMaxLdsBytes = 64 * 1024;     // per-workgroup budget we allow
constexpr int kMaxLdsCodebook = 16384;      // entries of fp32 codebook in LDS
constexpr int kTinyMinT = 5;                // K % 128 != 0: tiles of 5..16 to the fp32 matrix cores
// The x-in-registers path runs one block per CU, so it may use most of the
// CU's 160 KB of LDS (codebook + padded x + row partials).
constexpr int kMaxLdsBytesXReg = 152 * 1024;

template <typename XT>
__device__ __forceinline__ void load_x32(const XT *__restrict__ p, float xv[32]);

template <>
__device__ __forceinline__ void load_x32<float>(const float *__restrict__ p, float xv[32])
{
    __builtin_memcpy(xv, p, 32 * sizeof(float));
}

template <>
__device__ __forceinline__ void load_x32<uint16_t>(const uint16_t *__restrict__ p, float xv[32])
{
    uint32_t h[16];
    __builtin_memcpy(h, p, 32 * sizeof(uint16_t));
#pragma unroll
    for (int i = 0; i < 16; i++) {
        xv[2 * i] = __uint_as_float(h[i] << 16);
        xv[2 * i + 1] = __uint_as_float(h[i] & 0xffff0000u);
    }
}

// Indices of group `g` of the 32-index groups of a row, already clamped and
// turned into weights (the codebook gather).
template <int BITS>
__device__ __forceinline__ void gather_weights(const uint32_t w[BITS],
                                               const float *__restrict__ s_cb,
                                               uint32_t cmax, float wv[32])
{
    constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const int o = j * BITS;
        const int q = o >> 5;
        const int s = o & 31;
        uint32_t v;
        if (s + BITS <= 32)
            v = w[q] >> s;
        else
            v = funnel(w[q + 1], w[q], (uint32_t)s);
        v &= mask;
        v = v < cmax ? v : cmax;
        wv[j] = s_cb[v];
    }
}

// x row layout in LDS: each 32-element group padded to 36 floats, so the
// eight 16-byte reads a lane makes for its group hit distinct banks across
// lanes (a 128-byte stride would put all lanes on the same banks).
constexpr int kXGroupStride = 36;

// Block = RB * WPR waves (<= 16).  The block walks row groups of RB rows;
// each row is split over WPR waves (split-K), a wave's lanes take the row's
// 32-index groups g = kw*64 + lane + it*64*WPR.  Each lane streams its
// (row, group) items through a ring of D register buffers, so D groups of
// words are in flight while one is unpacked; the first D loads are issued
// before the LDS staging barrier.  When every lane owns a single group of
// each row (NGW == 1) and T == 1, XREG keeps that group's 32 x values in
// registers for the whole kernel.  Row results: wave butterfly, then
// (WPR > 1) a sum of the WPR wave partials through LDS.  T <= TMAX tokens.
template <int BITS, int TMAX, int D, int XMODE, typename XT, typename OT>
__global__ __launch_bounds__(kBlock) void fixed_gemv_kernel(
    const XT *__restrict__ x, const uint32_t *__restrict__ words,
    const float *__restrict__ cb, OT *__restrict__ out, int T, int M, int K, int C, int WPR,
    int RB)
{
    constexpr bool XREG = XMODE == 2;
    // x is staged in LDS for both XLDS and XREG (coalesced global loads; a
    // lane-private 128-byte global read per lane would cost 64 cache-line
    // lookups per instruction); XREG then copies a lane's 32 values to VGPRs.
    constexpr bool XLDS = XMODE == 1 || XREG;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int G = K >> 5;                          // 32-index groups per row
    float *s_cb = lds;
    float *s_red = lds + ((C + 3) & ~3);           // [kWavesPerBlock][TMAX]
    float *s_x = s_red + kWavesPerBlock * TMAX;    // [T][G * kXGroupStride]
    const int tid = threadIdx.x;
    const int wave_count = RB * WPR;
    const int lane = tid & (CBQ_WAVE - 1);
    const int wave = tid / CBQ_WAVE;
    const int rsub = wave / WPR, kw = wave % WPR;
    const int NGW = (G + CBQ_WAVE * WPR - 1) / (CBQ_WAVE * WPR);   // items per row per lane
    const int first = blockIdx.x * RB;
    const int rstride = gridDim.x * RB;
    const int n_iter = first < M ? (M - first + rstride - 1) / rstride : 0;
    const int n_items = n_iter * NGW;              // block-uniform
    const uint32_t cmax = (uint32_t)(C - 1);

    auto item_row = [&](int item) { return first + (item / NGW) * rstride + rsub; };
    auto item_grp = [&](int item) { return kw * CBQ_WAVE + lane + (item % NGW) * CBQ_WAVE * WPR; };

    // Prologue.  Only the first kStageWaves waves stage the codebook (and x
    // for XLDS), each with batches of unconditional loads issued before any
    // of their own weight loads; every other wave starts its weight prefetch
    // at once.  The LDS barrier then waits on those few staging loads only.
    // Every global load is unconditional (clamped addresses): loads under
    // divergent branches make the compiler wait for all outstanding loads,
    // which would defeat the prefetch ring.
    constexpr int kStageWaves = 4;
    constexpr int kStageBatch = 32;
    const int nsw = wave_count < kStageWaves ? wave_count : kStageWaves;
    const int st_threads = nsw * CBQ_WAVE;
    if (wave < nsw) {
        for (int base = 0; base < C; base += kStageBatch * st_threads) {
            float st[kStageBatch];
#pragma unroll
            for (int r = 0; r < kStageBatch; r++) {
                const int i = base + tid + r * st_threads;
                st[r] = cb[i < C ? i : C - 1];
            }
#pragma unroll
            for (int r = 0; r < kStageBatch; r++) {
                const int i = base + tid + r * st_threads;
                if (i < C) s_cb[i] = st[r];
            }
        }
        if (XLDS) {
            const int n = T * K;
            for (int base = 0; base < n; base += kStageBatch * st_threads) {
                float st[kStageBatch];
#pragma unroll
                for (int r = 0; r < kStageBatch; r++) {
                    const int i = base + tid + r * st_threads;
                    st[r] = to_f32<XT>(x[i < n ? i : n - 1]);
                }
#pragma unroll
                for (int r = 0; r < kStageBatch; r++) {
                    const int i = base + tid + r * st_threads;
                    if (i < n) {
                        const int t = i / K, k = i - t * K;
                        s_x[t * G * kXGroupStride + (k >> 5) * kXGroupStride + (k & 31)] = st[r];
                    }
                }
            }
        }
    }
    auto load_item = [&](uint32_t (&dst)[BITS], int item) {
        const int r = item_row(item), g = item_grp(item);
        const bool ok = item < n_items && r < M && g < G;
        __builtin_memcpy(dst, words + ((size_t)(ok ? r : 0) * G + (ok ? g : 0)) * BITS,
                         sizeof(dst));
    };
    uint32_t buf[D][BITS];
#pragma unroll
    for (int d = 0; d < D; d++) load_item(buf[d], d);
    lds_barrier();
    float xr[XREG ? 32 : 1];
    if (XREG) {
        const int g = item_grp(0);
        __builtin_memcpy(xr, s_x + (g < G ? g : 0) * kXGroupStride, sizeof(xr));
    }

    float acc[TMAX];
#pragma unroll
    for (int t = 0; t < TMAX; t++) acc[t] = 0.f;

    for (int base = 0; base < n_items; base += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int item = base + d;
            if (item < n_items) {
                const int row = item_row(item), g = item_grp(item);
                if (row < M && g < G) {
                    float wv[32];
                    gather_weights<BITS>(buf[d], s_cb, cmax, wv);
                    if (XREG) {
                        // four independent partial sums shorten the FMA chain
                        float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
                        for (int j = 0; j < 32; j += 4) {
                            p0 = fmaf(xr[j], wv[j], p0);
                            p1 = fmaf(xr[j + 1], wv[j + 1], p1);
                            p2 = fmaf(xr[j + 2], wv[j + 2], p2);
                            p3 = fmaf(xr[j + 3], wv[j + 3], p3);
                        }
                        acc[0] += (p0 + p1) + (p2 + p3);
                    } else {
#pragma unroll
                        for (int t = 0; t < TMAX; t++) {
                            if (t < T) {
                                float xv[32];
                                if (XLDS)
                                    __builtin_memcpy(xv, s_x + (t * G + g) * kXGroupStride, sizeof(xv));
                                else
                                    load_x32<XT>(x + (size_t)t * K + g * 32, xv);
                                float p0 = 0.f, p1 = 0.f;
#pragma unroll
                                for (int j = 0; j < 32; j += 2) {
                                    p0 = fmaf(xv[j], wv[j], p0);
                                    p1 = fmaf(xv[j + 1], wv[j + 1], p1);
                                }
                                acc[t] += p0 + p1;
                            }
                        }
                    }
                }
                load_item(buf[d], item + D);
                if (item % NGW == NGW - 1) {             // row done (block-uniform)
#pragma unroll
                    for (int t = 0; t < TMAX; t++) {
                        if (t < T) {
                            const float v = wave_sum(acc[t]);
                            if (WPR == 1) {
                                if (lane == 0 && row < M) out[(size_t)t * M + row] = from_f32<OT>(v);
                            } else if (lane == 0) {
                                s_red[wave * TMAX + t] = v;
                            }
                            acc[t] = 0.f;
                        }
                    }
                    if (WPR > 1) {
                        lds_barrier();
                        if (kw == 0 && lane < T && row < M) {
                            float v = 0.f;
                            for (int w = 0; w < WPR; w++) v += s_red[(wave + w) * TMAX + lane];
                            out[(size_t)lane * M + row] = from_f32<OT>(v);
                        }
                        lds_barrier();
                    }
                }
            }
        }
    }
}

// ---- streaming row-owner kernel --------------------------------------------
//
// One 8-wave block per CU.  Wave `wid` owns rows wid, wid + W, ... (W = all
// waves of the grid) and walks them in items of 64 groups: lane l takes group
// chunk*64 + l of the row, i.e. BITS consecutive index words, loaded with
// dwordx4 loads into a two-deep register ring.  The loop body has no barrier,
// no store and no divergent branch, so the only wait is on the oldest ring
// slot.  Row sums stay in lane (row & 63) of `res` and are written 64 rows at
// a time.  Codebook and x are staged into LDS by direct global->LDS loads
// issued before the first weight loads; the wave waits for those alone.

constexpr int kStreamWaves = 8;
constexpr int kStreamBlock = kStreamWaves * CBQ_WAVE;

// Diagnostic build (-DCBQ_TIMELINE): every wave of a one-token plain
// streaming launch records the 100 MHz s_memrealtime clock at entry, after
// the staging, after its first ring of items, after its loop and at exit,
// plus its item count, into cbq_timeline_wave (read by cbq_timeline_read).
// The product build has none of it.
constexpr int kTimelineWaves = 4096;
constexpr int kTimelineFields = 6;
#ifdef CBQ_TIMELINE
__device__ unsigned long long cbq_timeline_wave[kTimelineWaves * kTimelineFields];
#define CBQ_TS(var) const unsigned long long var = __builtin_amdgcn_s_memrealtime()
#endif
constexpr int kStreamD = 2;
// Folded norms with K <= kGlueSmallK (the hidden size of the 8B shapes) hold
// 4 of GlueTile's 16 terms per virtual thread: the 12 others are past K.
constexpr int kGlueSmallK = 4096;
static_assert(kGlueSmallK <= 1024 * 4, "4 terms per virtual thread cover kGlueSmallK");
// LDS for those launches' x0 and x1 (4 terms x 1024 virtual threads each).
constexpr size_t kGlueScratchBytes = 2 * 4 * 1024 * sizeof(float);
constexpr int kStreamLds = 152 * 1024;      // codebook + staged x, per block

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// Pieces [n16, n_pieces) of a padded LDS codebook, written from registers:
// piece n16 = mix (the last entries of cb, then cb[C - 1]), later pieces all
// cb[C - 1].  The 16-byte loads of the staging wrote pieces [0, n16) only.
__device__ __forceinline__ void pad_codebook(float *s_cb, int n16, int n_pieces,
                                             const float (&mix)[4], float last)
{
    typedef float f4v __attribute__((ext_vector_type(4)));
    for (int q = n16 + (int)threadIdx.x; q < n_pieces; q += (int)blockDim.x)
        ((f4v *)s_cb)[q] = q == n16 ? f4v{mix[0], mix[1], mix[2], mix[3]}
                                    : f4v{last, last, last, last};
}

// The 32 raw BITS-wide indices of a lane's group.
template <int BITS>
__device__ __forceinline__ void group_indices(const uint32_t (&w)[BITS], uint32_t idx[32])
{
    constexpr uint32_t m = (1u << BITS) - 1u;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const int o = j * BITS, q = o >> 5, s = o & 31;
        idx[j] = (s + BITS <= 32) ? ((w[q] >> s) & m) : (funnel(w[q + 1], w[q], (uint32_t)s) & m);
    }
}

// x staged in LDS as raw XT bits, one row of K per token.  A 32-element group
// (128 B fp32 / 64 B bf16) is stored as 16-byte chunks in swizzled order, so
// the ds_read_b128 of 8 neighbouring lanes hit distinct bank groups.
template <typename XT> struct XStage;
template <> struct XStage<float> {
    static constexpr int kGroupDw = 32;
    __device__ static int chunk(int c, int g) { return c ^ (g & 7); }
    __device__ static void read(const uint32_t *s, int g, float xv[32])
    {
        typedef uint32_t u4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const u4 v = *(const u4 *)(s + g * 32 + (chunk(c, g) << 2));
            xv[4 * c] = __uint_as_float(v.x);
            xv[4 * c + 1] = __uint_as_float(v.y);
            xv[4 * c + 2] = __uint_as_float(v.z);
            xv[4 * c + 3] = __uint_as_float(v.w);
        }
    }
};
template <> struct XStage<uint16_t> {
    static constexpr int kGroupDw = 16;
    __device__ static int chunk(int c, int g) { return c ^ ((g >> 1) & 3); }
    __device__ static void read(const uint32_t *s, int g, float xv[32])
    {
        typedef uint32_t u4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const u4 v = *(const u4 *)(s + g * 16 + (chunk(c, g) << 2));
            const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xv[8 * c + 2 * i] = __uint_as_float(u[i] << 16);
                xv[8 * c + 2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
            }
        }
    }
};

// AFFINE: no codebook table; index i stands for the bf16 value with bits
// aff_lo + i (i < aff_w), 0x8000 + aff_lo + i - aff_w (i < 2 aff_w), else 0:
// the re-indexed form of a codebook whose nonzero values all have bf16
// magnitudes in [aff_lo, aff_lo + aff_w) (cbq_linear_affine_f32).
// XMODE (T = 1, float x): x is staged as xform_value(XMODE, x, x1, ...) -
// silu(x) * x1, or the RMSNorm of x (+ x1) with block 0 storing x + x1 to
// h_out - so the decoder's separate glue launch disappears.
template <bool KCHUNK, typename OT>
__device__ __forceinline__ void put_out_t(OT *o, float v, int accum)
{
    if constexpr (KCHUNK) {
        static_assert(sizeof(OT) == sizeof(float), "column ranges accumulate fp32 outputs");
        *o = accum ? *o + v : v;
    } else {
        *o = from_f32<OT>(v);
    }
}

//
// GlueTile::load through LDS (K <= 1024 NJ): element i = tid + k NTHR +
// 1024 j of x0 goes to s_glue[(k NJ + j) NTHR + tid] (x1 after all of
// x0's), one direct global->LDS dword load per element; indices past K load
// element K - 1 again (finish() zeroes those terms).  A lane reads back only
// what its own loads wrote, so a wait for them is enough (no barrier).
template <int NTHR, int NJ, bool TWO>
__device__ __forceinline__ void glue_dma(const float *__restrict__ x0,
                                         const float *__restrict__ x1, int K, float *s_glue)
{
    constexpr int V = 1024 / NTHR;
    const int wbase = (int)(threadIdx.x & ~(CBQ_WAVE - 1));
#pragma unroll
    for (int k = 0; k < V; k++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int i = (int)threadIdx.x + k * NTHR + j * 1024;
            const int ic = i < K ? i : K - 1;
            const int slot = k * NJ + j;
            __builtin_amdgcn_global_load_lds((const void *)(x0 + ic),
                                             (lds_ptr_t)(s_glue + slot * NTHR + wbase), 4, 0, 0);
            if constexpr (TWO)
                __builtin_amdgcn_global_load_lds(
                    (const void *)(x1 + ic), (lds_ptr_t)(s_glue + (V * NJ + slot) * NTHR + wbase),
                    4, 0, 0);
        }
}

// KCHUNK: the launch covers index columns [k0, k0 + K) of rows Kfull long
// (x is [T, Kfull]); accum != 0 adds the partial products to out instead of
// writing them.  The host splits K this way when x of all T tokens does not
// fit in LDS, one launch per column range in order.
// GLU (T = 1): the matrix holds 2M rows, gate rows [0, M) then up rows
// [M, 2M); a wave takes gate row j and up row j back to back and writes
// out[j] = silu(gate_j . x) * (up_j . x), rounded as silu_mul_value, so the
// down projection that consumes it stages plain x.
template <int BITS, int TMAX, typename XT, typename OT, bool AFFINE = false, int XMODE = XF_NONE,
          bool KCHUNK = false, bool GLU = false, int NJ = 16>
__global__ __launch_bounds__(kStreamBlock) void fixed_stream_kernel(
    const XT *__restrict__ x, const uint32_t *__restrict__ words,
    const float *__restrict__ cb, OT *__restrict__ out, int T, int M, int K, int C,
    uint32_t aff_lo, uint32_t aff_w, const float *__restrict__ x1, float *__restrict__ h_out,
    float eps, int Kfull, int k0, int accum, float *__restrict__ arg_v = nullptr,
    int *__restrict__ arg_i = nullptr)
{
    static_assert(!KCHUNK || (XMODE == XF_NONE && !AFFINE), "column ranges: plain x only");
    static_assert(!GLU || (TMAX == 1 && !KCHUNK && XMODE != XF_SILU), "gate/up pairs: one token");
    // arg_v / arg_i (T = 1): besides writing out (when out is not null), the
    // block reduces its rows to one (max, first index) pair of the greedy
    // pick, written to arg_v / arg_i [blockIdx.x].
    constexpr bool PADDED = BITS <= 14 && !AFFINE;
    constexpr int D = kStreamD;
#ifdef CBQ_TIMELINE
    constexpr bool kTimed = TMAX == 1 && XMODE == XF_NONE && !KCHUNK && !AFFINE;
    CBQ_TS(ts_entry);
    unsigned long long ts_first = 0;
#endif
    __shared__ __attribute__((aligned(16))) float s_cbp[PADDED ? (1 << BITS) : 1];
    __shared__ float s_red16[XMODE >= XF_ADD_RMS ? 16 : 1];
    extern __shared__ __attribute__((aligned(16))) float s_dyn[];
    const int C_eff = C < (1 << BITS) ? C : (1 << BITS);
    const int cb_slots = AFFINE ? 0 : PADDED ? (1 << BITS) : ((C_eff + 63) & ~63);
    float *s_cb = PADDED ? s_cbp : s_dyn;
    uint32_t *s_x = (uint32_t *)(PADDED ? s_dyn : s_dyn + cb_slots);

    const int G = K >> 5;
    const int Gf = KCHUNK ? (Kfull >> 5) : G;      // groups per stored row
    const int g0 = KCHUNK ? (k0 >> 5) : 0;         // first group of this launch
    const int NGW = (G + CBQ_WAVE - 1) / CBQ_WAVE;
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / CBQ_WAVE);
    const int W = gridDim.x * kStreamWaves;
    const int wid = blockIdx.x * kStreamWaves + wave;
    // rows of this wave (GLU: two per output, gate then up)
    const int rows = wid < M ? (GLU ? 2 : 1) * ((M - wid + W - 1) / W) : 0;
    const int n_items = rows * NGW;
    const uint32_t cmax4 = (uint32_t)(C_eff - 1) << 2;

    // Folded glue: x0 (and x1) requested first, ahead of the codebook and
    // the weight stream.  At K <= kGlueSmallK the loads go straight to LDS
    // past the staged x (kGlueScratchBytes of dynamic LDS), so no register
    // waits on them and the explicit wait below leaves the ring in flight.
    GlueTile<kStreamBlock, XMODE, NJ> tile;       // NJ < 16: K <= 1024 NJ
    constexpr bool kGlueDma = XMODE != XF_NONE && NJ == 4;
    float *const s_glue =
        (float *)s_x + ((T * G * XStage<XT>::kGroupDw + 63) & ~63);
    if constexpr (kGlueDma) glue_dma<kStreamBlock, NJ, decltype(tile)::TWO>(
        (const float *)x, x1, K, s_glue);
    else if constexpr (XMODE != XF_NONE) tile.load((const float *)x, x1, K);

    // Staging: direct global->LDS loads, every wave a share.  Padded
    // codebook: whole 16-byte pieces of cb by 16-byte loads (lanes past them
    // idle); the piece holding entry C and the padding up to 2^BITS (all
    // cb[C - 1]) are written from registers once the loads have landed.
    int n16 = 0;                                   // 16-byte pieces loaded
    float pad_mix[4], pad_last = 0.f;
    if constexpr (PADDED) {
        n16 = C_eff >> 2;
        if (((uintptr_t)cb & 15) == 0) {
            for (int i = wave; i < ((n16 + 63) >> 6); i += kStreamWaves) {
                const int q = (i << 6) + lane;
                if (q < n16)
                    __builtin_amdgcn_global_load_lds((const void *)(cb + 4 * q),
                                                     (lds_ptr_t)(s_cb + (i << 8)), 16, 0, 0);
            }
        } else {
            // codebook off 16-byte alignment: the same 4 n16 entries by dword
            // loads (none past them: pad_codebook writes those slots)
            const int n4 = n16 << 2;
            for (int i = wave; i < ((n4 + 63) >> 6); i += kStreamWaves) {
                const int e = (i << 6) + lane;
                if (e < n4)
                    __builtin_amdgcn_global_load_lds((const void *)(cb + e),
                                                     (lds_ptr_t)(s_cb + (i << 6)), 4, 0, 0);
            }
        }
        pad_last = cb[C_eff - 1];
#pragma unroll
        for (int j = 0; j < 4; j++) pad_mix[j] = cb[min(4 * n16 + j, C_eff - 1)];
    } else {
        for (int i = wave; i < (cb_slots >> 6); i += kStreamWaves) {
            const int e = (i << 6) + lane;
            __builtin_amdgcn_global_load_lds((const void *)(cb + (e < C ? e : C - 1)),
                                             (lds_ptr_t)(s_cb + (i << 6)), 4, 0, 0);
        }
    }
    constexpr int GD = XStage<XT>::kGroupDw;
    const int xdw = G * GD;                        // dwords of one token's x
    const int n_xdw = T * xdw;
    const uint32_t *xw = (const uint32_t *)x;
    // x by 16-byte loads (each a swizzled chunk) when it is 16-byte aligned
    // and a whole number of 64-lane loads; else by dword loads.
    const bool x16 = ((uintptr_t)x & 15) == 0 && (n_xdw & 255) == 0;
    if (XMODE == XF_NONE && x16) {
        const int cpt = xdw >> 2, cpg = GD >> 2;   // chunks per token, per group
        for (int i = wave; i < (n_xdw >> 8); i += kStreamWaves) {
            const int qs = (i << 6) + lane;        // LDS chunk slot (this lane's)
            const int t = qs / cpt, dq = qs - t * cpt;
            const int g = dq / cpg, c = dq - g * cpg;
            const int src = t * (Gf * GD) + (g0 + g) * GD + (XStage<XT>::chunk(c, g) << 2);
            __builtin_amdgcn_global_load_lds((const void *)(xw + src),
                                             (lds_ptr_t)(s_x + (i << 8)), 16, 0, 0);
        }
    } else if constexpr (XMODE == XF_NONE) {
        for (int i = wave; i < ((n_xdw + 63) >> 6); i += kStreamWaves) {
            int sl = (i << 6) + lane;              // LDS dword slot (this lane's)
            sl = sl < n_xdw ? sl : n_xdw - 1;      // tail lanes re-copy the last dword
            const int t = sl / xdw, d = sl - t * xdw;
            const int g = d / GD, p = (d % GD) >> 2;
            const int src = t * (Gf * GD) + (g0 + g) * GD + (XStage<XT>::chunk(p, g) << 2) + (d & 3);
            __builtin_amdgcn_global_load_lds((const void *)(xw + src),
                                             (lds_ptr_t)(s_x + (i << 6)), 4, 0, 0);
        }
    }
    // The weight addresses depend on `zero`, produced by a volatile asm with a
    // memory clobber, so no weight load is issued before the staging loads.
    uint32_t zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero) : : "memory");

    auto item_ptr = [&](int item) {
        // past the wave's last item: re-read the last one (an L2 hit, no HBM traffic)
        const int it = item < n_items ? item : (n_items > 0 ? n_items - 1 : 0);
        const int ri = it / NGW, ch = it - ri * NGW;
        int g = ch * CBQ_WAVE + lane;
        g = g < G ? g : G - 1;
        const int row = rows <= 0 ? 0 : GLU ? ((ri & 1) ? M : 0) + wid + (ri >> 1) * W
                                            : wid + ri * W;
        return words + ((size_t)row * Gf + g0 + g) * BITS + zero;
    };
    // One token: only the first ring slot is requested before the staging
    // completes, the others right after the barrier.  Half the opening burst
    // lets the staging loads (queued behind it) land sooner: 0.4-0.5 us off
    // every 9B-shape launch.
    constexpr int kFirst = TMAX == 1 ? 1 : D;
    uint32_t buf[D][BITS];
#pragma unroll
    for (int d = 0; d < kFirst; d++) __builtin_memcpy(buf[d], item_ptr(d), sizeof(buf[d]));
    __builtin_amdgcn_sched_barrier(0);
    // vmcnt(N): at most N loads outstanding.  N = the fewest instructions the
    // kFirst ring loads can take (dwordx4), so every older staging (and glue)
    // load has landed while the ring stays in flight.  Explicit, since the
    // compiler's own wait before the first use of a glue value drains the
    // ring as well (it cannot count past the codebook DMA loop).
    constexpr int kAfter = kFirst * ((BITS + 3) / 4);
    __builtin_amdgcn_s_waitcnt((kAfter & 15) | (7 << 4) | (15 << 8) | ((kAfter >> 4) << 14));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XMODE == XF_NONE) {
        if constexpr (PADDED) pad_codebook(s_cb, n16, (1 << BITS) >> 2, pad_mix, pad_last);
        lds_barrier();
    } else {
        // the transformed x from registers, while the first weight loads fly;
        // element i goes where the swizzled staging above would put it
        if constexpr (kGlueDma) {                  // this lane's own direct loads
            constexpr int V = decltype(tile)::VPT;
#pragma unroll
            for (int k = 0; k < V; k++)
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    const int slot = k * NJ + j;
                    tile.a[k][j] = s_glue[slot * kStreamBlock + threadIdx.x];
                    if constexpr (decltype(tile)::TWO)
                        tile.b[k][j] = s_glue[(V * NJ + slot) * kStreamBlock + threadIdx.x];
                }
        }
        const float r = tile.finish(K, eps, s_red16);
        if (XMODE == XF_ADD_RMS && blockIdx.x == 0 && h_out != nullptr) tile.store_sum(h_out, K);
#pragma unroll
        for (int k = 0; k < tile.VPT; k++)
#pragma unroll
            for (int j = 0; j < tile.kJ; j++) {
                const int i = (int)threadIdx.x + k * kStreamBlock + j * 1024;
                const int g = i >> 5;
                const int sl = (g << 5) + ((((i >> 2) & 7) ^ (g & 7)) << 2) + (i & 3);
                if (i < K) s_x[sl] = __float_as_uint(tile.value(k, j, r));
            }
        // (the codebook loads landed before the glue loads finish() waited for)
        if constexpr (PADDED) pad_codebook(s_cb, n16, (1 << BITS) >> 2, pad_mix, pad_last);
        lds_barrier();
    }

#ifdef CBQ_TIMELINE
    CBQ_TS(ts_staged);
#endif
#pragma unroll
    for (int d = kFirst; d < D; d++) __builtin_memcpy(buf[d], item_ptr(d), sizeof(buf[d]));
    float acc[TMAX], res[TMAX];
#pragma unroll
    for (int t = 0; t < TMAX; t++) acc[t] = res[t] = 0.f;
    float a_best = -INFINITY;                      // greedy-pick candidate of this lane
    int a_idx = kArgNone;
    float g_res = 0.f;                             // GLU: gate sums, lane = pair % 64
    int ri = 0, ch = 0, base = 0;
    do {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int item = base + d;
            const int g = ch * CBQ_WAVE + lane;
            const int gg = g < G ? g : G - 1;
            const bool valid = item < n_items && g < G;
            float wv[32];
            if constexpr (AFFINE) {
                uint32_t idx[32];
                group_indices<BITS>(buf[d], idx);
                const uint32_t neg = aff_lo + 0x8000u - aff_w, w2 = 2u * aff_w;
#pragma unroll
                for (int j = 0; j < 32; j++) {
                    const uint32_t b = (idx[j] + (idx[j] < aff_w ? aff_lo : neg)) << 16;
                    wv[j] = __uint_as_float(idx[j] < w2 ? b : 0u);      // index 2w: zero
                }
            } else {
                uint32_t off[32];
                group_offsets<BITS, PADDED>(buf[d], cmax4, off);
#pragma unroll
                for (int j = 0; j < 32; j++) wv[j] = *(const float *)((const char *)s_cb + off[j]);
            }
#pragma unroll
            for (int t = 0; t < TMAX; t++) {
                if (t < T) {
                    float xv[32];
                    XStage<XT>::read(s_x + t * xdw, gg, xv);
                    float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
                    for (int j = 0; j < 32; j += 4) {
                        p0 = fmaf(xv[j], wv[j], p0);
                        p1 = fmaf(xv[j + 1], wv[j + 1], p1);
                        p2 = fmaf(xv[j + 2], wv[j + 2], p2);
                        p3 = fmaf(xv[j + 3], wv[j + 3], p3);
                    }
                    acc[t] += valid ? (p0 + p1) + (p2 + p3) : 0.f;
                }
            }
            __builtin_memcpy(buf[d], item_ptr(item + D), sizeof(buf[d]));
            if (GLU && ++ch == NGW) {                // gate or up row done (wave-uniform)
                ch = 0;
                // gate and up sums wait in lane pair % 64; each lane forms its
                // pair's SiLU product when the 64 pairs are written
                const float s = wave_sum(acc[0]);
                acc[0] = 0.f;
                const bool mine = lane == ((ri >> 1) & 63) && ri < rows;
                if (ri & 1) res[0] = mine ? s : res[0];
                else g_res = mine ? s : g_res;
                ri++;
                if ((ri & 127) == 0 && ri <= rows)
                    out[wid + ((ri >> 1) - 64 + lane) * W] =
                        from_f32<OT>(silu_mul_value(g_res, res[0]));
            } else if (!GLU && ++ch == NGW) {       // row done (wave-uniform)
                ch = 0;
#pragma unroll
                for (int t = 0; t < TMAX; t++) {
                    if (t < T) {
                        const float s = wave_sum(acc[t]);
                        acc[t] = 0.f;
                        res[t] = (lane == (ri & 63) && ri < rows) ? s : res[t];
                    }
                }
                ri++;
                if ((ri & 63) == 0 && ri <= rows) {
                    const int row = wid + (ri - 64 + lane) * W;
                    if (out) {
#pragma unroll
                        for (int t = 0; t < TMAX; t++)
                            if (t < T) put_out_t<KCHUNK>(out + (size_t)t * M + row, res[t], accum);
                    }
                    if (arg_v && arg_better(res[0], row, a_best, a_idx)) {
                        a_best = res[0];
                        a_idx = row;
                    }
                }
            }
        }
        base += D;
#ifdef CBQ_TIMELINE
        if (base == D) ts_first = __builtin_amdgcn_s_memrealtime();
#endif
    } while (base < n_items);
#ifdef CBQ_TIMELINE
    CBQ_TS(ts_loop);
#endif
    const int n_res = GLU ? rows >> 1 : rows;       // outputs of this wave
    const int rb = n_res & ~63;
    if (GLU) res[0] = silu_mul_value(g_res, res[0]);
    if (lane < n_res - rb) {
        const int row = wid + (rb + lane) * W;
        if (out) {
#pragma unroll
            for (int t = 0; t < TMAX; t++)
                if (t < T) put_out_t<KCHUNK>(out + (size_t)t * M + row, res[t], accum);
        }
        if (arg_v && arg_better(res[0], row, a_best, a_idx)) {
            a_best = res[0];
            a_idx = row;
        }
    }
    if (arg_v) {                                   // uniform: every thread takes part
        __shared__ float s_av[kStreamWaves];
        __shared__ int s_ai[kStreamWaves];
        arg_block_store(a_best, a_idx, s_av, s_ai, arg_v, arg_i);
    }
#ifdef CBQ_TIMELINE
    if constexpr (kTimed) {
        CBQ_TS(ts_exit);
        if (lane == 0 && wid < kTimelineWaves) {
            unsigned long long *tl = cbq_timeline_wave + (size_t)wid * kTimelineFields;
            tl[0] = ts_entry;
            tl[1] = ts_staged;
            tl[2] = ts_first;
            tl[3] = ts_loop;
            tl[4] = ts_exit;
            tl[5] = (unsigned long long)n_items;
        }
    }
#endif
}

// Any width, any K, codebook read through the cache: per-element 4-byte
// window like the reference (reads at most 3 bytes past the last index).
template <int TMAX, typename XT, typename OT>
__global__ __launch_bounds__(kBlock) void fixed_gemv_generic_kernel(
    const XT *__restrict__ x, const uint8_t *__restrict__ packed,
    const float *__restrict__ cb, OT *__restrict__ out, int T, int M, int K, int C,
    int bits)
{
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = threadIdx.x / CBQ_WAVE;
    const uint32_t mask = (1u << bits) - 1u;
    const uint32_t cmax = (uint32_t)(C - 1);
    for (int row = blockIdx.x * kWavesPerBlock + wave; row < M;
         row += gridDim.x * kWavesPerBlock) {
        float acc[TMAX];
#pragma unroll
        for (int t = 0; t < TMAX; t++) acc[t] = 0.f;
        for (int k = lane; k < K; k += CBQ_WAVE) {
            const int64_t bit = ((int64_t)row * K + k) * bits;
            const uint8_t *p = packed + (bit >> 3);
            uint32_t win = (uint32_t)p[0] | ((uint32_t)p[1] << 8) |
                           ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
            uint32_t v = (win >> (bit & 7)) & mask;
            v = v < cmax ? v : cmax;
            const float w = cb[v];
#pragma unroll
            for (int t = 0; t < TMAX; t++)
                if (t < T) acc[t] = fmaf(to_f32<XT>(x[(size_t)t * K + k]), w, acc[t]);
        }
#pragma unroll
        for (int t = 0; t < TMAX; t++) {
            if (t < T) {
                const float s = wave_sum(acc[t]);
                if (lane == 0) out[(size_t)t * M + row] = from_f32<OT>(s);
            }
        }
    }
}

// Embedding: one thread per 32-index group of a requested row (H % 32 == 0).
template <int BITS>
__global__ __launch_bounds__(kBlock) void fixed_embedding_kernel(
    const int32_t *__restrict__ ids, const uint32_t *__restrict__ words,
    const float *__restrict__ cb, float *__restrict__ out, int T, int vocab, int H,
    int C)
{
    const int G = H >> 5;
    const int g = blockIdx.x * kBlock + threadIdx.x;
    const int t = blockIdx.y;
    if (g >= G || t >= T) return;
    int id = ids[t];
    if (vocab > 0) id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
    uint32_t w[BITS];
    __builtin_memcpy(w, words + ((size_t)id * G + g) * BITS, BITS * sizeof(uint32_t));
    constexpr uint32_t mask = (1u << BITS) - 1u;
    const uint32_t cmax = (uint32_t)(C - 1);
    float v32[32];
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const int o = j * BITS, q = o >> 5, s = o & 31;
        uint32_t v = (s + BITS <= 32) ? (w[q] >> s) : funnel(w[q + 1], w[q], (uint32_t)s);
        v &= mask;
        v = v < cmax ? v : cmax;
        v32[j] = cb[v];
    }
    __builtin_memcpy(out + (size_t)t * H + (size_t)g * 32, v32, sizeof(v32));
}

__global__ __launch_bounds__(kBlock) void fixed_embedding_generic_kernel(
    const int32_t *__restrict__ ids, const uint8_t *__restrict__ packed,
    const float *__restrict__ cb, float *__restrict__ out, int T, int vocab, int H,
    int C, int bits)
{
    const int h = blockIdx.x * kBlock + threadIdx.x;
    const int t = blockIdx.y;
    if (h >= H || t >= T) return;
    int id = ids[t];
    if (vocab > 0) id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
    const int64_t bit = ((int64_t)id * H + h) * bits;
    const uint8_t *p = packed + (bit >> 3);
    uint32_t win = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                   ((uint32_t)p[3] << 24);
    uint32_t v = (win >> (bit & 7)) & ((1u << bits) - 1u);
    const uint32_t cmax = (uint32_t)(C - 1);
    out[(size_t)t * H + h] = cb[v < cmax ? v : cmax];
}

// ---- launch plumbing -------------------------------------------------------

// Waves per row.  Prefer one 32-index group per lane per row (WPR = G/64
// when that is <= 8), which lets T = 1 keep x in registers; otherwise split
// rows only as far as needed to give every CU ~16 waves.
int pick_wpr(int M, int G)
{
    const int full = (G + CBQ_WAVE - 1) / CBQ_WAVE;
    if (full <= kWavesPerBlock) return full;
    const int want_waves = cbq_num_cus() * 16;
    int wpr = 1;
    while (wpr < kWavesPerBlock && M * wpr < want_waves && G > CBQ_WAVE * wpr) wpr <<= 1;
    return wpr;
}

template <int BITS, int TMAX, int XMODE, typename XT, typename OT>
int launch_fast(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T,
                int M, int K, int C, hipStream_t st)
{
    const int G = K / 32;
    const int wpr = pick_wpr(M, G);
    const int rb = std::max(1, kWavesPerBlock / wpr);
    const size_t lds = (size_t)((C + 3) & ~3) * 4 + (size_t)kWavesPerBlock * TMAX * 4 +
                       (XMODE != 0 ? (size_t)T * G * kXGroupStride * 4 : 0);
    // One 16-wave block per CU: each block stages its own codebook copy.
    const int per_cu = 1;
    const int blocks = std::max(1, std::min((M + rb - 1) / rb, cbq_num_cus() * per_cu));
    constexpr int D = TMAX <= 4 ? 3 : 2;
    hipLaunchKernelGGL((fixed_gemv_kernel<BITS, TMAX, D, XMODE, XT, OT>), dim3(blocks),
                       dim3(rb * wpr * CBQ_WAVE), lds, st, x, (const uint32_t *)packed, cb, out,
                       T, M, K, C, wpr, rb);
    return cbq_launch_status("fixed_gemv_kernel");
}

template <int BITS, int TMAX, typename XT, typename OT>
int dispatch_x(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T,
               int M, int K, int C, hipStream_t st)
{
    const int G = K / 32;
    const size_t cb_bytes = (size_t)((C + 3) & ~3) * 4;
    if constexpr (TMAX == 1) {
        if ((G + CBQ_WAVE - 1) / CBQ_WAVE <= kWavesPerBlock &&
            cb_bytes + (size_t)G * kXGroupStride * 4 <= (size_t)kMaxLdsBytesXReg)
            return launch_fast<BITS, TMAX, 2>(x, packed, cb, out, T, M, K, C, st);   // x in VGPRs
    }
    if (cb_bytes + (size_t)T * G * kXGroupStride * 4 <= (size_t)kMaxLdsBytes)
        return launch_fast<BITS, TMAX, 1>(x, packed, cb, out, T, M, K, C, st);   // x in LDS
    return launch_fast<BITS, TMAX, 0>(x, packed, cb, out, T, M, K, C, st);       // x via cache
}

template <int BITS, int TMAX, typename XT, typename OT>
int launch_stream(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T, int M,
                  int K, int C, size_t dyn_lds, hipStream_t st)
{
    const int blocks =
        std::max(1, std::min(cbq_num_cus(), (M + kStreamWaves - 1) / kStreamWaves));
    hipLaunchKernelGGL((fixed_stream_kernel<BITS, TMAX, XT, OT>), dim3(blocks),
                       dim3(kStreamBlock), dyn_lds, st, x, (const uint32_t *)packed, cb, out, T,
                       M, K, C, 0u, 0u, (const float *)nullptr, (float *)nullptr, 0.f, K, 0, 0);
    return cbq_launch_status("fixed_stream_kernel");
}

template <int BITS, int TMAX>
int launch_affine(const float *x, const uint8_t *packed, uint32_t lo, uint32_t w, float *out,
                  int T, int M, int K, size_t dyn_lds, hipStream_t st)
{
    const int blocks =
        std::max(1, std::min(cbq_num_cus(), (M + kStreamWaves - 1) / kStreamWaves));
    hipLaunchKernelGGL((fixed_stream_kernel<BITS, TMAX, float, float, true>), dim3(blocks),
                       dim3(kStreamBlock), dyn_lds, st, x, (const uint32_t *)packed,
                       (const float *)nullptr, out, T, M, K, 1, lo, w, (const float *)nullptr,
                       (float *)nullptr, 0.f, K, 0, 0);
    return cbq_launch_status("fixed_stream_kernel<affine>");
}

template <int BITS>
int dispatch_affine(const float *x, const uint8_t *packed, uint32_t lo, uint32_t w, float *out,
                    int T, int M, int K, hipStream_t st)
{
    const size_t n_xdw = (size_t)T * (K / 32) * XStage<float>::kGroupDw;
    const size_t dyn = ((n_xdw + 63) & ~(size_t)63) * 4;
    if (dyn > (size_t)kStreamLds) return CK_ERR_ARG;
    if (T == 1) return launch_affine<BITS, 1>(x, packed, lo, w, out, T, M, K, dyn, st);
    if (T <= 4) return launch_affine<BITS, 4>(x, packed, lo, w, out, T, M, K, dyn, st);
    return launch_affine<BITS, 16>(x, packed, lo, w, out, T, M, K, dyn, st);
}

// Dynamic LDS the streaming kernel needs (0 if it does not fit): unpadded
// codebook (BITS > 14) + all T rows of x, rounded to 64-dword staging steps.
template <int BITS, typename XT>
size_t stream_dyn_lds(int T, int K, int C)
{
    const size_t c_eff = (size_t)std::min(C, 1 << BITS);
    const size_t cb_static = BITS <= 14 ? ((size_t)4 << BITS) : 0;
    const size_t cb_dyn = BITS <= 14 ? 0 : ((c_eff + 63) & ~(size_t)63) * 4;
    const size_t n_xdw = (size_t)T * (K / 32) * XStage<XT>::kGroupDw;
    const size_t x_bytes = ((n_xdw + 63) & ~(size_t)63) * 4;
    if (cb_static + cb_dyn + x_bytes > (size_t)kStreamLds) return 0;
    return cb_dyn + x_bytes;
}

// x of all T tokens too large for LDS (T = 16 at K = 4096): the columns go in
// ranges whose x does fit, one streaming launch per range in order, the first
// writing out and the rest adding to it.  Every weight is still read once.
template <int BITS, int TMAX>
int launch_stream_cols(const float *x, const uint8_t *packed, const float *cb, float *out,
                       int T, int M, int K, int C, hipStream_t st)
{
    const int G = K / 32;
    int gmax = G;
    while (gmax > 0 && !stream_dyn_lds<BITS, float>(T, gmax * 32, C)) gmax--;
    if (gmax == 0) return -1;
    const int n = (G + gmax - 1) / gmax;
    const int gc = (G + n - 1) / n;                  // balanced ranges, <= gmax groups
    const int blocks =
        std::max(1, std::min(cbq_num_cus(), (M + kStreamWaves - 1) / kStreamWaves));
    for (int i = 0; i * gc < G; i++) {
        const int ga = i * gc, gb = std::min(G, ga + gc);
        const int kc = (gb - ga) * 32;
        const size_t dyn = stream_dyn_lds<BITS, float>(T, kc, C);
        hipLaunchKernelGGL((fixed_stream_kernel<BITS, TMAX, float, float, false, XF_NONE, true>),
                           dim3(blocks), dim3(kStreamBlock), dyn, st, x,
                           (const uint32_t *)packed, cb, out, T, M, kc, C, 0u, 0u,
                           (const float *)nullptr, (float *)nullptr, 0.f, K, ga * 32, i > 0);
    }
    return cbq_launch_status("fixed_stream_kernel<columns>");
}

template <int BITS, typename XT, typename OT>
int dispatch_t(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T,
               int M, int K, int C, hipStream_t st)
{
    // Streaming kernel when x of all T tokens fits in LDS beside the codebook
    // (the x staging copies dwords, so x must be 4-byte aligned).
    const size_t dyn = ((uintptr_t)x & 3) == 0 ? stream_dyn_lds<BITS, XT>(T, K, C) : 0;
    if (dyn) {
        if (T == 1) return launch_stream<BITS, 1>(x, packed, cb, out, T, M, K, C, dyn, st);
        if (T <= 4) return launch_stream<BITS, 4>(x, packed, cb, out, T, M, K, C, dyn, st);
        return launch_stream<BITS, 16>(x, packed, cb, out, T, M, K, C, dyn, st);
    }
    if constexpr (std::is_same<XT, float>::value && std::is_same<OT, float>::value) {
        if (T > 1 && ((uintptr_t)x & 3) == 0) {
            const int rc = T <= 4 ? launch_stream_cols<BITS, 4>(x, packed, cb, out, T, M, K, C, st)
                                  : launch_stream_cols<BITS, 16>(x, packed, cb, out, T, M, K, C, st);
            if (rc >= 0) return rc;
        }
    }
    if (T == 1) return dispatch_x<BITS, 1>(x, packed, cb, out, T, M, K, C, st);
    if (T <= 4) return dispatch_x<BITS, 4>(x, packed, cb, out, T, M, K, C, st);
    return dispatch_x<BITS, 16>(x, packed, cb, out, T, M, K, C, st);
}

template <int TMAX, typename XT, typename OT>
int launch_generic(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T,
                   int M, int K, int C, int bits, hipStream_t st)
{
    const int blocks = std::max(1, std::min((M + kWavesPerBlock - 1) / kWavesPerBlock,
                                            cbq_num_cus() * 8));
    hipLaunchKernelGGL((fixed_gemv_generic_kernel<TMAX, XT, OT>), dim3(blocks),
                       dim3(kBlock), 0, st, x, packed, cb, out, T, M, K, C, bits);
    return cbq_launch_status("fixed_gemv_generic_kernel");
}

// One token tile (T <= 16).
template <typename XT, typename OT>
int linear_tile(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T,
                int M, int K, int C, int bits, hipStream_t st)
{
    const bool fast = (K % 32 == 0) && C <= kMaxLdsCodebook &&
                      ((uintptr_t)packed & 3) == 0;
    if (fast && T >= 2) {
        int rc = -1;
        if constexpr (std::is_same<XT, float>::value && std::is_same<OT, float>::value) {
            rc = cbq_fixed_fewtok_t(x, packed, cb, out, T, M, K, C, bits, st);
            if (rc < 0 && T >= kTinyMinT) rc = cbq_fixed_tiny_t(x, packed, cb, out, T, M, K, C, bits, st);
        }
        if constexpr (std::is_same<XT, uint16_t>::value && std::is_same<OT, uint16_t>::value) {
            rc = cbq_fixed_fewtok_t_bf16(x, packed, cb, out, T, M, K, C, bits, st);
            if (rc < 0 && T >= kTinyMinT)
                rc = cbq_fixed_tiny_t_bf16(x, packed, cb, out, T, M, K, C, bits, st);
        }
        if (rc >= 0) return rc;
    }
    if (fast) {
        switch (bits) {
        case 8: return dispatch_t<8>(x, packed, cb, out, T, M, K, C, st);
        case 10: return dispatch_t<10>(x, packed, cb, out, T, M, K, C, st);
        case 11: return dispatch_t<11>(x, packed, cb, out, T, M, K, C, st);
        case 12: return dispatch_t<12>(x, packed, cb, out, T, M, K, C, st);
        case 13: return dispatch_t<13>(x, packed, cb, out, T, M, K, C, st);
        case 14: return dispatch_t<14>(x, packed, cb, out, T, M, K, C, st);
        case 16: return dispatch_t<16>(x, packed, cb, out, T, M, K, C, st);
        default: break;
        }
    }
    if (T == 1) return launch_generic<1>(x, packed, cb, out, T, M, K, C, bits, st);
    if (T <= 4) return launch_generic<4>(x, packed, cb, out, T, M, K, C, bits, st);
    return launch_generic<16>(x, packed, cb, out, T, M, K, C, bits, st);
}

template <typename XT, typename OT>
int linear_any_t(const XT *x, const uint8_t *packed, const float *cb, OT *out, int T,
                 int M, int K, int C, int bits, hipStream_t st)
{
    if (!x || !packed || !cb || !out) return CK_ERR_ARG;
    if (T <= 0 || M <= 0 || K <= 0 || C <= 0 || bits < 1 || bits > 16) return CK_ERR_ARG;
    for (int t0 = 0; t0 < T; t0 += 16) {
        const int tt = std::min(16, T - t0);
        int rc = linear_tile<XT, OT>(x + (size_t)t0 * K, packed, cb, out + (size_t)t0 * M,
                                     tt, M, K, C, bits, st);
        if (rc) return rc;
    }
    return CK_SUCCESS;
}

template <int BITS>
int launch_emb_fast(const int32_t *ids, const uint8_t *packed, const float *cb, float *out,
                    int T, int vocab, int H, int C, hipStream_t st)
{
    dim3 grid((unsigned)((H / 32 + kBlock - 1) / kBlock), (unsigned)T);
    hipLaunchKernelGGL((fixed_embedding_kernel<BITS>), grid, dim3(kBlock), 0, st, ids,
                       (const uint32_t *)packed, cb, out, T, vocab, H, C);
    return cbq_launch_status("fixed_embedding_kernel");
}

int embedding_impl(const int32_t *ids, const uint8_t *packed, const float *cb, float *out,
                   int T, int vocab, int H, int C, int bits, hipStream_t st)
{
    if (!ids || !packed || !cb || !out) return CK_ERR_ARG;
    if (T <= 0 || H <= 0 || C <= 0 || bits < 1 || bits > 16) return CK_ERR_ARG;
    if (T > 65535) return CK_ERR_ARG;
    if (H % 32 == 0) {
        switch (bits) {
        case 8: return launch_emb_fast<8>(ids, packed, cb, out, T, vocab, H, C, st);
        case 12: return launch_emb_fast<12>(ids, packed, cb, out, T, vocab, H, C, st);
        case 13: return launch_emb_fast<13>(ids, packed, cb, out, T, vocab, H, C, st);
        case 14: return launch_emb_fast<14>(ids, packed, cb, out, T, vocab, H, C, st);
        case 16: return launch_emb_fast<16>(ids, packed, cb, out, T, vocab, H, C, st);
        default: break;
        }
    }
    dim3 grid((unsigned)((H + kBlock - 1) / kBlock), (unsigned)T);
    hipLaunchKernelGGL(fixed_embedding_generic_kernel, grid, dim3(kBlock), 0, st, ids,
                       packed, cb, out, T, vocab, H, C, bits);
    return cbq_launch_status("fixed_embedding_generic_kernel");
}

}  // namespace

// bf16 MFMA prefill path (cbq_prefill.hip); -1 = shape not handled there.
// ws (256-byte aligned, >= cbq_prefill_ws_bytes) holds x in fragment order
// and the split-K partials; without it x is read row-major and K not split.
int cbq_prefill_bf16(const uint16_t *x, const uint8_t *packed, const float *cb, uint16_t *out,
                     int T, int M, int K, int C, int bits, hipStream_t st, void *ws,
                     size_t ws_bytes);
size_t cbq_prefill_ws_bytes(int T, int M, int K);
// fp32 MFMA prefill path (cbq_prefill_f32.hip); -1 = shape not handled there.
int cbq_prefill_f32(const float *x, const uint8_t *packed, const float *cb, float *out, int T,
                    int M, int K, int C, int bits, hipStream_t st, int S, float *ws);
int cbq_prefill_f32_splits(int T, int M, int K);

int cbq_num_cus()
{
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cache[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

extern "C" {

const char *ck_error_string(int err)
{
    switch (err) {
    case CK_SUCCESS: return "success";
    case CK_ERR_HIP: return "HIP runtime error";
    case CK_ERR_ARG: return "invalid argument";
    default: return "unknown error";
    }
}

const char *cbq_version(void) { return "cbq_hip 0.1 gfx950"; }

int ck_linear_f32(const float *x, const uint8_t *packed, const float *codebook, float *out,
                  int T, int M, int K, int C, int bits, hipStream_t stream)
{
    // T >= 64: the GEMM regime, fp32 MFMA (cbq_prefill_f32.hip)
    if (x && packed && codebook && out && T >= 64 && M > 0 && K > 0 && C > 0 && bits >= 1 &&
        bits <= 16) {
        const int rc = cbq_prefill_f32(x, packed, codebook, out, T, M, K, C, bits, stream, 1,
                                       nullptr);
        if (rc >= 0) return rc;
    }
    return linear_any_t<float, float>(x, packed, codebook, out, T, M, K, C, bits, stream);
}

size_t cbq_linear_f32_workspace(int T, int M, int K)
{
    if (T <= 0 || M <= 0 || K <= 0) return 0;
    const int S = cbq_prefill_f32_splits(T, M, K);
    return S > 1 ? (size_t)S * T * M * sizeof(float) : 0;
}

int cbq_linear_f32_ws(const float *x, const uint8_t *packed, const float *codebook, float *out,
                      int T, int M, int K, int C, int bits, void *workspace, size_t ws_bytes,
                      hipStream_t stream)
{
    if (x && packed && codebook && out && T >= 64 && M > 0 && K > 0 && C > 0 && bits >= 1 &&
        bits <= 16) {
        const size_t need = cbq_linear_f32_workspace(T, M, K);
        const bool split = need > 0 && workspace && ws_bytes >= need &&
                           ((uintptr_t)workspace & 15) == 0;
        const int rc = cbq_prefill_f32(x, packed, codebook, out, T, M, K, C, bits, stream,
                                       split ? cbq_prefill_f32_splits(T, M, K) : 1,
                                       split ? (float *)workspace : nullptr);
        if (rc >= 0) return rc;
    }
    return ck_linear_f32(x, packed, codebook, out, T, M, K, C, bits, stream);
}

int cbq_linear_xform_f32(const float *x0, const float *x1, float *h_out, int mode, float eps,
                         const uint8_t *packed, const float *codebook, float *out, int M, int K,
                         int C, int bits, hipStream_t stream)
{
    if (!x0 || !packed || !codebook || !out || M <= 0 || K <= 0 || K % 32 != 0 || C <= 0 ||
        C > kMaxLdsCodebook)
        return CK_ERR_ARG;
    if (mode < XF_SILU || mode > XF_RMS || ((mode == XF_SILU || mode == XF_ADD_RMS) && !x1))
        return CK_ERR_ARG;
    // x is staged by GlueTile<.., 16>: 16 terms of 1024 virtual threads
    if (K > 16384) return CK_ERR_ARG;
    if (((uintptr_t)packed & 3) != 0) return CK_ERR_ARG;
    const int blocks =
        std::max(1, std::min(cbq_num_cus(), (M + kStreamWaves - 1) / kStreamWaves));
    size_t dyn = 0;
#define CBQ_XF(B, MODE, NJ)                                                                    \
    hipLaunchKernelGGL((fixed_stream_kernel<B, 1, float, float, false, MODE, false, false, NJ>), \
                       dim3(blocks), dim3(kStreamBlock),                                        \
                       dyn + (NJ == 4 ? kGlueScratchBytes : 0), stream, x0,                     \
                       (const uint32_t *)packed, codebook, out, 1, M, K, C, 0u, 0u, x1, h_out,  \
                       eps, K, 0, 0)
#define CBQ_XF_MODES(B)                                                                        \
    do {                                                                                       \
        dyn = stream_dyn_lds<B, float>(1, K, C);                                               \
        if (!dyn) return CK_ERR_ARG;                                                           \
        if (mode == XF_SILU) CBQ_XF(B, XF_SILU, 16);                                           \
        else if (mode == XF_ADD_RMS && K <= kGlueSmallK) CBQ_XF(B, XF_ADD_RMS, 4);             \
        else if (mode == XF_ADD_RMS) CBQ_XF(B, XF_ADD_RMS, 16);                                \
        else if (K <= kGlueSmallK) CBQ_XF(B, XF_RMS, 4);                                       \
        else CBQ_XF(B, XF_RMS, 16);                                                            \
    } while (0)
    switch (bits) {
    case 8: CBQ_XF_MODES(8); break;
    case 10: CBQ_XF_MODES(10); break;
    case 11: CBQ_XF_MODES(11); break;
    case 12: CBQ_XF_MODES(12); break;
    case 13: CBQ_XF_MODES(13); break;
    case 14: CBQ_XF_MODES(14); break;
    default: return CK_ERR_ARG;
    }
#undef CBQ_XF_MODES
#undef CBQ_XF
    return cbq_launch_status("fixed_stream_kernel<xform>");
}

int cbq_linear_xform_glu_f32(const float *x0, const float *x1, float *h_out, int mode,
                             float eps, const uint8_t *packed, const float *codebook, float *out,
                             int M, int K, int C, int bits, hipStream_t stream)
{
    if (!x0 || !packed || !codebook || !out || M <= 0 || M > (1 << 29) || K <= 0 ||
        K % 32 != 0 || C <= 0 || C > kMaxLdsCodebook)
        return CK_ERR_ARG;
    if (mode != XF_NONE && mode != XF_ADD_RMS && mode != XF_RMS) return CK_ERR_ARG;
    if ((mode == XF_ADD_RMS && !x1) || (mode != XF_NONE && K > 16384)) return CK_ERR_ARG;
    if (((uintptr_t)packed & 3) != 0 || ((uintptr_t)x0 & 3) != 0) return CK_ERR_ARG;
    const int blocks =
        std::max(1, std::min(cbq_num_cus(), (M + kStreamWaves - 1) / kStreamWaves));
    size_t dyn = 0;
#define CBQ_XG(B, MODE, NJ)                                                                    \
    hipLaunchKernelGGL((fixed_stream_kernel<B, 1, float, float, false, MODE, false, true, NJ>), \
                       dim3(blocks), dim3(kStreamBlock),                                        \
                       dyn + (NJ == 4 ? kGlueScratchBytes : 0), stream, x0,                     \
                       (const uint32_t *)packed, codebook, out, 1, M, K, C, 0u, 0u, x1, h_out,  \
                       eps, K, 0, 0)
#define CBQ_XG_MODES(B)                                                                        \
    do {                                                                                       \
        dyn = stream_dyn_lds<B, float>(1, K, C);                                               \
        if (!dyn) return CK_ERR_ARG;                                                           \
        if (mode == XF_ADD_RMS && K <= kGlueSmallK) CBQ_XG(B, XF_ADD_RMS, 4);                  \
        else if (mode == XF_ADD_RMS) CBQ_XG(B, XF_ADD_RMS, 16);                                \
        else if (mode == XF_RMS && K <= kGlueSmallK) CBQ_XG(B, XF_RMS, 4);                     \
        else if (mode == XF_RMS) CBQ_XG(B, XF_RMS, 16);                                        \
        else CBQ_XG(B, XF_NONE, 16);                                                           \
    } while (0)
    switch (bits) {
    case 8: CBQ_XG_MODES(8); break;
    case 10: CBQ_XG_MODES(10); break;
    case 11: CBQ_XG_MODES(11); break;
    case 12: CBQ_XG_MODES(12); break;
    case 13: CBQ_XG_MODES(13); break;
    case 14: CBQ_XG_MODES(14); break;
    default: return CK_ERR_ARG;
    }
#undef CBQ_XG_MODES
#undef CBQ_XG
    return cbq_launch_status("fixed_stream_kernel<glu>");
}

int cbq_linear_xform_argmax_f32(const float *x0, const float *x1, float *h_out, int mode,
                                float eps, const uint8_t *packed, const float *codebook,
                                float *out, int M, int K, int C, int bits, void *workspace,
                                size_t workspace_bytes, int32_t *ids32, int64_t *toks,
                                int64_t *pos, int64_t first, int64_t n_toks, hipStream_t stream)
{
    if (!x0 || !packed || !codebook || M <= 0 || K <= 0 || K % 32 != 0 || C <= 0 ||
        C > kMaxLdsCodebook || !workspace || !ids32 || !toks || !pos || n_toks <= 0)
        return CK_ERR_ARG;
    if (mode < XF_NONE || mode > XF_RMS || ((mode == XF_SILU || mode == XF_ADD_RMS) && !x1))
        return CK_ERR_ARG;
    if (mode != XF_NONE && K > 16384) return CK_ERR_ARG;   // GlueTile<.., 16> covers 16384
    if (((uintptr_t)packed & 3) != 0 || ((uintptr_t)x0 & 3) != 0 ||
        ((uintptr_t)workspace & 3) != 0 || workspace_bytes < CBQ_ARGMAX_WORKSPACE)
        return CK_ERR_ARG;
    const int blocks =
        std::max(1, std::min(cbq_num_cus(), (M + kStreamWaves - 1) / kStreamWaves));
    if (blocks > kArgMaxParts) return CK_ERR_ARG;
    float *part_v = (float *)workspace;
    int *part_i = (int *)(part_v + kArgMaxParts);
    size_t dyn = 0;
#define CBQ_XA(B, MODE, NJ)                                                                    \
    hipLaunchKernelGGL((fixed_stream_kernel<B, 1, float, float, false, MODE, false, false, NJ>), \
                       dim3(blocks), dim3(kStreamBlock),                                        \
                       dyn + (NJ == 4 ? kGlueScratchBytes : 0), stream, x0,                     \
                       (const uint32_t *)packed, codebook, out, 1, M, K, C, 0u, 0u, x1, h_out,  \
                       eps, K, 0, 0, part_v, part_i)
#define CBQ_XA_MODES(B)                                                                        \
    do {                                                                                       \
        dyn = stream_dyn_lds<B, float>(1, K, C);                                               \
        if (!dyn) return CK_ERR_ARG;                                                           \
        if (mode == XF_SILU) CBQ_XA(B, XF_SILU, 16);                                           \
        else if (mode == XF_ADD_RMS && K <= kGlueSmallK) CBQ_XA(B, XF_ADD_RMS, 4);             \
        else if (mode == XF_ADD_RMS) CBQ_XA(B, XF_ADD_RMS, 16);                                \
        else if (mode == XF_RMS && K <= kGlueSmallK) CBQ_XA(B, XF_RMS, 4);                     \
        else if (mode == XF_RMS) CBQ_XA(B, XF_RMS, 16);                                        \
        else CBQ_XA(B, XF_NONE, 16);                                                           \
    } while (0)
    switch (bits) {
    case 8: CBQ_XA_MODES(8); break;
    case 10: CBQ_XA_MODES(10); break;
    case 11: CBQ_XA_MODES(11); break;
    case 12: CBQ_XA_MODES(12); break;
    case 13: CBQ_XA_MODES(13); break;
    case 14: CBQ_XA_MODES(14); break;
    default: return CK_ERR_ARG;
    }
#undef CBQ_XA_MODES
#undef CBQ_XA
    const int rc = cbq_launch_status("fixed_stream_kernel<argmax>");
    if (rc) return rc;
    return cbq_argmax_merge(part_v, part_i, blocks, M, ids32, toks, pos, first, n_toks, stream);
}

int cbq_linear_affine_f32(const float *x, const uint8_t *packed, uint32_t lo, uint32_t w,
                          float *out, int T, int M, int K, int bits, hipStream_t stream)
{
    if (!x || !packed || !out || T <= 0 || M <= 0 || K <= 0 || K % 32 != 0) return CK_ERR_ARG;
    if (((uintptr_t)x & 3) || ((uintptr_t)packed & 3)) return CK_ERR_ARG;
    if (w == 0 || lo == 0 || lo + w > 0x8000u || 2ull * w > (1ull << bits)) return CK_ERR_ARG;
    for (int t0 = 0; t0 < T; t0 += 16) {
        const int tt = std::min(16, T - t0);
        const float *xt = x + (size_t)t0 * K;
        float *ot = out + (size_t)t0 * M;
        int rc;
        switch (bits) {
        case 8: rc = dispatch_affine<8>(xt, packed, lo, w, ot, tt, M, K, stream); break;
        case 10: rc = dispatch_affine<10>(xt, packed, lo, w, ot, tt, M, K, stream); break;
        case 11: rc = dispatch_affine<11>(xt, packed, lo, w, ot, tt, M, K, stream); break;
        case 12: rc = dispatch_affine<12>(xt, packed, lo, w, ot, tt, M, K, stream); break;
        case 13: rc = dispatch_affine<13>(xt, packed, lo, w, ot, tt, M, K, stream); break;
        case 14: rc = dispatch_affine<14>(xt, packed, lo, w, ot, tt, M, K, stream); break;
        default: return CK_ERR_ARG;
        }
        if (rc) return rc;
    }
    return CK_SUCCESS;
}

int ck_linear_bf16(const void *x_bf16, const uint8_t *packed, const float *codebook,
                   void *out_bf16, int T, int M, int K, int C, int bits, hipStream_t stream)
{
    // T >= 64: the GEMM regime, bf16 MFMA with fp32 accumulation (cbq_prefill.hip)
    if (x_bf16 && packed && codebook && out_bf16 && T >= 64 && M > 0 && K > 0 && C > 0 &&
        bits >= 1 && bits <= 16) {
        const int rc = cbq_prefill_bf16((const uint16_t *)x_bf16, packed, codebook,
                                        (uint16_t *)out_bf16, T, M, K, C, bits, stream, nullptr,
                                        0);
        if (rc >= 0) return rc;
    }
    return linear_any_t<uint16_t, uint16_t>((const uint16_t *)x_bf16, packed, codebook,
                                            (uint16_t *)out_bf16, T, M, K, C, bits, stream);
}

size_t cbq_linear_bf16_workspace(int T, int M, int K)
{
    if (T <= 0 || M <= 0 || K <= 0) return 0;
    return cbq_prefill_ws_bytes(T, M, K);
}

int cbq_linear_bf16_ws(const void *x_bf16, const uint8_t *packed, const float *codebook,
                       void *out_bf16, int T, int M, int K, int C, int bits, void *workspace,
                       size_t ws_bytes, hipStream_t stream)
{
    if (x_bf16 && packed && codebook && out_bf16 && T >= 64 && M > 0 && K > 0 && C > 0 &&
        bits >= 1 && bits <= 16) {
        // workspace = [x in fragment order][fp32 split partials]; a smaller one
        // runs as ck_linear_bf16
        const int rc = cbq_prefill_bf16((const uint16_t *)x_bf16, packed, codebook,
                                        (uint16_t *)out_bf16, T, M, K, C, bits, stream, workspace,
                                        ws_bytes);
        if (rc >= 0) return rc;
    }
    return ck_linear_bf16(x_bf16, packed, codebook, out_bf16, T, M, K, C, bits, stream);
}

int ck_embedding_f32(const int32_t *token_ids, const uint8_t *packed, const float *codebook,
                     float *out, int T, int H, int C, int bits, hipStream_t stream)
{
    return embedding_impl(token_ids, packed, codebook, out, T, 0, H, C, bits, stream);
}

int cbq_embedding_f32(const int32_t *token_ids, const uint8_t *packed, const float *codebook,
                      float *out, int T, int vocab, int H, int C, int bits,
                      hipStream_t stream)
{
    if (vocab <= 0) return CK_ERR_ARG;
    return embedding_impl(token_ids, packed, codebook, out, T, vocab, H, C, bits, stream);
}

}  // extern "C"

// Per-wave timeline of the last one-token plain streaming launch, in a
// -DCBQ_TIMELINE build: kTimelineWaves x 6 uint64 (entry, staged, first
// ring done, loop done, exit in 10 ns ticks; item count).  CK_ERR_ARG in
// the product build or when dst_bytes is short.
extern "C" int cbq_timeline_read(void *dst, size_t dst_bytes)
{
#ifdef CBQ_TIMELINE
    const size_t n = sizeof(unsigned long long) * kTimelineWaves * kTimelineFields;
    if (!dst || dst_bytes < n) return CK_ERR_ARG;
    const hipError_t e = hipMemcpyFromSymbol(dst, HIP_SYMBOL(cbq_timeline_wave), n, 0,
                                             hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        fprintf(stderr, "cbq_timeline_read: %s\n", hipGetErrorString(e));
        return CK_ERR_HIP;
    }
    return CK_SUCCESS;
#else
    (void)dst;
    (void)dst_bytes;
    return CK_ERR_ARG;
#endif
}
