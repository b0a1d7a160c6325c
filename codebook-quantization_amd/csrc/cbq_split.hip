// Split device format and its one-token GEMV, for gfx950.
//
// The canonical-Huffman index stream of the reference
// (src/huffman_codebook.py:126-226) spends ~10.5 bits per weight, and its
// decode is a chain of three dependent table reads per symbol.  When every
// codebook value is a bf16 number (the lossless direct-codebook mode), the
// same weights can be held instead as
//
//   raw   one byte per weight: the low byte of its bf16 bits (exponent bit 0
//         and the 7 mantissa bits);
//   code  the high byte (sign and exponent bits 7..1), Huffman-coded with
//         codes of at most 7 bits (~2.9 bits per weight on N(0, sigma)
//         weights),
//
// built once at load from the decoded indices.  The codes of each 64-weight
// sub-block form an LSB-first bit stream stored in the column layout: chunk
// c (4096 weights, 64 sub-blocks) owns rows row_off[c] .. row_off[c+1]-1 of
// 64 words, word l of a row belonging to sub-block l, so a wave reads a row
// with one conflict-free LDS access.  Codes have at most 7 bits, so any 14
// stream bits hold the next two codes whole: a 16384-entry table (64 KiB of
// LDS) maps them to hi1 << 24 | hi2 << 16 | (len1 + len2), and one v_perm
// assembles a weight's fp32 bits from its table byte and its raw byte: one
// table read per two weights and ~4.5 VALU operations per weight.
//
// The GEMV walks a chunk exactly as the column-layout Huffman GEMV does (lane
// l takes sub-block l, symbols in order, fmaf into one accumulator, wave sum
// per chunk, chunks of a row added in order), so the two give identical
// outputs on the same weights and x.
#include "cbq_device.h"

#include <algorithm>

namespace {

constexpr int kSChunk = 4096;
constexpr int kSSub = 64;
constexpr int kSMaxLen = 7;                       // code length limit
constexpr int kSLut = 1 << (2 * kSMaxLen);        // two-code table entries
// A chunk has at most ceil(64 * 7 / 32) = 14 rows; the slot holds two more,
// since the decoder reads up to two rows past a sub-block's last code.
constexpr int kSRows = 14;
constexpr int kSSlotRows = 16;
constexpr int kSSlotWords = kSSlotRows * kSSub;   // one wave's chunk slot
constexpr int kSMaxSeg = 4;

// Diagnostic build (-DCBQ_TIMELINE): wave w of block b of a split_gemv_kernel
// launch records the 100 MHz s_memrealtime clock at entry, after the first
// barrier (table, x tile and the first chunk's offsets staged), after its
// first chunk is decoded, after its row loop and at exit, plus its rows, in
// cbq_split_timeline[b * NW + w] (read by cbq_split_timeline_read).  The
// product build has none of it.
constexpr int kSplitTimelineWaves = 4096;
constexpr int kSplitTimelineFields = 6;
#ifdef CBQ_TIMELINE
__device__ unsigned long long cbq_split_timeline[kSplitTimelineWaves * kSplitTimelineFields];
#endif

constexpr int split_lds_words(int nw) { return kSLut + kSChunk + nw * kSSlotWords; }

struct SplitSeg {
    const uint32_t *cwords;
    const uint32_t *row_off;
    const uint8_t *raw;
    const uint32_t *lut;
    float *out;
    int M;
    int block0;
    int nblocks;
};
struct SplitSegs {
    SplitSeg s[kSMaxSeg];
    int n;
};

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// One item's global data in registers: the 64 raw bytes of this lane's
// sub-block, and the chunk's code rows 0 .. H-1 (rounded up to 4) as 16-byte
// pieces: piece k of lane l is row 4k + l/16, words 4(l%16) .. 4(l%16)+3.
struct SplitItem {
    uint32_t raw[16];
    u4 ew[(kSRows + 3) / 4];
};

__device__ __forceinline__ void split_load(SplitItem &it, const SplitSeg &S, int64_t c, uint32_t r0,
                                           uint32_t H, int lane)
{
    const u4 *rp = (const u4 *)(S.raw + (size_t)c * kSChunk + lane * kSSub);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const u4 v = rp[k];
        it.raw[4 * k] = v.x;
        it.raw[4 * k + 1] = v.y;
        it.raw[4 * k + 2] = v.z;
        it.raw[4 * k + 3] = v.w;
    }
    // Piece 0 unconditionally (a chunk holds at least two code rows: 64
    // codes of at least one bit), so the wait for it, which covers the raw
    // loads issued before it, is on every path.
    const u4 *wp = (const u4 *)(S.cwords + (size_t)r0 * kSSub) + lane;
#pragma unroll
    for (int k = 0; k < (kSRows + 3) / 4; k++)
        if (k == 0 || 4 * k < (int)H) it.ew[k] = wp[k * kSSub];
}

// split_load with every load issued (4 + (kSRows + 3) / 4 of them): code
// pieces past the item's last one re-load that piece (an address split_load
// reads too), so the count does not depend on H and a wait can leave these
// loads in flight while everything issued before them has landed.
__device__ __forceinline__ void split_load_all(SplitItem &it, const SplitSeg &S, int64_t c,
                                               uint32_t r0, uint32_t H, int lane)
{
    const u4 *rp = (const u4 *)(S.raw + (size_t)c * kSChunk + lane * kSSub);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const u4 v = rp[k];
        it.raw[4 * k] = v.x;
        it.raw[4 * k + 1] = v.y;
        it.raw[4 * k + 2] = v.z;
        it.raw[4 * k + 3] = v.w;
    }
    const u4 *wp = (const u4 *)(S.cwords + (size_t)r0 * kSSub) + lane;
    const int klast = H > 0 ? (int)((H - 1) >> 2) : 0;
#pragma unroll
    for (int k = 0; k < (kSRows + 3) / 4; k++) it.ew[k] = wp[(k < klast ? k : klast) * kSSub];
}

// Writes an item's code rows into the wave's slot (same row-major layout).
__device__ __forceinline__ void split_stage(const SplitItem &it, uint32_t H, uint32_t *s_slot,
                                            int lane)
{
#pragma unroll
    for (int k = 0; k < (kSRows + 3) / 4; k++)
        if (k == 0 || 4 * k < (int)H) *(u4 *)(s_slot + k * 4 * kSSub + 4 * lane) = it.ew[k];
}

// split_stage of an item loaded by split_load_all, every piece written (the
// slot's rows past the item's last code row hold copies of its last piece,
// which the decoder reads past the end of a sub-block's codes and never
// consumes): every load of the item is waited for on every path.
__device__ __forceinline__ void split_stage_all(const SplitItem &it, uint32_t *s_slot, int lane)
{
#pragma unroll
    for (int k = 0; k < (kSRows + 3) / 4; k++)
        *(u4 *)(s_slot + k * 4 * kSSub + 4 * lane) = it.ew[k];
}

// Decodes the 64 weights of this lane's sub-block against the staged x and
// returns the dot product.  s_lds: the two-code table at LDS address 0 and
// this wave's slot (already written); lane_addr: byte address of the lane's
// column in row 0 of the slot.  A group of 4 codes spans at most 28 bits, so
// the next group's window starts in the current word or the one after it:
// the words (d, d+1) of the current window and word d+2, read one group
// ahead, stay in registers and the table reads are the only LDS accesses on
// the dependent chain.
//
// The stream position is kept as the plain sum of the table entries read
// (plus a bias of 32): an entry's bits 8..15 are zero, so bits 0..15 of the
// sum are the bits consumed so far (at most 64 * 7 + 32 < 2^16) and the
// hi-byte fields only pile up above them.  Shifts use bits 0..4 of their
// amount, so no masking is needed between the table read and the next
// window.
__device__ __forceinline__ float split_decode(const uint32_t (&raw)[16], const uint32_t *s_lds,
                                              int lane_addr, const float *xr, int xsw)
{
    float acc = 0.f;
    uint32_t pos = 30;                                // (stream bit position - 2) + 32
    uint32_t d1 = 0;                                  // (word of bit position - 2) + 1
    const char *base = (const char *)s_lds + lane_addr;
    uint32_t w0 = *(const uint32_t *)(base - 4 * kSSub);
    uint32_t w1 = *(const uint32_t *)base;
#pragma unroll
    for (int g = 0; g < 16; g++) {
        const uint32_t w2 = *(const uint32_t *)(base + (d1 + 1) * (4 * kSSub));
        const f4 xv4 = *(const f4 *)(xr + ((4 * g) ^ xsw));
        const float xv[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
        uint32_t w = __builtin_amdgcn_alignbit(w1, w0, pos);   // 30 bits in 2..31
#pragma unroll
        for (int u = 0; u < 4; u += 2) {
            const uint32_t e = *(const uint32_t *)((const char *)s_lds + (w & (4u * kSLut - 4u)));
            // weight = high byte from the table entry | raw low byte, << 16
            const uint32_t v0 = __builtin_amdgcn_perm(e, raw[g], 0x07000c0cu | (u << 16));
            const uint32_t v1 = __builtin_amdgcn_perm(e, raw[g], 0x06000c0cu | ((u + 1) << 16));
            acc = fmaf(xv[u], __uint_as_float(v0), acc);
            acc = fmaf(xv[u + 1], __uint_as_float(v1), acc);
            w >>= (e & 31u);
            pos += e;
        }
        const uint32_t dn = __builtin_amdgcn_ubfe(pos, 5, 11);   // d1 or d1 + 1
        w0 = dn != d1 ? w1 : w0;
        w1 = dn != d1 ? w2 : w1;
        d1 = dn;
    }
    return acc;
}

// Row groups: the flat symbol stream is cut into 4096-symbol chunks, so with
// K % 4096 != 0 a chunk holds parts of several rows.  The GEMV therefore
// walks groups of GR = 4096 / gcd(K, 4096) rows, which are exactly
// R = GR * K / 4096 whole chunks; chunk p of every group covers the same x
// columns, (p * 4096 + i) mod K, so the block stages one 4096-float x tile
// per phase p as before.  Lane l's sub-block lies in row (p * 4096 + 64 l) / K
// of the group (K % 64 == 0), and a chunk's dot products are summed per row
// with masked wave sums.  GR = 1 (K % 4096 == 0) is the plain row walk.
//
// GLU (GR = 1, one segment): the segment's matrix holds 2M rows, gate rows
// [0, M) then up rows [M, 2M), under one code table; a wave takes gate row j
// and up row j as consecutive items and writes out[j] = silu(gate_j . x) *
// (up_j . x), rounded as silu_mul_value, so the down projection stages
// plain x.  Each product sums exactly as the plain launch does.
template <int NW, int XMODE, int GR, int NJ = 16, bool GLU = false>
__global__ __launch_bounds__(NW * CBQ_WAVE) void split_gemv_kernel(const float *__restrict__ x,
                                                                   SplitSegs segs, int K,
                                                                   const float *__restrict__ x1,
                                                                   float *__restrict__ h_out,
                                                                   float eps,
                                                                   float *__restrict__ arg_v,
                                                                   int *__restrict__ arg_i)
{
    static_assert(!GLU || (GR == 1 && XMODE != XF_SILU), "gate/up pairs: whole-chunk rows");
    constexpr int NI = GLU ? 2 : 1;                    // items per output row
    int sidx = 0;
#pragma unroll
    for (int i = 1; i < kSMaxSeg; i++)
        if (i < segs.n && (int)blockIdx.x >= segs.s[i].block0) sidx = i;
    const SplitSeg &S = segs.s[sidx];
    const int M = S.M;
    const int bid = (int)blockIdx.x - S.block0;
    __shared__ __attribute__((aligned(16))) uint32_t s_lds[split_lds_words(NW)];
    float *const s_x = (float *)(s_lds + kSLut);
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / CBQ_WAVE);
#ifdef CBQ_TIMELINE
    const unsigned long long ts_entry = __builtin_amdgcn_s_memrealtime();
    unsigned long long ts_staged = 0, ts_first = 0;
#endif
    uint32_t *const s_slot = s_lds + kSLut + kSChunk + wave * kSSlotWords;
    const int lane_addr =
        __builtin_amdgcn_readfirstlane(4 * (kSLut + kSChunk + wave * kSSlotWords)) + 4 * lane;

    const int R = K * GR / kSChunk;                    // chunks per row group
    const int Mg = M / GR;                              // row groups
    // Wave w of block b is walker w nblocks + pos and takes rows (groups)
    // wid, wid + W, ...: when the rows do not divide evenly, the extra ones
    // go to the low waves of every block, not to every wave of the low
    // blocks, so no CU holds more than its share plus one row per wave.
    // pos numbers the blocks XCD by XCD (blocks b and b + 8 share one), so
    // neighbouring rows are read and written through one L2: a chunk's code
    // pieces past its last row and an output line stay in that XCD.
    const int nbk = S.nblocks;
    const int xu = bid & 7;
    const int pos = xu * (nbk >> 3) + min(xu, nbk & 7) + (bid >> 3);
    const int W = nbk * NW;
    const int wid = wave * nbk + pos;
    const int rows = wid < Mg ? (Mg - wid + W - 1) / W : 0;
    const int rows_max = pos < Mg ? (Mg - pos + W - 1) / W : 0;   // wave 0's
    const int n_seg = (rows_max + 63) >> 6;
    const float *const xr = s_x + lane * 64;
    const int xsw = (lane & 15) << 2;
    auto chunk_of = [&](int seg, int p, int b, uint32_t &r0, uint32_t &H) {
        // item b: output row seg * 64 + b / NI of this wave (GLU: odd b the up row)
        const int64_t row = wid + (int64_t)(seg * 64 + b / NI) * W + (GLU && (b & 1) ? M : 0);
        const int64_t c = __builtin_amdgcn_readfirstlane((int)(row * R + p));
        r0 = S.row_off[c];
        H = S.row_off[c + 1] - r0;
        H = H < (uint32_t)kSRows ? H : (uint32_t)kSRows;
        return c;
    };

    GlueTile<NW * CBQ_WAVE, XMODE == XF_SILU ? XF_NONE : XMODE, NJ> tile;   // K <= 1024 NJ
    if constexpr (XMODE == XF_ADD_RMS || XMODE == XF_RMS) tile.load(x, x1, K);
    // Two items in flight: the next one's loads go out before this one is
    // decoded.  The wave's first item is requested before the table staging.
    SplitItem A, B;
    uint32_t rA = 0, hA = 0, rB = 0, hB = 0;
    // The first chunk's row offsets are requested first, its data last:
    // lanes 0 and 1 read row_off[c0] and row_off[c0 + 1] (a wave without
    // rows reads chunk 0's, unused); the table and x loads go out while they
    // return, and the first barrier waits for those alone.
    const int64_t c0 = rows > 0 ? (int64_t)__builtin_amdgcn_readfirstlane(wid * R) : 0;
    const uint32_t v_off0 = S.row_off[c0 + (lane & 1)];
    for (int i = wave; i < kSLut / (4 * CBQ_WAVE); i += NW)
        __builtin_amdgcn_global_load_lds(S.lut + i * 4 * CBQ_WAVE + 4 * lane,
                                         (__attribute__((address_space(3))) void *)(s_lds + i * 4 * CBQ_WAVE),
                                         16, 0, 0);
    // Plain x: the first x tile (seg 0, phase 0) goes to LDS together with
    // the table, so the first barrier waits for one round trip of both
    // instead of the tile's loads following it.
    constexpr bool kXDma = XMODE == XF_NONE;
    if (kXDma && rows_max > 0) {                   // (the block then reaches the barrier)
        if (((uintptr_t)x & 15) == 0) {
            // 16-byte pieces: chunk c of row r holds x chunk c ^ (r & 15) of
            // that row; one load covers 4 rows
            for (int i = wave; i < 16; i += NW) {
                const int r = (i << 2) + (lane >> 4), c = lane & 15;
                int t = (r << 6) + ((c ^ (r & 15)) << 2);
                if constexpr (GR > 1) t %= K;
                __builtin_amdgcn_global_load_lds(
                    x + t, (__attribute__((address_space(3))) void *)(s_x + (i << 8)), 16, 0, 0);
            }
        } else {
            for (int r = wave; r < 64; r += NW) {
                int t = (r << 6) + (lane ^ ((r & 15) << 2));
                if constexpr (GR > 1) t %= K;
                __builtin_amdgcn_global_load_lds(
                    x + t, (__attribute__((address_space(3))) void *)(s_x + (r << 6)), 4, 0, 0);
            }
        }
    }
    // SiLU product: the first tile's inputs are read into registers now
    // (their loads overlap the table's) and multiplied after the barrier.
    // The norms with whole-chunk rows write the first tile from the glue
    // registers (the normalised x, already in this thread) before it.
    constexpr bool kXRegs = XMODE == XF_SILU;
    constexpr bool kXTile = (XMODE == XF_ADD_RMS || XMODE == XF_RMS) && GR == 1;
    constexpr int kXR = kXRegs ? 64 / NW : 1;      // tile rows per wave
    float x0r[kXR], x1r[kXR];
    if (kXRegs && rows_max > 0) {
#pragma unroll
        for (int i = 0; i < kXR; i++) {
            const int r = wave + i * NW;
            int t = (r << 6) + (lane ^ ((r & 15) << 2));
            if constexpr (GR > 1) t %= K;
            x0r[i] = x[t];
            x1r[i] = x1[t];
        }
    }
    // the first chunk: exactly kFirstLoads loads, issued after every other
    // load of the prologue
    constexpr int kFirstLoads = 4 + (kSRows + 3) / 4;
    __builtin_amdgcn_sched_barrier(0);
    rA = __builtin_amdgcn_readfirstlane(v_off0);
    hA = __builtin_amdgcn_readlane(v_off0, 1) - rA;
    hA = hA < (uint32_t)kSRows ? hA : (uint32_t)kSRows;
    split_load_all(A, S, c0, rA, hA, lane);
    __builtin_amdgcn_sched_barrier(0);
    float xr_scale = 1.f;
    const bool store_h = XMODE == XF_ADD_RMS && blockIdx.x == 0 && h_out != nullptr;
    if constexpr (XMODE == XF_ADD_RMS || XMODE == XF_RMS) {
        // the norm's 16 wave sums go to wave 0's code slot (first written
        // two barriers later), so the first x tile can be written at once
        xr_scale = tile.finish(K, eps, kXTile ? (float *)(s_lds + kSLut + kSChunk) : s_x);
        if constexpr (kXTile) {
            // element i = tid + k NW*64 + 1024 j (< 4096) goes to the slot
            // the staging loop below gives it
#pragma unroll
            for (int k = 0; k < tile.VPT; k++)
#pragma unroll
                for (int j = 0; j < kSChunk / 1024; j++) {
                    const int i = (int)threadIdx.x + k * NW * CBQ_WAVE + j * 1024;
                    const int r = i >> 6;
                    s_x[(r << 6) + ((i & 63) ^ ((r & 15) << 2))] = tile.value(k, j, xr_scale);
                }
            if (store_h) tile.store_sum(h_out, K);
        }
    }
    float a_best = -INFINITY;                      // greedy-pick candidate of this lane
    int a_idx = kArgNone;

    for (int seg = 0; seg < n_seg; seg++) {
        float res[GR];
#pragma unroll
        for (int q = 0; q < GR; q++) res[q] = 0.f;
        float res_u = 0.f;                         // GLU: up sums, lane = row % 64
        const int seg_rows = min(64, rows - seg * 64);
        const int seg_items = seg_rows * NI;
        for (int p = 0; p < R; p++) {
            if (seg == 0 && p == 0) {
                // every prologue load but the first chunk's has landed (they
                // were issued before it); the first chunk stays in flight
                __builtin_amdgcn_s_waitcnt((kFirstLoads & 15) | (7 << 4) | (15 << 8) |
                                           ((kFirstLoads >> 4) << 14));
                lds_barrier();
#ifdef CBQ_TIMELINE
                ts_staged = __builtin_amdgcn_s_memrealtime();
#endif
            } else {
                __syncthreads();
            }
            if (seg == 0 && p == 0 && (kXDma || kXRegs || kXTile)) {
                // first tile: DMA'd with the table, written already, or from registers
                if constexpr (kXRegs) {
#pragma unroll
                    for (int i = 0; i < kXR; i++) {
                        const int r = wave + i * NW;
                        int t = (r << 6) + (lane ^ ((r & 15) << 2));
                        if constexpr (GR > 1) t %= K;
                        s_x[(r << 6) + lane] =
                            xform_of(XMODE, x0r[i], x1r[i], h_out, store_h, t, xr_scale);
                    }
                }
            } else {
                // a wave's 64 / NW rows of the tile: every load first, then
                // the transforms and stores (one round trip, not one per row)
                constexpr int kRows = 64 / NW;
                constexpr bool kTwoIn = XMODE == XF_SILU || XMODE == XF_ADD_RMS;
                float a0[kRows], a1[kRows];
#pragma unroll
                for (int i = 0; i < kRows; i++) {
                    const int r = wave + i * NW;
                    int t = p * kSChunk + (r << 6) + (lane ^ ((r & 15) << 2));
                    if constexpr (GR > 1) t %= K;
                    a0[i] = x[t];
                    a1[i] = kTwoIn ? x1[t] : 0.f;
                }
#pragma unroll
                for (int i = 0; i < kRows; i++) {
                    const int r = wave + i * NW;
                    int t = p * kSChunk + (r << 6) + (lane ^ ((r & 15) << 2));
                    if constexpr (GR > 1) t %= K;
                    s_x[(r << 6) + lane] = XMODE == XF_NONE
                                               ? a0[i]
                                               : xform_of(XMODE, a0[i], a1[i], h_out, store_h, t,
                                                          xr_scale);
                }
            }
            __syncthreads();
            // rows of the group that chunk p touches, and this lane's row
            const int q_lo = p * kSChunk / K, q_hi = (p * kSChunk + kSChunk - 1) / K;
            const int q_me = (p * kSChunk + lane * kSSub) / K;
            auto add_rows = [&](float acc, int b) {
                if constexpr (GLU) {
                    const float s = wave_sum(acc);
                    if (lane == (b >> 1)) {
                        if (b & 1) res_u += s;
                        else res[0] += s;
                    }
                } else if constexpr (GR == 1) {
                    const float s = wave_sum(acc);
                    if (lane == b) res[0] += s;
                } else {
#pragma unroll
                    for (int q = 0; q < GR; q++)
                        if (q >= q_lo && q <= q_hi) {
                            const float s = wave_sum(q_me == q ? acc : 0.f);
                            if (lane == b) res[q] += s;
                        }
                }
            };
            // The slot is rewritten only after the previous item's reads (LDS
            // operations of a wave complete in order).  The next item's loads
            // go out after this one is staged: the wait the staging needs
            // (for loads issued on some paths only) then comes before them,
            // and the decode runs with them in flight.
            if (seg_items > 0 && (seg > 0 || p > 0)) {
                const int64_t c = chunk_of(seg, p, 0, rA, hA);
                split_load(A, S, c, rA, hA, lane);
            }
            for (int b = 0; b < seg_items; b += 2) {
                split_stage(A, hA, s_slot, lane);
                if (b + 1 < seg_items) {
                    const int64_t c = chunk_of(seg, p, b + 1, rB, hB);
                    split_load(B, S, c, rB, hB, lane);
                }
                add_rows(split_decode(A.raw, s_lds, lane_addr, xr, xsw), b);
#ifdef CBQ_TIMELINE
                if (seg == 0 && p == 0 && b == 0) ts_first = __builtin_amdgcn_s_memrealtime();
#endif
                if (b + 1 >= seg_items) break;
                split_stage(B, hB, s_slot, lane);
                if (b + 2 < seg_items) {
                    const int64_t c = chunk_of(seg, p, b + 2, rA, hA);
                    split_load(A, S, c, rA, hA, lane);
                }
                add_rows(split_decode(B.raw, s_lds, lane_addr, xr, xsw), b + 1);
            }
        }
        if (GLU && lane < seg_rows) {
            const int64_t g = wid + (int64_t)(seg * 64 + lane) * W;
            S.out[g] = silu_mul_value(res[0], res_u);
        } else if (!GLU && lane < seg_rows) {
            const int64_t g = wid + (int64_t)(seg * 64 + lane) * W;
#pragma unroll
            for (int q = 0; q < GR; q++) {
                if (S.out) S.out[g * GR + q] = res[q];
                if (arg_v && arg_better(res[q], (int)(g * GR + q), a_best, a_idx)) {
                    a_best = res[q];
                    a_idx = (int)(g * GR + q);
                }
            }
        }
    }
#ifdef CBQ_TIMELINE
    const unsigned long long ts_loop = __builtin_amdgcn_s_memrealtime();
#endif
    if (arg_v) {                                   // one matrix per launch (checked on the host)
        __shared__ float s_av[NW];
        __shared__ int s_ai[NW];
        arg_block_store(a_best, a_idx, s_av, s_ai, arg_v, arg_i);
    }
#ifdef CBQ_TIMELINE
    const unsigned long long ts_exit = __builtin_amdgcn_s_memrealtime();
    const int twid = (int)blockIdx.x * NW + wave;
    if (lane == 0 && twid < kSplitTimelineWaves) {
        unsigned long long *tl = cbq_split_timeline + (size_t)twid * kSplitTimelineFields;
        tl[0] = ts_entry;
        tl[1] = ts_staged;
        tl[2] = ts_first;
        tl[3] = ts_loop;
        tl[4] = ts_exit;
        tl[5] = (unsigned long long)rows;
    }
#endif
}

// Rows or row groups of several chunks (R = K GR / 4096 > 1: K = 3072,
// 5120, 6144, 7168 in groups, K = 8192, 12288 as whole rows), plain x, one
// matrix.  split_gemv_kernel walks a group's R chunks in one wave, one x
// tile per chunk, with a barrier and the next tile's staging between them.
// Here the whole x is staged once (K <= rg_max_k(NW), in the tile's
// swizzled 64-float rows) and the R chunks of a group go to R waves: the
// block holds GPB R waves (<= NW), and wave (gl, p) = gl R + p decodes chunk
// p of the block's groups gl, gl + GPB, gl + 2 GPB, ... one after another,
// the next one's loads in flight while one is decoded.  The wave sums of a
// chunk's rows (at most two rows: K is a multiple of 1024 and at least
// 3072) stay in the register of lane (item mod 64).  After every 64 items
// the waves write them to their slots, and after a barrier one thread per
// output row adds them in chunk order.  That is the order in which
// split_gemv_kernel adds its chunks' wave sums, over the same per-lane dot
// products, so the outputs are equal bit for bit.  LDS: the table, x and NW
// slots fill the 160 KiB.
constexpr int kRgLdsWords = 40960;
constexpr int rg_max_k(int nw) { return kRgLdsWords - kSLut - nw * kSSlotWords; }

template <int NW>
__global__ __launch_bounds__(NW * CBQ_WAVE) void split_gemv_rg_kernel(const float *__restrict__ x,
                                                                      SplitSeg S, int K, int GR,
                                                                      int R, int GPB)
{
    constexpr int kMaxK = rg_max_k(NW);
    __shared__ __attribute__((aligned(16))) uint32_t s_lds[kRgLdsWords];
    float *const s_x = (float *)(s_lds + kSLut);
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / CBQ_WAVE);
    uint32_t *const s_slots = s_lds + kSLut + kMaxK;
    uint32_t *const s_slot = s_slots + wave * kSSlotWords;
    const int lane_addr =
        __builtin_amdgcn_readfirstlane(4 * (kSLut + kMaxK + wave * kSSlotWords)) + 4 * lane;
    const int nw = GPB * R;                        // waves in the block (blockDim / 64)
    const int Mg = S.M / GR;
    // block b owns groups pos, pos + nblk, ... with the blocks numbered XCD
    // by XCD (b and b + 8 share one), so neighbouring groups go through one
    // L2 (a chunk's code pieces past its last row, an output line)
    const int nblk = gridDim.x, b = blockIdx.x;
    const int pos = (b & 7) * (nblk >> 3) + min(b & 7, nblk & 7) + (b >> 3);
    const int nb = (Mg - pos + nblk - 1) / nblk;   // groups of this block (>= 1: nblk <= Mg)
    const int gl = wave / R, p = wave - gl * R;    // this wave: chunk p of groups gl + i GPB
    const int ni = gl < nb ? (nb - gl + GPB - 1) / GPB : 0;
    const int n_seg = ((nb + GPB - 1) / GPB + 63) >> 6;   // wave gl = 0's items, by 64
    // rows of the group that chunk p touches, this lane's row, and the x row
    // (64 floats) of this lane's sub-block: columns (p 4096 + 64 lane) mod K
    const int q_lo = p * kSChunk / K, q_hi = (p * kSChunk + kSChunk - 1) / K;
    const int q_me = (p * kSChunk + lane * kSSub) / K;
    const int xrow = ((p * kSChunk + lane * kSSub) % K) >> 6;
    const float *const xr = s_x + xrow * 64;
    const int xsw = (xrow & 15) << 2;
    const __attribute__((address_space(4))) uint32_t *const ro =
        (const __attribute__((address_space(4))) uint32_t *)S.row_off;
    // chunk of item i of this wave (group pos + (gl + i GPB) nblk)
    auto chunk_of = [&](int i) -> int64_t {
        return (int64_t)__builtin_amdgcn_readfirstlane(((gl + i * GPB) * nblk + pos) * R + p);
    };

    // the table, then x in 16-byte pieces (piece c of 64-float row r holds x
    // piece c ^ (r & 15) of that row), then the first item's chunk (a wave
    // without items reads chunk 0, unused)
    for (int i = wave; i < kSLut / (4 * CBQ_WAVE); i += nw) {
        __builtin_amdgcn_global_load_lds(S.lut + i * 4 * CBQ_WAVE + 4 * lane,
                                         (__attribute__((address_space(3))) void *)(s_lds + i * 4 * CBQ_WAVE),
                                         16, 0, 0);
    }
    for (int i = wave; i < (K >> 8); i += nw) {    // 4 rows of 64 floats a load
        const int r = (i << 2) + (lane >> 4), c = lane & 15;
        __builtin_amdgcn_global_load_lds(x + (r << 6) + ((c ^ (r & 15)) << 2),
                                         (__attribute__((address_space(3))) void *)(s_x + (i << 8)),
                                         16, 0, 0);
    }
    SplitItem A, B;
    int64_t c = ni > 0 ? chunk_of(0) : 0;
    const uint32_t rA = ro[c];
    uint32_t hA = ro[c + 1] - rA;
    hA = hA < (uint32_t)kSRows ? hA : (uint32_t)kSRows;
    constexpr int kFirstLoads = 4 + (kSRows + 3) / 4;
    __builtin_amdgcn_sched_barrier(0);
    split_load_all(A, S, c, rA, hA, lane);
    __builtin_amdgcn_sched_barrier(0);
    // every staging load has landed (issued before the chunk's), the chunk's stay in flight
    __builtin_amdgcn_s_waitcnt((kFirstLoads & 15) | (7 << 4) | (15 << 8) |
                               ((kFirstLoads >> 4) << 14));
    lds_barrier();

    // Item k's loads (item ni - 1's again past the last one, so that every
    // path issues the same loads and the wait for the item being decoded
    // leaves them in flight); items alternate between A and B.
    auto load_item = [&](SplitItem &it, uint32_t &h, int k) {
        const int64_t ck = chunk_of(k < ni ? k : ni - 1);
        const uint32_t r0 = ro[ck];
        h = ro[ck + 1] - r0;
        h = h < (uint32_t)kSRows ? h : (uint32_t)kSRows;
        split_load_all(it, S, ck, r0, h, lane);
    };
    uint32_t hB = 0;
    int i = 0;
    for (int seg = 0; seg < n_seg; seg++) {
        float r0 = 0.f, r1 = 0.f;                  // lane l: item 64 seg + l's row sums
        const int end = min(ni, 64 * seg + 64);
        auto take = [&](float acc, int k) {
            const float s0 = wave_sum(q_me == q_lo ? acc : 0.f);
            const float s1 = q_hi > q_lo ? wave_sum(q_me == q_hi ? acc : 0.f) : 0.f;
            if (lane == k - 64 * seg) {
                r0 = s0;
                r1 = s1;
            }
        };
        // (64 seg is even, so a pair never straddles two segments; an odd
        // count ends only the last one)
        for (; i < end; i += 2) {                  // wave-uniform
            load_item(B, hB, i + 1);
            split_stage_all(A, s_slot, lane);
            take(split_decode(A.raw, s_lds, lane_addr, xr, xsw), i);
            if (i + 1 >= end) {
                i = end;
                break;
            }
            load_item(A, hA, i + 2);
            split_stage_all(B, s_slot, lane);
            take(split_decode(B.raw, s_lds, lane_addr, xr, xsw), i + 1);
        }
        // the last decode's slot reads are done (its sums used them), so the
        // slot's first 128 words take the row sums until the next staging
        s_slot[2 * lane] = __float_as_uint(r0);
        s_slot[2 * lane + 1] = __float_as_uint(r1);
        __syncthreads();
        // one thread per row: its chunks' sums in chunk order
        const int base = 64 * GPB * seg;
        for (int t = (int)threadIdx.x; t < 64 * GPB * GR; t += nw * CBQ_WAVE) {
            const int jl = t / GR, q = t - jl * GR;
            if (base + jl >= nb) break;            // (t rises with jl)
            const int g2 = jl % GPB, il = jl / GPB;
            float res = 0.f;
            for (int pp = 0; pp < R; pp++) {
                const int lo = pp * kSChunk / K, hi = (pp * kSChunk + kSChunk - 1) / K;
                if (q >= lo && q <= hi)
                    res += __uint_as_float(s_slots[(g2 * R + pp) * kSSlotWords + 2 * il + (q - lo)]);
            }
            S.out[((int64_t)(base + jl) * nblk + pos) * GR + q] = res;
        }
        // nothing in flight into the next segment's loop (the next item's
        // loads, an unused pair half's, the stores): the compiler then keeps
        // the next item's loads in flight over each decode
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));   // vmcnt(0)
        __syncthreads();                           // sums read before the next item's staging
    }
}

// ---- split format -> fixed-width indices (batched tokens) ------------------

// The 64 weights of this lane's sub-block as bf16 bit patterns, mapped to
// codebook indices through inv (65536 entries): split_decode's walk with the
// table value instead of the product.
__device__ __forceinline__ void split_decode_index(const uint32_t (&raw)[16], const uint32_t *s_lds,
                                                   int lane_addr, const uint16_t *__restrict__ inv,
                                                   uint32_t (&idx)[64])
{
    uint32_t pos = 30;
    uint32_t d1 = 0;
    const char *base = (const char *)s_lds + lane_addr;
    uint32_t w0 = *(const uint32_t *)(base - 4 * kSSub);
    uint32_t w1 = *(const uint32_t *)base;
#pragma unroll
    for (int g = 0; g < 16; g++) {
        const uint32_t w2 = *(const uint32_t *)(base + (d1 + 1) * (4 * kSSub));
        uint32_t w = __builtin_amdgcn_alignbit(w1, w0, pos);
#pragma unroll
        for (int u = 0; u < 4; u += 2) {
            const uint32_t e = *(const uint32_t *)((const char *)s_lds + (w & (4u * kSLut - 4u)));
            // high byte from the entry, low byte raw: the weight's bf16 bits
            const uint32_t b0 = __builtin_amdgcn_perm(e, raw[g], 0x0c0c0700u | u);
            const uint32_t b1 = __builtin_amdgcn_perm(e, raw[g], 0x0c0c0600u | (u + 1));
            idx[4 * g + u] = inv[b0];
            idx[4 * g + u + 1] = inv[b1];
            w >>= (e & 31u);
            pos += e;
        }
        const uint32_t dn = __builtin_amdgcn_ubfe(pos, 5, 11);
        w0 = dn != d1 ? w1 : w0;
        w1 = dn != d1 ? w2 : w1;
        d1 = dn;
    }
}

constexpr int kPackWaves = 4;

// One wave per chunk (waves stride over the chunks): lane l decodes
// sub-block l and writes its 64 indices as the 2 BITS words they occupy in
// the LSB-first stream (src/bitpack.py:32-95): chunk c, sub-block l starts at
// word 128 BITS c + 2 BITS l.
template <int BITS>
__global__ __launch_bounds__(kPackWaves * CBQ_WAVE) void split_to_packed_kernel(
    SplitSeg S, int64_t n_chunks, const uint16_t *__restrict__ inv, uint32_t *__restrict__ packed)
{
    __shared__ __attribute__((aligned(16))) uint32_t s_lds[kSLut + kPackWaves * kSSlotWords];
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / CBQ_WAVE);
    uint32_t *const s_slot = s_lds + kSLut + wave * kSSlotWords;
    const int lane_addr =
        __builtin_amdgcn_readfirstlane(4 * (kSLut + wave * kSSlotWords)) + 4 * lane;
    for (int i = wave; i < kSLut / (4 * CBQ_WAVE); i += kPackWaves)
        __builtin_amdgcn_global_load_lds(S.lut + i * 4 * CBQ_WAVE + 4 * lane,
                                         (__attribute__((address_space(3))) void *)(s_lds + i * 4 * CBQ_WAVE),
                                         16, 0, 0);
    __syncthreads();                                  // table staged
    const int64_t W = (int64_t)gridDim.x * kPackWaves;
    for (int64_t c = (int64_t)blockIdx.x * kPackWaves + wave; c < n_chunks; c += W) {
        const uint32_t r0 = S.row_off[c];
        uint32_t H = S.row_off[c + 1] - r0;
        H = H < (uint32_t)kSRows ? H : (uint32_t)kSRows;
        SplitItem it;
        split_load(it, S, c, r0, H, lane);
        split_stage(it, H, s_slot, lane);
        uint32_t idx[64];
        split_decode_index(it.raw, s_lds, lane_addr, inv, idx);
        uint32_t *dst = packed + (size_t)c * (128 * BITS) + lane * (2 * BITS);
        uint64_t acc = 0;
        int nb = 0, q = 0;
#pragma unroll
        for (int i = 0; i < 64; i++) {
            acc |= (uint64_t)idx[i] << nb;
            nb += BITS;
            if (nb >= 32) {
                dst[q++] = (uint32_t)acc;
                acc >>= 32;
                nb -= 32;
            }
        }
    }
}

// ---- a few tokens straight from the split format -------------------------------
//
// y[t, r] = W[r, :] . x[t, :] for up to 16 tokens on the bf16 matrix cores,
// every weight decoded once for all tokens and never written out.  The split
// weights are bf16 numbers; x is split exactly into three bf16 parts
// (cbq_split3), so each product is exact and only the fp32 summation order
// differs from the reference loop (src/compressed_matmul.c:208-239).
//
// Block: 16 waves (one per CU, persistent over tiles).  A tile is TR whole
// rows (SfGeo): with K % 4096 == 0, 16 rows, wave w decoding row w chunk by
// chunk (CPR chunks); otherwise GPT groups of GR rows (GR = 4096 / gcd(K,
// 4096), RCH chunks each), wave w decoding chunk w of the tile.  A wave
// decodes its chunk in eight phases of 8 weights per lane (lane l holds
// sub-block l: 64 consecutive weights of a row, as the one-token GEMV's
// decode) and writes them as bf16 to a phase tile in LDS, [TR rows][per_row
// sub-blocks][8 values], sub-block slot m ^ (row & 15).  After one barrier
// the block runs the phase's MFMAs: pair q (row tile q / KBt, k-block
// q % KBt: 4 sub-blocks x 8 columns) goes to wave q % 16, in pass q / 16
// (at most two passes, npairs <= 32); the x columns of lane group j are
// 4096 cc + 64 (4 kb + j) + 8 p + e.  The phase tiles are double-buffered.
// At the end of a tile the pairs' 16 x 16 partials are summed through LDS,
// per row tile in k-block order.
//
// LDS: the two-code table at address 0 (64 KiB), 16 code slots (64 KiB),
// two phase tiles (32 KiB; the partials reuse them): 160 KiB.
constexpr int kSfWaves = 16;
constexpr int kSfPhaseWords = 4096;               // 16 KiB

struct SfGeo {
    int GR;       // rows per group
    int RCH;      // chunks per group
    int GPT;      // groups per tile
    int CPR;      // chunks per row, walked in turn by one wave (K % 4096 == 0), else 1
    int TR;       // rows per tile (GPT * GR)
    int per_row;  // sub-blocks of a row in a phase tile
    int KBt;      // k-blocks per row tile (per_row / 4)
    int npairs;   // (row tile, k-block) pairs: ceil(TR / 16) * KBt, <= 32
};

__device__ __forceinline__ int sf_slot(int row, int m, int per_row)
{
    return (row * per_row + (m ^ (row & 15))) * 4;   // word offset of (row, sub-block m)
}

// x operands of one MFMA step for this lane: 8 fp32 values split in the
// kernel, or (PRE) the three bf16 parts read from the fragment-order
// workspace that split_x_parts_kernel wrote: part q of columns 8 piece .. +7
// of token n is the 16-byte word (piece * 3 + q) * 16 + n, so for one piece
// and part the 16 tokens are 256 contiguous bytes.
template <bool PRE> struct SfX;
template <> struct SfX<false> {
    float v[8];
};
template <> struct SfX<true> {
    cbq_u32x4 q[3];
};

__global__ __launch_bounds__(256) void split_x_parts_kernel(const float *__restrict__ x, int T,
                                                            int K, cbq_u32x4 *__restrict__ ws)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t piece = i >> 4;
    const int n = (int)(i & 15);
    if (piece >= K / 8) return;
    float v[8];
    if (n < T) {
        __builtin_memcpy(v, x + (size_t)n * K + 8 * piece, sizeof(v));
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = 0.f;
    }
    cbq_u32x4 h, m, l;
    cbq_split3(v, h, m, l);
    ws[(piece * 3 + 0) * 16 + n] = h;
    ws[(piece * 3 + 1) * 16 + n] = m;
    ws[(piece * 3 + 2) * 16 + n] = l;
}

// NSUB: MFMA passes per phase (1 when npairs <= 16, else 2).
template <typename OT, bool PRE, int NSUB>
__global__ __launch_bounds__(kSfWaves * CBQ_WAVE) void split_fewtok_kernel(
    const float *__restrict__ x, const cbq_u32x4 *__restrict__ xws, SplitSegs segs, int T, int K,
    SfGeo G)
{
    // the block's matrix: blocks [block0, block0 + nblocks) of the grid
    int sidx = 0;
#pragma unroll
    for (int i = 1; i < kSMaxSeg; i++)
        if (i < segs.n && (int)blockIdx.x >= segs.s[i].block0) sidx = i;
    const SplitSeg &S = segs.s[sidx];
    const int M = S.M;
    OT *__restrict__ const out = (OT *)S.out;
    const int bid = (int)blockIdx.x - S.block0, nbl = S.nblocks;
    const int groups = M / G.GR;
    const int n_tiles = (groups + G.GPT - 1) / G.GPT;
    __shared__ __attribute__((aligned(16))) uint32_t
        s_lds[kSLut + kSfWaves * kSSlotWords + 2 * kSfPhaseWords];
    uint32_t *const s_ph = s_lds + kSLut + kSfWaves * kSSlotWords;
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / CBQ_WAVE);
    uint32_t *const s_slot = s_lds + kSLut + wave * kSSlotWords;
    const int lane_addr =
        __builtin_amdgcn_readfirstlane(4 * (kSLut + wave * kSSlotWords)) + 4 * lane;
    const int rsub = lane & 15, j = lane >> 4;
    const int per_row = G.per_row;
    // this lane's place in the phase tile when it decodes: chunk wave % RCH
    // of group wave / RCH (a chunk's sub-block l starts 64 l into it)
    const bool decodes = wave < G.GPT * G.RCH;
    const int cw = G.CPR > 1 ? kSChunk : K;        // columns a phase tile row covers
    const int f = kSChunk * (wave % G.RCH) + 64 * lane;
    const int my_row = (wave / G.RCH) * G.GR + f / cw;
    const int my_m = (f % cw) >> 6;
    // MFMA pairs of this wave: q = wave + 16 s
    int rt[NSUB], kb[NSUB];
    bool on[NSUB];
#pragma unroll
    for (int sp = 0; sp < NSUB; sp++) {
        const int q = wave + kSfWaves * sp;
        on[sp] = q < G.npairs;
        const int qq = on[sp] ? q : 0;
        rt[sp] = qq / G.KBt;
        kb[sp] = qq - rt[sp] * G.KBt;
    }

    for (int i = wave; i < kSLut / (4 * CBQ_WAVE); i += kSfWaves)
        __builtin_amdgcn_global_load_lds(S.lut + i * 4 * CBQ_WAVE + 4 * lane,
                                         (__attribute__((address_space(3))) void *)(s_lds + i * 4 * CBQ_WAVE),
                                         16, 0, 0);

    // items of this wave: (tile, chunk cc of its row); all waves of the block
    // walk the same count, so every barrier is reached by all of them
    const int my_tiles = bid < n_tiles ? (n_tiles - bid + nbl - 1) / nbl : 0;
    const int n_items = my_tiles * G.CPR;
    auto item_chunk = [&](int k, bool &valid) {
        const int tile = bid + (k / G.CPR) * nbl;
        valid = decodes && tile * G.GPT + wave / G.RCH < groups;
        const int64_t unit = (int64_t)tile * G.GPT * G.RCH + wave;
        return valid ? unit * G.CPR + (k % G.CPR) : (int64_t)0;
    };
    // row offsets by scalar loads (a uniform address in the constant space),
    // so waiting for them does not wait for the vector loads before them;
    // every chunk load is issued (split_load_all), so the wait counts are static
    const __attribute__((address_space(4))) uint32_t *const ro =
        (const __attribute__((address_space(4))) uint32_t *)S.row_off;
    auto load_item = [&](int k, SplitItem &it, uint32_t &H) {
        bool v;
        const int64_t c = __builtin_amdgcn_readfirstlane((int)item_chunk(k < n_items ? k : 0, v));
        const uint32_t r0 = ro[c];
        H = ro[c + 1] - r0;
        H = H < (uint32_t)kSRows ? H : (uint32_t)kSRows;
        split_load_all(it, S, c, r0, H, lane);
    };
    // x of one MFMA step (phase p, pass sp) for lane (token rsub, k-block
    // lane group j).  Every load is issued (tokens past T read token T - 1
    // and are zeroed, items past the last read the last), so the compiler's
    // wait counts stay exact and a wait for x never drains the chunk loads
    // issued after it.
    const bool tok_on = rsub < T;
    const float *const xrow = x + (size_t)(tok_on ? rsub : T - 1) * K;
    auto load_x = [&](int k, int p, int sp, SfX<PRE> &xv) {
        const int cc = (k < n_items ? k : (n_items > 0 ? n_items - 1 : 0)) % G.CPR;
        const size_t col = (size_t)cc * kSChunk + 64 * (4 * kb[sp] + j) + 8 * p;
        if constexpr (PRE) {
            const cbq_u32x4 *w = xws + (col / 8) * 48 + rsub;
#pragma unroll
            for (int q = 0; q < 3; q++) xv.q[q] = w[16 * q];
        } else {
            __builtin_memcpy(xv.v, xrow + col, sizeof(xv.v));
        }
    };

    // x PD steps ahead (step u = NSUB p + sp in slot u % PD); the next
    // chunk's loads go out after the x loads issued in phase 0, so waiting
    // for the x of the next steps leaves them in flight (loads complete in
    // issue order).  PRE: the parts take 12 registers a step, one step ahead.
    constexpr int PD = PRE ? 1 : 2;
    constexpr int NSTEP = 8 * NSUB;
    SplitItem A, B;
    uint32_t hA = 0, hB = 0;
    load_item(0, A, hA);
    SfX<PRE> xq[PD];
#pragma unroll
    for (int d = 0; d < PD; d++) load_x(0, d / NSUB, d % NSUB, xq[d]);
    __syncthreads();                               // table staged: the barrier waits for the DMA
    f4 acc[NSUB];
#pragma unroll
    for (int sp = 0; sp < NSUB; sp++) acc[sp] = f4{0.f, 0.f, 0.f, 0.f};

    for (int k = 0; k < n_items; k++) {
        bool valid;
        (void)item_chunk(k, valid);
        split_stage(A, hA, s_slot, lane);
        uint32_t pos = 30;                          // as split_decode
        uint32_t d1 = 0;
        const char *base = (const char *)s_lds + lane_addr;
        uint32_t w0 = *(const uint32_t *)(base - 4 * kSSub);
        uint32_t w1 = *(const uint32_t *)base;
#pragma unroll
        for (int p = 0; p < 8; p++) {
            uint32_t pr[4];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int g = 2 * p + h;
                const uint32_t w2 = *(const uint32_t *)(base + (d1 + 1) * (4 * kSSub));
                uint32_t w = __builtin_amdgcn_alignbit(w1, w0, pos);
#pragma unroll
                for (int u = 0; u < 4; u += 2) {
                    const uint32_t e =
                        *(const uint32_t *)((const char *)s_lds + (w & (4u * kSLut - 4u)));
                    // bf16 of weights 4g+u and 4g+u+1: raw low byte, table high byte
                    pr[2 * h + (u >> 1)] = __builtin_amdgcn_perm(
                        e, A.raw[g], 0x06000700u | (uint32_t)u | ((uint32_t)(u + 1) << 16));
                    w >>= (e & 31u);
                    pos += e;
                }
                const uint32_t dn = __builtin_amdgcn_ubfe(pos, 5, 11);
                w0 = dn != d1 ? w1 : w0;
                w1 = dn != d1 ? w2 : w1;
                d1 = dn;
            }
            uint32_t *ph = s_ph + (p & 1) * kSfPhaseWords;
            if (decodes)
                *(u4 *)(ph + sf_slot(my_row, my_m, per_row)) =
                    valid ? u4{pr[0], pr[1], pr[2], pr[3]} : u4{0u, 0u, 0u, 0u};
            // this phase's x parts; the x of the step PD ahead requested
            cbq_u32x4 xb[NSUB][3];
#pragma unroll
            for (int sp = 0; sp < NSUB; sp++) {
                const int u = NSUB * p + sp;
                if constexpr (PRE) {
#pragma unroll
                    for (int q = 0; q < 3; q++) xb[sp][q] = xq[u % PD].q[q];
                } else {
                    float xv[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) xv[e] = tok_on ? xq[u % PD].v[e] : 0.f;
                    cbq_split3(xv, xb[sp][0], xb[sp][1], xb[sp][2]);
                }
                const int un = u + PD;
                if (un < NSTEP) load_x(k, un / NSUB, un % NSUB, xq[u % PD]);
                else load_x(k + 1, (un - NSTEP) / NSUB, (un - NSTEP) % NSUB, xq[u % PD]);
            }
            if (p == 0) {
                __builtin_amdgcn_sched_barrier(0);
                load_item(k + 1, B, hB);           // past the last item: item 0 again
                __builtin_amdgcn_sched_barrier(0);
            }
            __syncthreads();                       // the phase tile is complete
#pragma unroll
            for (int sp = 0; sp < NSUB; sp++) {
                if (on[sp]) {                      // wave-uniform
                    int r = 16 * rt[sp] + rsub;
                    r = r < G.TR ? r : G.TR - 1;   // rows past the tile: not written
                    const u4 a = *(const u4 *)(ph + sf_slot(r, 4 * kb[sp] + j, per_row));
#pragma unroll
                    for (int q = 0; q < 3; q++) acc[sp] = cbq_mfma_bf16(a, xb[sp][q], acc[sp]);
                }
            }
        }
        if (k % G.CPR == G.CPR - 1) {
            // tile done: the pairs' partial tiles summed per row tile in
            // k-block order (partial q at s_ph + 256 q words, both phase tiles)
            __syncthreads();                       // every wave's phase-7 reads are done
#pragma unroll
            for (int sp = 0; sp < NSUB; sp++)
                if (on[sp])
                    *(f4 *)(s_ph + 256 * (wave + kSfWaves * sp) + 4 * lane) = acc[sp];
            __syncthreads();
            const int NRT = (G.TR + 15) / 16;
            if (wave < NRT) {
                const int r0 = wave;
                f4 sum = *(const f4 *)(s_ph + 256 * (r0 * G.KBt) + 4 * lane);
                for (int q = 1; q < G.KBt; q++) {
                    const f4 v = *(const f4 *)(s_ph + 256 * (r0 * G.KBt + q) + 4 * lane);
                    sum.x += v.x;
                    sum.y += v.y;
                    sum.z += v.z;
                    sum.w += v.w;
                }
                const int tile = bid + (k / G.CPR) * nbl;
                const int rloc = 16 * r0 + 4 * j;          // first of this lane's 4 rows
                const int64_t row0 = (int64_t)tile * G.TR + rloc;
                const float vals[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
                for (int v = 0; v < 4; v++)
                    if (rloc + v < G.TR && row0 + v < M && rsub < T)
                        out[(size_t)rsub * M + row0 + v] = from_f32<OT>(vals[v]);
            }
            __syncthreads();                       // partials read before phase 0 rewrites them
#pragma unroll
            for (int sp = 0; sp < NSUB; sp++) acc[sp] = f4{0.f, 0.f, 0.f, 0.f};
        }
        A = B;
        hA = hB;
    }
}

// ---- build ------------------------------------------------------------------

// sym_code[i]: bit-reversed high-byte code | len << 24 of symbol i.
__global__ void split_bits_kernel(const int32_t *__restrict__ idx, int64_t n_sub,
                                  const uint32_t *__restrict__ sym_code, int n_sym,
                                  uint32_t *__restrict__ sub_bits)
{
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n_sub) return;
    const int32_t *p = idx + s * kSSub;
    uint32_t bits = 0;
    for (int i = 0; i < kSSub; i++) {
        int v = p[i];
        v = v < 0 ? 0 : (v >= n_sym ? n_sym - 1 : v);
        bits += sym_code[v] >> 24;
    }
    sub_bits[s] = bits;
}

__global__ void split_pack_kernel(const int32_t *__restrict__ idx, int64_t n_sub,
                                  const uint32_t *__restrict__ sym_code,
                                  const uint8_t *__restrict__ sym_raw, int n_sym,
                                  const uint32_t *__restrict__ row_off, uint32_t *__restrict__ cwords,
                                  uint8_t *__restrict__ raw)
{
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n_sub) return;
    const int64_t c = s / kSSub;
    const int l = (int)(s % kSSub);
    const uint32_t r0 = row_off[c], H = row_off[c + 1] - r0;
    const int32_t *p = idx + s * kSSub;
    uint32_t *col = cwords + (size_t)r0 * kSSub + l;
    uint32_t *rw = (uint32_t *)(raw + s * kSSub);
    uint64_t acc = 0;
    uint32_t nb = 0, row = 0, rb = 0;
    for (int i = 0; i < kSSub; i++) {
        int v = p[i];
        v = v < 0 ? 0 : (v >= n_sym ? n_sym - 1 : v);
        const uint32_t code = sym_code[v];
        acc |= (uint64_t)(code & 0xffffffu) << nb;
        nb += code >> 24;
        if (nb >= 32) {
            col[(size_t)row * kSSub] = (uint32_t)acc;
            row++;
            acc >>= 32;
            nb -= 32;
        }
        rb |= (uint32_t)sym_raw[v] << (8 * (i & 3));
        if ((i & 3) == 3) {
            rw[i >> 2] = rb;
            rb = 0;
        }
    }
    for (; row < H; row++) {                     // the partial word, then zero rows
        col[(size_t)row * kSSub] = (uint32_t)acc;
        acc = 0;
    }
}

// LSB-first fixed-width packing (src/bitpack.py:32-95) of int32 indices,
// clamped to [0, 2^bits - 1]: one thread per 32-index group, which is `bits`
// whole words.
template <int BITS>
__global__ void pack_indices_kernel(const int32_t *__restrict__ idx, int64_t n_groups,
                                    uint32_t *__restrict__ words)
{
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    const int32_t *p = idx + g * 32;
    uint32_t *w = words + g * BITS;
    constexpr uint32_t top = (1u << BITS) - 1u;
    uint64_t acc = 0;
    int nb = 0, q = 0;
    for (int i = 0; i < 32; i++) {
        const int32_t v = p[i];
        const uint32_t u = v < 0 ? 0u : ((uint32_t)v > top ? top : (uint32_t)v);
        acc |= (uint64_t)u << nb;
        nb += BITS;
        if (nb >= 32) {
            w[q++] = (uint32_t)acc;
            acc >>= 32;
            nb -= 32;
        }
    }
}

}  // namespace

extern "C" {

int cbq_pack_indices(const int32_t *indices, int64_t n, int bits, uint8_t *packed,
                     hipStream_t stream)
{
    if (!indices || !packed || n <= 0 || n % 32 != 0 || ((uintptr_t)packed & 3) != 0)
        return CK_ERR_ARG;
    const int64_t groups = n / 32;
    const dim3 grid((unsigned)((groups + 255) / 256));
    switch (bits) {
    case 8: hipLaunchKernelGGL(pack_indices_kernel<8>, grid, dim3(256), 0, stream, indices, groups, (uint32_t *)packed); break;
    case 10: hipLaunchKernelGGL(pack_indices_kernel<10>, grid, dim3(256), 0, stream, indices, groups, (uint32_t *)packed); break;
    case 11: hipLaunchKernelGGL(pack_indices_kernel<11>, grid, dim3(256), 0, stream, indices, groups, (uint32_t *)packed); break;
    case 12: hipLaunchKernelGGL(pack_indices_kernel<12>, grid, dim3(256), 0, stream, indices, groups, (uint32_t *)packed); break;
    case 13: hipLaunchKernelGGL(pack_indices_kernel<13>, grid, dim3(256), 0, stream, indices, groups, (uint32_t *)packed); break;
    default: return CK_ERR_ARG;
    }
    return cbq_launch_status("pack_indices_kernel");
}

int cbq_split_bits(const int32_t *indices, int64_t n_symbols, const uint32_t *sym_code, int n_sym,
                   uint32_t *sub_bits, hipStream_t stream)
{
    if (!indices || !sym_code || !sub_bits || n_symbols <= 0 || n_symbols % kSChunk != 0 ||
        n_sym <= 0)
        return CK_ERR_ARG;
    const int64_t n_sub = n_symbols / kSSub;
    hipLaunchKernelGGL(split_bits_kernel, dim3((unsigned)((n_sub + 255) / 256)), dim3(256), 0,
                       stream, indices, n_sub, sym_code, n_sym, sub_bits);
    return cbq_launch_status("split_bits_kernel");
}

int cbq_split_pack(const int32_t *indices, int64_t n_symbols, const uint32_t *sym_code,
                   const uint8_t *sym_raw, int n_sym, const uint32_t *row_off, uint32_t *cwords,
                   uint8_t *raw, hipStream_t stream)
{
    if (!indices || !sym_code || !sym_raw || !row_off || !cwords || !raw || n_symbols <= 0 ||
        n_symbols % kSChunk != 0 || n_sym <= 0)
        return CK_ERR_ARG;
    if (((uintptr_t)raw & 3) != 0) return CK_ERR_ARG;
    const int64_t n_sub = n_symbols / kSSub;
    hipLaunchKernelGGL(split_pack_kernel, dim3((unsigned)((n_sub + 255) / 256)), dim3(256), 0,
                       stream, indices, n_sub, sym_code, sym_raw, n_sym, row_off, cwords, raw);
    return cbq_launch_status("split_pack_kernel");
}

int cbq_split_to_packed(const cbq_split_matrix *m, const uint16_t *inv, int bits, uint8_t *packed,
                        hipStream_t stream)
{
    if (!m || !m->cwords || !m->row_off || !m->raw || !m->lut || !inv || !packed ||
        m->n_chunks <= 0)
        return CK_ERR_ARG;
    if (((uintptr_t)m->raw & 15) != 0 || ((uintptr_t)m->lut & 15) != 0 ||
        ((uintptr_t)m->cwords & 15) != 0 || ((uintptr_t)packed & 3) != 0)
        return CK_ERR_ARG;
    SplitSeg g = {};
    g.cwords = m->cwords;
    g.row_off = m->row_off;
    g.raw = m->raw;
    g.lut = m->lut;
    const int64_t want = (m->n_chunks + kPackWaves - 1) / kPackWaves;
    const int blocks = (int)(want < (int64_t)cbq_num_cus() * 2 ? want : (int64_t)cbq_num_cus() * 2);
#define CBQ_S2P(B)                                                                             \
    hipLaunchKernelGGL(split_to_packed_kernel<B>, dim3(blocks), dim3(kPackWaves * CBQ_WAVE), 0, \
                       stream, g, m->n_chunks, inv, (uint32_t *)packed)
    switch (bits) {
    case 8: CBQ_S2P(8); break;
    case 10: CBQ_S2P(10); break;
    case 11: CBQ_S2P(11); break;
    case 12: CBQ_S2P(12); break;
    case 13: CBQ_S2P(13); break;
    case 16: CBQ_S2P(16); break;
    case 32: CBQ_S2P(32); break;
    default: return CK_ERR_ARG;
    }
#undef CBQ_S2P
    return cbq_launch_status("split_to_packed_kernel");
}

size_t cbq_split_fewtok_ws_bytes(int K) { return K > 0 ? (size_t)K * 96 : 0; }

// The tile geometry of split_fewtok_kernel at this K; false when it does not
// take the shape.
static bool sf_geometry(int K, SfGeo &g)
{
    if (K <= 0 || K % 1024 != 0) return false;
    if (K % kSChunk == 0) {                        // a wave per row, K / 4096 chunks in turn
        g.GR = 1;
        g.RCH = 1;
        g.GPT = kSfWaves;
        g.CPR = K / kSChunk;
        g.per_row = kSSub;
    } else {
        int a = K, b = kSChunk;                    // gcd(K, 4096)
        while (b) {
            const int t = a % b;
            a = b;
            b = t;
        }
        g.GR = kSChunk / a;
        g.RCH = K / a;
        g.GPT = kSfWaves / g.RCH;
        g.CPR = 1;
        g.per_row = K / kSSub;
        if (g.GPT < 1) return false;
    }
    g.TR = g.GPT * g.GR;
    g.KBt = g.per_row / 4;
    g.npairs = (g.TR + 15) / 16 * g.KBt;
    // the phase tile (TR x per_row x 16 bytes) fits 16 KiB; at most two passes
    return g.per_row % 16 == 0 && g.TR * g.per_row * 4 <= kSfPhaseWords && g.npairs <= 32 &&
           g.npairs >= 1;
}

int cbq_split_linear_fewtok_f32(const float *x, int T, int n, const cbq_split_matrix *const *mats,
                                float *const *outs, const int *Ms, int K, void *ws,
                                size_t ws_bytes, hipStream_t stream)
{
    if (!x || T < 1 || n < 1 || n > kSMaxSeg || !mats || !outs || !Ms || K <= 0)
        return CK_ERR_ARG;
    SfGeo geo;
    if (!sf_geometry(K, geo) || ((uintptr_t)x & 15) != 0) return CK_ERR_ARG;
    SplitSegs segs = {};
    segs.n = n;
    int64_t tiles_sum = 0;
    int tiles[kSMaxSeg];
    for (int i = 0; i < n; i++) {
        const cbq_split_matrix *m = mats[i];
        if (!m || !m->cwords || !m->row_off || !m->raw || !m->lut || !outs[i] || Ms[i] <= 0)
            return CK_ERR_ARG;
        if (Ms[i] % geo.GR != 0 || (int64_t)Ms[i] * K % kSChunk != 0 ||
            m->n_chunks != (int64_t)Ms[i] * K / kSChunk)
            return CK_ERR_ARG;
        if (((uintptr_t)m->raw & 15) != 0 || ((uintptr_t)m->lut & 15) != 0 ||
            ((uintptr_t)m->cwords & 15) != 0)
            return CK_ERR_ARG;
        SplitSeg &g = segs.s[i];
        g.cwords = m->cwords;
        g.row_off = m->row_off;
        g.raw = m->raw;
        g.lut = m->lut;
        g.out = outs[i];
        g.M = Ms[i];
        const int groups = Ms[i] / geo.GR;
        tiles[i] = (groups + geo.GPT - 1) / geo.GPT;
        tiles_sum += tiles[i];
    }
    // one block per CU in all: a matrix gets one block per tile when the
    // tiles fit, else blocks in proportion to its tiles, rounded down, and
    // the CUs left over one at a time to the matrix with the most tiles per
    // block (each block then walks several tiles, staging the table once)
    const int cus = cbq_num_cus();
    int blocks = 0;
    for (int i = 0; i < n; i++) {
        SplitSeg &g = segs.s[i];
        const int share = tiles_sum <= cus
                              ? tiles[i]
                              : (int)std::max<int64_t>(1, cus * (int64_t)tiles[i] / tiles_sum);
        g.nblocks = std::max(1, std::min(share, tiles[i]));
        blocks += g.nblocks;
    }
    for (; blocks < cus; blocks++) {
        int best = -1;
        for (int i = 0; i < n; i++) {
            if (segs.s[i].nblocks >= tiles[i]) continue;
            if (best < 0 || (int64_t)tiles[i] * segs.s[best].nblocks >
                                (int64_t)tiles[best] * segs.s[i].nblocks)
                best = i;
        }
        if (best < 0) break;
        segs.s[best].nblocks++;
    }
    for (int i = 0, b0 = 0; i < n; i++) {
        segs.s[i].block0 = b0;
        b0 += segs.s[i].nblocks;
    }
    // with a workspace, x's three bf16 parts are written once per 16 tokens
    // in fragment order and the GEMM loads them ready-made
    const bool pre = ws && ws_bytes >= cbq_split_fewtok_ws_bytes(K) && ((uintptr_t)ws & 15) == 0;
    const bool two = geo.npairs > kSfWaves;
    if (two && !pre) return CK_ERR_ARG;            // two passes need the staged x parts
    for (int t0 = 0; t0 < T; t0 += 16) {
        const int tt = std::min(16, T - t0);
        SplitSegs sg = segs;
        for (int i = 0; i < n; i++) sg.s[i].out = outs[i] + (size_t)t0 * Ms[i];
        const float *xt = x + (size_t)t0 * K;
        const cbq_u32x4 *xw = pre ? (const cbq_u32x4 *)ws : nullptr;
        if (pre) {
            const int64_t threads = (int64_t)(K / 8) * 16;
            hipLaunchKernelGGL(split_x_parts_kernel, dim3((unsigned)((threads + 255) / 256)),
                               dim3(256), 0, stream, xt, tt, K, (cbq_u32x4 *)ws);
        }
#define CBQ_SF(PRE, NS)                                                                          \
    hipLaunchKernelGGL((split_fewtok_kernel<float, PRE, NS>), dim3(blocks),                       \
                       dim3(kSfWaves * CBQ_WAVE), 0, stream, xt, xw, sg, tt, K, geo)
        if (pre && two) CBQ_SF(true, 2);
        else if (pre) CBQ_SF(true, 1);
        else CBQ_SF(false, 1);
#undef CBQ_SF
        const int rc = cbq_launch_status("split_fewtok_kernel");
        if (rc) return rc;
    }
    return CK_SUCCESS;
}

}  // extern "C"

namespace {

// Norm modes with K <= 4096 hold 4 of GlueTile's 16 terms per virtual thread.
template <int NW, int XMODE, int GR, bool GLU = false>
void launch_split_gemv(int blocks, hipStream_t stream, const float *x, const SplitSegs &segs,
                       int K, const float *x1, float *h_out, float eps, float *arg_v, int *arg_i)
{
    if constexpr (XMODE == XF_ADD_RMS || XMODE == XF_RMS) {
        if (K <= 4096) {
            hipLaunchKernelGGL((split_gemv_kernel<NW, XMODE, GR, 4, GLU>), dim3(blocks),
                               dim3(NW * CBQ_WAVE), 0, stream, x, segs, K, x1, h_out, eps, arg_v,
                               arg_i);
            return;
        }
    }
    hipLaunchKernelGGL((split_gemv_kernel<NW, XMODE, GR, 16, GLU>), dim3(blocks),
                       dim3(NW * CBQ_WAVE), 0, stream, x, segs, K, x1, h_out, eps, arg_v, arg_i);
}

// One stacked [gate; up] matrix (2M rows, one code table), out[j] =
// silu(gate_j . x) * (up_j . x); K % 4096 == 0.
int split_linear_glu(const float *x, const float *x1, float *h_out, int mode, float eps,
                     const cbq_split_matrix *m, float *out, int M, int K, hipStream_t stream)
{
    if (!x || !m || !out || M <= 0 || M > (1 << 29) || K <= 0 || K % kSChunk != 0)
        return CK_ERR_ARG;
    if (mode != XF_NONE && mode != XF_ADD_RMS && mode != XF_RMS) return CK_ERR_ARG;
    if ((mode == XF_ADD_RMS && !x1) || (mode != XF_NONE && K > 16384)) return CK_ERR_ARG;
    if (!m->cwords || !m->row_off || !m->raw || !m->lut ||
        m->n_chunks * kSChunk != 2 * (int64_t)M * K)
        return CK_ERR_ARG;
    if (((uintptr_t)m->raw & 15) != 0 || ((uintptr_t)m->lut & 15) != 0 ||
        ((uintptr_t)m->cwords & 15) != 0)
        return CK_ERR_ARG;
    SplitSegs segs = {};
    segs.n = 1;
    SplitSeg &g = segs.s[0];
    g.cwords = m->cwords;
    g.row_off = m->row_off;
    g.raw = m->raw;
    g.lut = m->lut;
    g.out = out;
    g.M = M;                                       // outputs: pairs of rows
    const int cus = cbq_num_cus();
    const int per = M / cus;                       // pairs per CU (two items each)
    const int nw = per >= 8 ? 16 : per >= 4 ? 8 : 4;
    g.block0 = 0;
    g.nblocks = std::max(1, std::min(cus, (M + nw - 1) / nw));
#define CBQ_GLU(NWV, MODE)                                                                        \
    launch_split_gemv<NWV, MODE, 1, true>(g.nblocks, stream, x, segs, K, x1, h_out, eps, nullptr, \
                                          nullptr)
#define CBQ_GLU_MODES(NWV)                                                                        \
    do {                                                                                          \
        if (mode == XF_ADD_RMS) CBQ_GLU(NWV, XF_ADD_RMS);                                         \
        else if (mode == XF_RMS) CBQ_GLU(NWV, XF_RMS);                                            \
        else CBQ_GLU(NWV, XF_NONE);                                                               \
    } while (0)
    if (nw == 4) CBQ_GLU_MODES(4);
    else if (nw == 8) CBQ_GLU_MODES(8);
    else CBQ_GLU_MODES(16);
#undef CBQ_GLU_MODES
#undef CBQ_GLU
    return cbq_launch_status("split_gemv_kernel<glu>");
}

// cbq_split_linear_f32, with the greedy-pick pairs of every block written to
// arg_v / arg_i when those are not null (one matrix; outs[0] may be null).
int split_linear(const float *x, const float *x1, float *h_out, int mode, float eps, int n,
                 const cbq_split_matrix *const *mats, float *const *outs, const int *Ms, int K,
                 float *arg_v, int *arg_i, int *n_blocks, hipStream_t stream)
{
    if (!x || n < 1 || n > kSMaxSeg || !mats || !outs || !Ms || K <= 0 || K % 1024 != 0)
        return CK_ERR_ARG;
    if (arg_v && n != 1) return CK_ERR_ARG;
    const int GR = K % kSChunk == 0 ? 1 : K % 2048 == 0 ? 2 : 4;   // 4096 / gcd(K, 4096)
    if (mode < XF_NONE || mode > XF_RMS || ((mode == XF_SILU || mode == XF_ADD_RMS) && !x1) ||
        (mode >= XF_ADD_RMS && K > 16384))
        return CK_ERR_ARG;
    SplitSegs segs = {};
    segs.n = n;
    for (int i = 0; i < n; i++) {
        const cbq_split_matrix *m = mats[i];
        if (!m || !m->cwords || !m->row_off || !m->raw || !m->lut || (!outs[i] && !arg_v) ||
            Ms[i] <= 0)
            return CK_ERR_ARG;
        if (Ms[i] % GR != 0 || m->n_chunks * kSChunk != (int64_t)Ms[i] * K) return CK_ERR_ARG;
        if (((uintptr_t)m->raw & 15) != 0 || ((uintptr_t)m->lut & 15) != 0 ||
            ((uintptr_t)m->cwords & 15) != 0)
            return CK_ERR_ARG;
        SplitSeg &g = segs.s[i];
        g.cwords = m->cwords;
        g.row_off = m->row_off;
        g.raw = m->raw;
        g.lut = m->lut;
        g.out = outs[i];
        g.M = Ms[i];
    }
    // Rows or row groups of several chunks, plain x, one matrix: the chunks
    // of a group to separate waves (split_gemv_rg_kernel), the same outputs
    // bit for bit.  16 waves a block up to K = 8192, 12 up to K = 12288 (x
    // and the slots share what the table leaves of the LDS).  One block per
    // CU, GPB R waves each: a round of one chunk per wave takes about as
    // long as 6 + GPB R chunks' worth of decode work (one wave's decode is
    // latency-bound; more waves share the SIMDs), so the GPB with the least
    // rounds x (6 + GPB R) (ties to the larger GPB).
    const int R = K * GR / kSChunk;
    const int rg_nw = K <= rg_max_k(16) ? 16 : K <= rg_max_k(12) ? 12 : 0;
    if (mode == XF_NONE && n == 1 && !arg_v && R > 1 && R <= rg_nw && ((uintptr_t)x & 15) == 0) {
        const int Mg = Ms[0] / GR;
        const int blocks = std::max(1, std::min(cbq_num_cus(), Mg));
        const int nb = (Mg + blocks - 1) / blocks;   // groups of block 0 (the most)
        int GPB = 1;
        int64_t best = -1;
        for (int gpb = 1; gpb * R <= rg_nw; gpb++) {
            const int64_t cost = (int64_t)((nb + gpb - 1) / gpb) * (6 + gpb * R);
            if (best < 0 || cost <= best) { best = cost; GPB = gpb; }
        }
        if (rg_nw == 16)
            hipLaunchKernelGGL(split_gemv_rg_kernel<16>, dim3(blocks), dim3(GPB * R * CBQ_WAVE), 0,
                               stream, x, segs.s[0], K, GR, R, GPB);
        else
            hipLaunchKernelGGL(split_gemv_rg_kernel<12>, dim3(blocks), dim3(GPB * R * CBQ_WAVE), 0,
                               stream, x, segs.s[0], K, GR, R, GPB);
        if (n_blocks) *n_blocks = blocks;
        return cbq_launch_status("split_gemv_rg_kernel");
    }
    // One block per CU in all (a second round of blocks would pay the table
    // staging and the first loads again): each matrix gets blocks in
    // proportion to its rows, with 16 waves per block unless that leaves CUs
    // idle.
    // (in row groups: a group of GR rows is one unit of work)
    int64_t m_sum = 0;
    for (int i = 0; i < n; i++) m_sum += Ms[i] / GR;
    const int cus = cbq_num_cus();
    const int64_t per = m_sum / cus;
    const int nw = per >= 16 ? 16 : per >= 8 ? 8 : 4;
    // Shares rounded down (at least one block), then the CUs left over one
    // at a time to the matrix with the most rows per block, so the launch
    // never holds more blocks than CUs unless it has more matrices.
    int blocks = 0;
    for (int i = 0; i < n; i++) {
        SplitSeg &g = segs.s[i];
        const int Mg = g.M / GR;
        const int share = (int)std::max<int64_t>(1, cus * (int64_t)Mg / m_sum);
        g.nblocks = std::max(1, std::min(share, (Mg + nw - 1) / nw));
        blocks += g.nblocks;
    }
    for (; blocks < cus; blocks++) {
        int best = -1;
        for (int i = 0; i < n; i++) {
            const SplitSeg &g = segs.s[i];
            const int Mg = g.M / GR;
            if (g.nblocks >= (Mg + nw - 1) / nw) continue;   // every wave holds a row already
            if (best < 0 || (int64_t)Mg * segs.s[best].nblocks > (int64_t)(segs.s[best].M / GR) * g.nblocks)
                best = i;
        }
        if (best < 0) break;
        segs.s[best].nblocks++;
    }
    for (int i = 0, b0 = 0; i < n; i++) {
        segs.s[i].block0 = b0;
        b0 += segs.s[i].nblocks;
    }
#define CBQ_SPLIT_GR(NWV, MODE, G)                                                                \
    launch_split_gemv<NWV, MODE, G>(blocks, stream, x, segs, K, x1, h_out, eps, arg_v, arg_i)
#define CBQ_SPLIT(NWV, MODE)                                                                      \
    do {                                                                                          \
        if (GR == 1) CBQ_SPLIT_GR(NWV, MODE, 1);                                                  \
        else if (GR == 2) CBQ_SPLIT_GR(NWV, MODE, 2);                                             \
        else CBQ_SPLIT_GR(NWV, MODE, 4);                                                          \
    } while (0)
#define CBQ_SPLIT_MODES(NWV)                                                                      \
    do {                                                                                          \
        if (mode == XF_SILU) CBQ_SPLIT(NWV, XF_SILU);                                             \
        else if (mode == XF_ADD_RMS) CBQ_SPLIT(NWV, XF_ADD_RMS);                                  \
        else if (mode == XF_RMS) CBQ_SPLIT(NWV, XF_RMS);                                          \
        else CBQ_SPLIT(NWV, XF_NONE);                                                             \
    } while (0)
    if (nw == 4) CBQ_SPLIT_MODES(4);
    else if (nw == 8) CBQ_SPLIT_MODES(8);
    else CBQ_SPLIT_MODES(16);
#undef CBQ_SPLIT_MODES
#undef CBQ_SPLIT
#undef CBQ_SPLIT_GR
    if (n_blocks) *n_blocks = blocks;
    return cbq_launch_status("split_gemv_kernel");
}

}  // namespace

extern "C" {

int cbq_split_linear_f32(const float *x, const float *x1, float *h_out, int mode, float eps, int n,
                         const cbq_split_matrix *const *mats, float *const *outs, const int *Ms,
                         int K, hipStream_t stream)
{
    return split_linear(x, x1, h_out, mode, eps, n, mats, outs, Ms, K, nullptr, nullptr, nullptr,
                        stream);
}

int cbq_split_linear_glu_f32(const float *x0, const float *x1, float *h_out, int mode, float eps,
                             const cbq_split_matrix *m, float *out, int M, int K,
                             hipStream_t stream)
{
    return split_linear_glu(x0, x1, h_out, mode, eps, m, out, M, K, stream);
}

int cbq_split_linear_argmax_f32(const float *x0, const float *x1, float *h_out, int mode,
                                float eps, const cbq_split_matrix *m, float *out, int M, int K,
                                void *workspace, size_t workspace_bytes, int32_t *ids32,
                                int64_t *toks, int64_t *pos, int64_t first, int64_t n_toks,
                                hipStream_t stream)
{
    if (!m || !workspace || ((uintptr_t)workspace & 3) != 0 ||
        workspace_bytes < CBQ_ARGMAX_WORKSPACE || !ids32 || !toks || !pos || n_toks <= 0)
        return CK_ERR_ARG;
    if (cbq_num_cus() > kArgMaxParts) return CK_ERR_ARG;
    float *part_v = (float *)workspace;
    int *part_i = (int *)(part_v + kArgMaxParts);
    int blocks = 0;
    const int rc = split_linear(x0, x1, h_out, mode, eps, 1, &m, &out, &M, K, part_v, part_i,
                                &blocks, stream);
    if (rc) return rc;
    return cbq_argmax_merge(part_v, part_i, blocks, M, ids32, toks, pos, first, n_toks, stream);
}

}  // extern "C"

// Per-wave timeline of the last split_gemv_kernel launch, in a
// -DCBQ_TIMELINE build: kSplitTimelineWaves x 6 uint64 (entry, staged, first
// chunk decoded, row loop done, exit in 10 ns ticks; rows).  CK_ERR_ARG in
// the product build or when dst_bytes is short.
extern "C" int cbq_split_timeline_read(void *dst, size_t dst_bytes)
{
#ifdef CBQ_TIMELINE
    const size_t n = sizeof(unsigned long long) * kSplitTimelineWaves * kSplitTimelineFields;
    if (!dst || dst_bytes < n) return CK_ERR_ARG;
    if (hipMemcpyFromSymbol(dst, HIP_SYMBOL(cbq_split_timeline), n, 0, hipMemcpyDeviceToHost) !=
        hipSuccess)
        return CK_ERR_HIP;
    return CK_SUCCESS;
#else
    (void)dst;
    (void)dst_bytes;
    return CK_ERR_ARG;
#endif
}
