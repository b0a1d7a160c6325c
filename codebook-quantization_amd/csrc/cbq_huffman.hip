// Canonical-Huffman compressed GEMV / embedding / decode for gfx950.
//
// Stream semantics are those of the reference decoder
// (src/compressed_matmul.c:121-186, rocm/huffman_kernel.hip:78-115): codes
// are canonical (RFC 1951), MSB-first in the byte stream; a 12-bit table
// resolves codes <= 12 bits, longer codes are matched length by length, and
// a prefix that matches no code yields symbol 0 and advances one bit.
//
// Device format (built once at load, see cbq_hip.h): the bits of each stream
// byte are reversed so the stream reads LSB-first from little-endian 32-bit
// words; `window = alignbit(w[d+1], w[d], pos)` then holds the next 32 stream
// bits with the first one in bit 0, and a code's first 12 bits are
// `window & 0xfff` (bit-reversed).  Decode tables:
//   lut1[4096]  leaf: len (bits 0-5) | payload << 16, or pointer: len 0,
//               nb (bits 6-10) extra bits, base (bits 11-31) into lut2;
//   lut2        leaf entries of the per-prefix subtables (2^nb each); 0
//               marks "longer than 24 bits": resolved from canon tables.
// payload = bf16 value of codebook[min(sym, C-1)], or the symbol itself.
//
// Work decomposition of the fused GEMV: flat symbols are cut into 64-symbol
// sub-blocks (one per lane) and 4096-symbol chunks (one per wave step); a
// sub-block's start bit is chunk_off[c] + the wave's exclusive scan of the
// chunk's sub_len[].  A wave owns a row group (the least number of whole rows
// that is also a whole number of chunks), stages each chunk's words in LDS,
// decodes 64 symbols per lane straight into the dot product and reduces per
// row with masked wave sums, carrying the one row that spans two chunks.
#include "cbq_device.h"
#include "cbq_huff_format.h"

#include <algorithm>
#include <climits>
#include <vector>

namespace {

using namespace cbq_huff;
constexpr int kHBlock = 512;                        // 8 waves
constexpr int kHWaves = kHBlock / CBQ_WAVE;
constexpr int kLut2LdsMax = 8192;                   // lut2 entries kept in LDS
constexpr int kStageMaxWords = 4096;                // per-wave staging cap (16 KB)

// ---------------------------------------------------------------------------
// Device: decode tables in LDS and the per-symbol step
// ---------------------------------------------------------------------------

struct Tabs {
    const uint32_t *lut1;       // LDS
    const uint32_t *lut2;       // LDS or global
    uint32_t n_lut2;
    const int32_t *canon;       // global
    const int32_t *canon_pay;   // global
};

// Codes longer than 24 bits (and their corrupt neighbours): length by length
// over the canonical first codes, as the reference's slow path.
__device__ __noinline__ uint32_t decode_canon(uint32_t w, const int32_t *__restrict__ canon,
                                              const int32_t *__restrict__ pay)
{
    const uint32_t msb = __brev(w);
    for (int L = kLutBits + 1; L <= kMaxLen; L++) {
        const int32_t cnt = canon[(kMaxLen + 1) + L];
        if (!cnt) continue;
        const uint32_t code = msb >> (32 - L);
        const uint32_t first = (uint32_t)canon[L];   // < 2^L, stored as raw bits
        if (code >= first && code - first < (uint32_t)cnt)
            return (uint32_t)L | ((uint32_t)pay[canon[2 * (kMaxLen + 1) + L] + (code - first)] << 16);
    }
    return 1u | ((uint32_t)canon[3 * (kMaxLen + 1)] << 16);
}

__device__ __forceinline__ uint32_t decode_entry(uint32_t w, const Tabs &tb)
{
    uint32_t e = tb.lut1[w & (kLutSize - 1)];
    if ((e & 63u) == 0u) {
        const uint32_t nb = (e >> 6) & 31u;
        uint32_t i = (e >> 11) + ((w >> kLutBits) & ((1u << nb) - 1u));
        i = i < tb.n_lut2 ? i : tb.n_lut2 - 1u;
        e = tb.lut2[i];
        if ((e & 63u) == 0u) e = decode_canon(w, tb.canon, tb.canon_pay);
    }
    return e;
}

// Stage the words of bit range [b0, b1) (plus one word of look-ahead) into a
// wave's LDS slot.  Returns false when the range does not fit (the caller
// then reads windows from global memory).
__device__ __forceinline__ bool stage_words(uint32_t *__restrict__ stg, int stg_words,
                                            const uint32_t *__restrict__ words,
                                            int64_t n_words, uint64_t b0, uint64_t b1,
                                            int lane)
{
    const int64_t w0 = (int64_t)(b0 >> 5);
    const int nw = (int)((int64_t)((b1 + 31) >> 5) - w0 + 2);
    if (nw > stg_words || n_words <= 0) return false;
    // 8 loads of a lane in flight before its stores; slots past nw copy the
    // last word again (same value, same place), so nothing is conditional
    for (int b = 0; b < nw; b += 8 * CBQ_WAVE) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int64_t src = w0 + min(b + u * CBQ_WAVE + lane, nw - 1);
            v[u] = words[src < n_words ? src : n_words - 1];
            v[u] = src < n_words ? v[u] : 0u;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) stg[min(b + u * CBQ_WAVE + lane, nw - 1)] = v[u];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    return true;
}

__device__ __forceinline__ void wave_sync_lds()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 32 stream bits at relative bit `pos` of a staged range (staged) or of the
// global stream starting at word w0 (fallback; word index clamped).
__device__ __forceinline__ uint32_t window_lds(const uint32_t *__restrict__ stg, uint32_t pos)
{
    const uint32_t d = pos >> 5;
    return funnel(stg[d + 1], stg[d], pos);
}

__device__ __forceinline__ uint32_t window_global(const uint32_t *__restrict__ words,
                                                  int64_t n_words, int64_t w0, uint32_t pos)
{
    int64_t d = w0 + (pos >> 5);
    d = d < n_words - 1 ? d : n_words - 2;
    d = d < 0 ? 0 : d;
    return funnel(words[d + 1], words[d], pos);
}

// Load the block-shared decode tables into LDS.
// n words global -> LDS, with a thread's loads of up to 8 pieces in flight
// before its first store (one round trip per 8 pieces, not one per element);
// 16-byte pieces when both ends are 16-byte aligned.  Indices past the end
// copy the last piece again (the same value to the same place), so loads and
// stores are unconditional and no wait is needed before the next batch.
__device__ __forceinline__ void copy_to_lds(uint32_t *dst, const uint32_t *__restrict__ src,
                                            int n)
{
    const int nt = (int)blockDim.x, t = (int)threadIdx.x;
    int done = 0;
    if ((((uintptr_t)src | (uintptr_t)dst) & 15) == 0 && n >= 4) {
        typedef uint32_t w4 __attribute__((ext_vector_type(4)));
        const int n4 = n >> 2;
        const w4 *s4 = (const w4 *)src;
        w4 *d4 = (w4 *)dst;
        for (int b = 0; b < n4; b += 8 * nt) {
            w4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = s4[min(b + u * nt + t, n4 - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) d4[min(b + u * nt + t, n4 - 1)] = v[u];
        }
        done = n4 << 2;
    }
    if (done < n) {
        for (int b = done; b < n; b += 8 * nt) {
            uint32_t v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = src[min(b + u * nt + t, n - 1)];
#pragma unroll
            for (int u = 0; u < 8; u++) dst[min(b + u * nt + t, n - 1)] = v[u];
        }
    }
}

__device__ __forceinline__ void load_tables(uint32_t *s_lut1, uint32_t *s_lut2,
                                            const uint32_t *__restrict__ lut1,
                                            const uint32_t *__restrict__ lut2, int n_lut2,
                                            bool lut2_lds, float *s_cb,
                                            const float *__restrict__ cb, int n_cb)
{
    copy_to_lds(s_lut1, lut1, kLutSize);
    if (lut2_lds) copy_to_lds(s_lut2, lut2, n_lut2);
    if (n_cb > 0) copy_to_lds((uint32_t *)s_cb, (const uint32_t *)cb, n_cb);
}

// Payload -> weight.  VALUE_MODE: bf16 bits in the payload; else symbol
// index into the (clamped-at-build-time) LDS codebook.
template <bool VALUE_MODE>
__device__ __forceinline__ float payload_value(uint32_t e, const float *__restrict__ s_cb)
{
    if (VALUE_MODE) return __uint_as_float(e & 0xffff0000u);
    return s_cb[e >> 16];
}

struct HuffArgs {
    const uint32_t *words;
    int64_t n_words;
    const uint64_t *chunk_off;
    const uint16_t *sub_len;
    const uint32_t *lut1;
    const uint32_t *lut2;
    int n_lut2;
    const int32_t *canon;
    const int32_t *canon_pay;
    const float *value_cb;
    int C;
    int64_t n_sym;      // flat symbols
    int64_t n_chunks;
    int64_t n_sub;
};

// Start bit (absolute) of sub-block c*64 + lane, via a wave scan of the
// chunk's sub-block lengths.  Lanes past the last sub-block get length 0.
__device__ __forceinline__ uint64_t subblock_start(const HuffArgs &a, int64_t c, int lane,
                                                   uint32_t &my_len)
{
    const int64_t s = c * kSub + lane;
    my_len = s < a.n_sub ? (uint32_t)a.sub_len[s] : 0u;
    const uint32_t incl = wave_incl_scan(my_len);
    return a.chunk_off[c] + (uint64_t)(incl - my_len);
}

// ---------------------------------------------------------------------------
// Fused GEMV
// ---------------------------------------------------------------------------

template <int TMAX, bool VALUE_MODE>
__global__ __launch_bounds__(kHBlock) void huff_gemv_kernel(
    const float *__restrict__ x, float *__restrict__ out, HuffArgs a, int T, int M, int K,
    int RW, int SPL, int stg_words, int lut2_lds, int n_cb)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t hlds[];
    uint32_t *s_lut1 = hlds;
    uint32_t *s_lut2 = s_lut1 + kLutSize;
    const int lut2_slots = lut2_lds ? ((a.n_lut2 + 3) & ~3) : 0;
    float *s_cb = (float *)(s_lut2 + lut2_slots);
    uint32_t *s_stg = (uint32_t *)(s_cb + ((n_cb + 3) & ~3));
    load_tables(s_lut1, s_lut2, a.lut1, a.lut2, a.n_lut2, lut2_lds, s_cb, a.value_cb, n_cb);
    lds_barrier();

    const Tabs tb{s_lut1, lut2_lds ? s_lut2 : a.lut2, (uint32_t)a.n_lut2, a.canon, a.canon_pay};
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = threadIdx.x / CBQ_WAVE;
    uint32_t *stg = s_stg + wave * stg_words;
    const int64_t n_groups = ((int64_t)M + RW - 1) / RW;

    for (int64_t grp = (int64_t)blockIdx.x * kHWaves + wave; grp < n_groups;
         grp += (int64_t)gridDim.x * kHWaves) {
        float carry[TMAX];
#pragma unroll
        for (int t = 0; t < TMAX; t++) carry[t] = 0.f;
        int64_t carry_row = -1;
        for (int ci = 0; ci < SPL; ci++) {
            const int64_t c = grp * SPL + ci;
            if (c >= a.n_chunks) break;
            uint32_t my_len;
            const uint64_t start = subblock_start(a, c, lane, my_len);
            const uint64_t cbeg = a.chunk_off[c], cend = a.chunk_off[c + 1];
            const bool staged = stage_words(stg, stg_words, a.words, a.n_words, cbeg, cend, lane);
            const int64_t w0 = (int64_t)(cbeg >> 5);
            uint32_t pos = (uint32_t)(start - ((uint64_t)w0 << 5));

            const int64_t s = c * kSub + lane;
            const int64_t sym0 = s * kSub;
            const bool active = s < a.n_sub;
            const int64_t row = active ? sym0 / K : -1;
            const int k0 = active ? (int)(sym0 - row * K) : 0;
            float acc[TMAX];
#pragma unroll
            for (int t = 0; t < TMAX; t++) acc[t] = 0.f;
            if (active) {
                const float *xr = x + k0;
#pragma unroll 4
                for (int i = 0; i < kSub; i += 4) {
                    float wv[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t w = staged ? window_lds(stg, pos)
                                                  : window_global(a.words, a.n_words, w0, pos);
                        const uint32_t e = decode_entry(w, tb);
                        pos += e & 63u;
                        wv[j] = payload_value<VALUE_MODE>(e, s_cb);
                    }
#pragma unroll
                    for (int t = 0; t < TMAX; t++) {
                        if (t < T) {
                            float xv[4];
                            __builtin_memcpy(xv, xr + (size_t)t * K + i, sizeof(xv));
                            float v = acc[t];
#pragma unroll
                            for (int j = 0; j < 4; j++) v = fmaf(xv[j], wv[j], v);
                            acc[t] = v;
                        }
                    }
                }
            }
            // per-row reduction of this chunk's lanes; rows are contiguous lane runs
            const int64_t first_row = (c * kChunk) / K;
            int64_t last_row = (std::min<int64_t>(c * kChunk + kChunk, a.n_sym) - 1) / K;
            for (int64_t r = first_row; r <= last_row; r++) {
                const bool mine = row == r;
                const bool row_ends_here = (r + 1) * (int64_t)K <= std::min<int64_t>(c * kChunk + kChunk, a.n_sym);
#pragma unroll
                for (int t = 0; t < TMAX; t++) {
                    if (t < T) {
                        float v = wave_sum(mine ? acc[t] : 0.f);
                        if (r == carry_row) v += carry[t];
                        if (row_ends_here) {
                            if (lane == 0 && r < M) out[(size_t)t * M + r] = v;
                        } else {
                            carry[t] = v;
                        }
                    }
                }
                if (!row_ends_here) carry_row = r;
            }
            wave_sync_lds();   // staging slot is rewritten by the next chunk
        }
    }
}

// ---------------------------------------------------------------------------
// Fused GEMV, K % 4096 == 0, T == 1: k-tiled, two chunks per lane
// ---------------------------------------------------------------------------
//
// With K a multiple of 4096 every 4096-symbol chunk is exactly one 4096-wide
// k-tile of one row, so the block runs K/4096 phases.  Each phase stages one
// x tile (16 KB) in LDS, and every wave decodes chunk (row, phase) of NCH of
// its rows at once: lane l decodes sub-block l of each of the NCH chunks.
// That gives NCH independent decode chains per lane, all using the same x
// values.  Row sums build up over the phases in lane (row & 63) of `res`.
//
// A chunk's words reach the wave's LDS slot by direct global->LDS dwordx4
// loads.  A lane keeps q = (its bit position) - 2 into the slot.  From that,
// `win2 = alignbit(slot[d+1], slot[d], q)` holds stream bits q+2.. at bit 2,
// so `win2 & 0x3ffc` is the byte offset of the code's lut1 entry.  A chunk
// whose words exceed the slot is decoded from global memory instead.

constexpr int kTWaves = 8;
constexpr int kTBlock = kTWaves * CBQ_WAVE;
constexpr int kXRun = 68;            // LDS floats per 64-float run of x (bank spread)

typedef __attribute__((address_space(3))) void *lds_ptr_t;

__device__ __forceinline__ void dma_dword(const void *g, void *lds_base)
{
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds_base, 4, 0, 0);
}

__device__ __forceinline__ void dma_dwordx4(const void *g, void *lds_base)
{
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds_base, 16, 0, 0);
}

// Second table level and the >24-bit canonical search for an entry whose
// 12-bit prefix is a pointer (len field 0).  win2: stream bits at bit 2+.
template <bool LUT2_LDS>
__device__ __forceinline__ uint32_t decode_long(uint32_t e, uint32_t win2, uint32_t win,
                                                const uint32_t *__restrict__ lut2,
                                                uint32_t n_lut2,
                                                const int32_t *__restrict__ canon,
                                                const int32_t *__restrict__ pay)
{
    const uint32_t nb = (e >> 6) & 31u;
    uint32_t i = (e >> 11) + __builtin_amdgcn_ubfe(win2, kLutBits + 2, nb);
    i = i < n_lut2 ? i : n_lut2 - 1u;             // tables from other builders stay in bounds
    e = lut2[i];
    if ((e & 63u) == 0u) e = decode_canon(win, canon, pay);
    return e;
}

template <int NCH, bool VALUE_MODE, bool LUT2_LDS>
__global__ __launch_bounds__(kTBlock) void huff_tile_kernel(
    const float *__restrict__ x, float *__restrict__ out, HuffArgs a, int M, int K,
    int slot_words, int n_cb)
{
    __shared__ uint32_t s_lut1[kLutSize];                      // static: fixed LDS offset
    extern __shared__ __attribute__((aligned(16))) uint32_t hlds[];
    uint32_t *s_lut2 = hlds;
    const int n2 = LUT2_LDS ? ((a.n_lut2 + 63) & ~63) : 0;
    float *s_cb = (float *)(s_lut2 + n2);
    const int ncb = VALUE_MODE ? 0 : ((n_cb + 63) & ~63);
    float *s_x = s_cb + ncb;                                   // 64 runs of kXRun
    uint32_t *s_slots = (uint32_t *)(s_x + 64 * kXRun);
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / CBQ_WAVE);
    const int nwv = blockDim.x / CBQ_WAVE;                     // waves per block
    uint32_t *slot = s_slots + wave * NCH * slot_words;

    // Tables into LDS (every wave a share of 64-dword steps; sources clamped).
    for (int i = wave; i < (kLutSize >> 6); i += nwv)
        dma_dword(a.lut1 + (i << 6) + lane, s_lut1 + (i << 6));
    if (LUT2_LDS)
        for (int i = wave; i < (n2 >> 6); i += nwv) {
            const int e = (i << 6) + lane;
            dma_dword(a.lut2 + (e < a.n_lut2 ? e : a.n_lut2 - 1), s_lut2 + (i << 6));
        }
    if (!VALUE_MODE)
        for (int i = wave; i < (ncb >> 6); i += nwv) {
            const int e = (i << 6) + lane;
            dma_dword(a.value_cb + (e < n_cb ? e : n_cb - 1), s_cb + (i << 6));
        }
    const uint32_t *lut2 = LUT2_LDS ? s_lut2 : a.lut2;
    const uint32_t n_lut2 = (uint32_t)a.n_lut2;

    const int R = K / kChunk;                                  // phases (k-tiles)
    const int W = gridDim.x * nwv;
    const int wid = blockIdx.x * nwv + wave;
    const int rows = wid < M ? (M - wid + W - 1) / W : 0;
    const int b0 = blockIdx.x * nwv;                           // the block's first wave
    const int rows_max = b0 < M ? (M - b0 + W - 1) / W : 0;    // = wave 0's count
    const int n_seg = (rows_max + 63) >> 6;

    for (int seg = 0; seg < n_seg; seg++) {
        float res = 0.f;
        const int seg_rows = min(64, rows - seg * 64);         // may be <= 0
        for (int p = 0; p < R; p++) {
            __syncthreads();                                   // x tile no longer read
            // x tile p: 64 runs of 64 floats, run r at s_x + r * kXRun
            for (int r = wave; r < 64; r += nwv)
                dma_dword(x + (size_t)p * kChunk + (r << 6) + lane, s_x + r * kXRun);
            __syncthreads();                                   // waits for all loads
            for (int b = 0; b < seg_rows; b += NCH) {
                uint64_t q0[NCH];
                bool big = false;
                uint32_t sl[NCH];
                int64_t wbase[NCH];
#pragma unroll
                for (int j = 0; j < NCH; j++) {
                    const int ri = seg * 64 + b + j;
                    const int64_t row = ri < rows ? wid + (int64_t)ri * W : wid;
                    const int64_t c = __builtin_amdgcn_readfirstlane((int)(row * R + p));
                    sl[j] = a.sub_len[c * kSub + lane];
                    const uint64_t off0 = a.chunk_off[c], off1 = a.chunk_off[c + 1];
                    const int64_t wb = (int64_t)(off0 >> 5) & ~(int64_t)3;
                    // words to stage, in whole 256-word DMA steps (64 lanes x 16 B)
                    const int64_t need = ((int64_t)((off1 + 31) >> 5) + 2 - wb + 255) & ~(int64_t)255;
                    wbase[j] = wb;
                    q0[j] = off0 - ((uint64_t)wb << 5);
                    big |= need > slot_words;
                    if (need <= slot_words) {
                        for (int i = 0; i < need; i += 4 * CBQ_WAVE) {
                            int64_t src = wb + i + 4 * lane;
                            src = src < a.n_words - 4 ? src : a.n_words - 4;
                            dma_dwordx4(a.words + src, slot + j * slot_words + i);
                        }
                    }
                }
                __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));   // vmcnt(0)
                uint32_t q[NCH];
                float acc[NCH];
#pragma unroll
                for (int j = 0; j < NCH; j++) {
                    const uint32_t incl = wave_incl_scan(sl[j]);
                    q[j] = (uint32_t)q0[j] + (incl - sl[j]) - 2u;
                    acc[j] = 0.f;
                }
                const float *xr = s_x + lane * kXRun;
                if (!big) {
                    for (int i = 0; i < kSub; i += 4) {
                        typedef float f4 __attribute__((ext_vector_type(4)));
                        const f4 xv4 = *(const f4 *)(xr + i);
                        const float xv[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            // Stage by stage over the NCH chains so their LDS reads
                            // overlap.  The second table level is read by every
                            // lane (short codes read one clamped, shared entry), so
                            // no branch is taken for the 12..24-bit codes.
                            uint32_t lo[NCH], hi[NCH], win2[NCH], e[NCH], e2[NCH];
#pragma unroll
                            for (int j = 0; j < NCH; j++) {
                                const int d = (int)q[j] >> 5;
                                lo[j] = slot[j * slot_words + d];
                                hi[j] = slot[j * slot_words + d + 1];
                            }
#pragma unroll
                            for (int j = 0; j < NCH; j++) {
                                win2[j] = funnel(hi[j], lo[j], q[j]);
                                e[j] = *(const uint32_t *)((const char *)s_lut1 + (win2[j] & 0x3ffcu));
                            }
                            if (LUT2_LDS) {
#pragma unroll
                                for (int j = 0; j < NCH; j++) {
                                    const uint32_t nb = __builtin_amdgcn_ubfe(e[j], 6, 5);
                                    uint32_t i2 = (e[j] >> 11) + __builtin_amdgcn_ubfe(win2[j], kLutBits + 2, nb);
                                    i2 = i2 < n_lut2 ? i2 : n_lut2 - 1u;
                                    e2[j] = lut2[i2];
                                }
#pragma unroll
                                for (int j = 0; j < NCH; j++) e[j] = (e[j] & 63u) ? e[j] : e2[j];
                            }
                            bool any_long = false;
#pragma unroll
                            for (int j = 0; j < NCH; j++) any_long |= (e[j] & 63u) == 0u;
                            if (any_long) {
                                // LUT2_LDS: only codes longer than 24 bits (canonical
                                // search); otherwise the second level from global memory.
#pragma unroll
                                for (int j = 0; j < NCH; j++) {
                                    if ((e[j] & 63u) == 0u) {
                                        const uint32_t *sj = slot + j * slot_words;
                                        const uint32_t q2 = q[j] + 2u;
                                        const uint32_t win = funnel(sj[(q2 >> 5) + 1], sj[q2 >> 5], q2);
                                        e[j] = LUT2_LDS ? decode_canon(win, a.canon, a.canon_pay)
                                                        : decode_long<LUT2_LDS>(e[j], win2[j], win, lut2,
                                                                                n_lut2, a.canon,
                                                                                a.canon_pay);
                                    }
                                }
                            }
#pragma unroll
                            for (int j = 0; j < NCH; j++) {
                                q[j] += e[j] & 63u;
                                acc[j] = fmaf(xv[u], payload_value<VALUE_MODE>(e[j], s_cb), acc[j]);
                            }
                        }
                    }
                } else {
                    // Oversized chunk(s): windows straight from global memory.
                    for (int i = 0; i < kSub; i++) {
                        const float xv = xr[i];
#pragma unroll
                        for (int j = 0; j < NCH; j++) {
                            const uint32_t q2 = q[j] + 2u;
                            const uint32_t win = window_global(a.words, a.n_words, wbase[j], q2);
                            uint32_t e = s_lut1[win & (kLutSize - 1)];
                            if ((e & 63u) == 0u) e = decode_long<LUT2_LDS>(e, win << 2, win,
                                                                         lut2, n_lut2, a.canon,
                                                                         a.canon_pay);
                            q[j] += e & 63u;
                            acc[j] = fmaf(xv, payload_value<VALUE_MODE>(e, s_cb), acc[j]);
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < NCH; j++) {
                    const float s = wave_sum(acc[j]);
                    if (b + j < seg_rows && lane == b + j) res += s;
                }
                __builtin_amdgcn_wave_barrier();               // slot reuse by the next batch
            }
        }
        if (lane < seg_rows) out[wid + (int64_t)(seg * 64 + lane) * W] = res;
    }
}

// Fast variant for bf16-value payloads with lut2 <= 8192 entries.  One static
// LDS array at fixed offsets (lut1 at 0, so a code's lut1 byte offset is the
// LDS address; lut2 and the x tile within the 16-bit DS offset range), an
// XOR-swizzled x tile (no padding), and a 13-bit lut2 base field, so that the
// per-symbol step needs no clamp and no base adds.  A block whose lut2 holds
// unresolved (> 24-bit) entries decodes every chunk on the general path.
constexpr int kFastSlot = 1536;                               // words per chain slot
constexpr int kFastLut2 = 8192;                               // lut2 entries in LDS
constexpr int kFastChains = 16;                               // chains per block
constexpr int kFOffLut1 = kFastLut2;                          // word offsets into s_lds
constexpr int kFOffX = kFOffLut1 + kLutSize;
constexpr int kFOffSlots = kFOffX + kChunk;
constexpr int kFastLdsWords = kFOffSlots + kFastChains * kFastSlot;
static_assert(kFastLdsWords * 4 == 160 * 1024, "fast Huffman kernel fills the 160 KB LDS");

template <int NW, int NCH>
__global__ __launch_bounds__(NW * CBQ_WAVE) void huff_tile_fast_kernel(
    const float *__restrict__ x, float *__restrict__ out, HuffArgs a, int M, int K,
    int slot_cap)
{
    static_assert(NW * NCH == kFastChains, "one slot per chain");
    __shared__ __attribute__((aligned(16))) uint32_t s_lds[kFastLdsWords];
    uint32_t *const s_lut2 = s_lds;
    uint32_t *const s_lut1 = s_lds + kFOffLut1;
    float *const s_x = (float *)(s_lds + kFOffX);
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / CBQ_WAVE);
    uint32_t *const s_slot = s_lds + kFOffSlots + wave * (NCH * kFastSlot);
    int slot_addr[NCH];                                           // LDS byte addresses, in SGPRs
#pragma unroll
    for (int j = 0; j < NCH; j++)
        slot_addr[j] = __builtin_amdgcn_readfirstlane(4 * (kFOffSlots + (wave * NCH + j) * kFastSlot));

    for (int i = wave; i < (kLutSize >> 6); i += NW)
        dma_dword(a.lut1 + (i << 6) + lane, s_lut1 + (i << 6));
    const int n2 = (a.n_lut2 + 63) & ~63;
    for (int i = wave; i < (n2 >> 6); i += NW) {
        const int e = (i << 6) + lane;
        dma_dword(a.lut2 + (e < a.n_lut2 ? e : a.n_lut2 - 1), s_lut2 + (i << 6));
    }
    __syncthreads();
    // 0 entries mark codes beyond 24 bits (resolved from the canon tables).
    int unresolved = 0;
    for (int i = threadIdx.x; i < a.n_lut2; i += NW * CBQ_WAVE) unresolved |= s_lut2[i] == 0u;
    {   // block-wide OR through the (not yet used) x tile
        const bool wany = __ballot(unresolved) != 0;
        if (lane == 0) ((uint32_t *)s_x)[wave] = wany ? 1u : 0u;
    }
    __syncthreads();
    uint32_t any_unresolved = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) any_unresolved |= ((const uint32_t *)s_x)[w];
    const bool general = any_unresolved != 0;

    const int R = K / kChunk;
    const int W = gridDim.x * NW;
    const int wid = blockIdx.x * NW + wave;
    const int rows = wid < M ? (M - wid + W - 1) / W : 0;
    const int b0 = blockIdx.x * NW;
    const int rows_max = b0 < M ? (M - b0 + W - 1) / W : 0;
    const int n_seg = (rows_max + 63) >> 6;
    // lane's x run: element i at column i ^ xsw (16 lanes cover all banks)
    const float *const xr = s_x + lane * 64;
    const int xsw = (lane & 15) << 2;

    for (int seg = 0; seg < n_seg; seg++) {
        float res = 0.f;
        const int seg_rows = min(64, rows - seg * 64);
        for (int p = 0; p < R; p++) {
            __syncthreads();
            for (int r = wave; r < 64; r += NW)
                dma_dword(x + (size_t)p * kChunk + (r << 6) + (lane ^ ((r & 15) << 2)),
                          s_x + (r << 6));
            __syncthreads();
            for (int b = 0; b < seg_rows; b += NCH) {
                uint64_t q0[NCH];
                bool big = general;
                uint32_t sl[NCH];
                int64_t wbase[NCH];
#pragma unroll
                for (int j = 0; j < NCH; j++) {
                    const int ri = seg * 64 + b + j;
                    const int64_t row = ri < rows ? wid + (int64_t)ri * W : wid;
                    const int64_t c = __builtin_amdgcn_readfirstlane((int)(row * R + p));
                    sl[j] = a.sub_len[c * kSub + lane];
                    const uint64_t off0 = a.chunk_off[c], off1 = a.chunk_off[c + 1];
                    const int64_t wb = (int64_t)(off0 >> 5) & ~(int64_t)3;
                    const int64_t need =
                        ((int64_t)((off1 + 31) >> 5) + 2 - wb + 255) & ~(int64_t)255;
                    wbase[j] = wb;
                    q0[j] = off0 - ((uint64_t)wb << 5);
                    big |= need > slot_cap;
                    if (need <= slot_cap && !general) {
                        for (int i = 0; i < need; i += 4 * CBQ_WAVE) {
                            int64_t src = wb + i + 4 * lane;
                            src = src < a.n_words - 4 ? src : a.n_words - 4;
                            dma_dwordx4(a.words + src, s_slot + j * kFastSlot + i);
                        }
                    }
                }
                __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));   // vmcnt(0)
                uint32_t q[NCH];
                float acc[NCH];
#pragma unroll
                for (int j = 0; j < NCH; j++) {
                    const uint32_t incl = wave_incl_scan(sl[j]);
                    q[j] = (uint32_t)q0[j] + (incl - sl[j]) - 2u;
                    acc[j] = 0.f;
                }
                if (!big) {
                    for (int i = 0; i < kSub; i += 4) {
                        typedef float f4 __attribute__((ext_vector_type(4)));
                        const f4 xv4 = *(const f4 *)(xr + (i ^ xsw));
                        const float xv[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            uint32_t lo[NCH], hi[NCH], win2[NCH], e[NCH];
#pragma unroll
                            for (int j = 0; j < NCH; j++) {
                                const int d = (int)q[j] >> 5;
                                const uint32_t *w = (const uint32_t *)((const char *)s_lds + slot_addr[j]) + d;
                                lo[j] = w[0];
                                hi[j] = w[1];
                            }
#pragma unroll
                            for (int j = 0; j < NCH; j++) {
                                win2[j] = funnel(hi[j], lo[j], q[j]);
                                // the masked window is the byte offset of the lut1 entry
                                e[j] = *(const uint32_t *)((const char *)s_lut1 + (win2[j] & 0x3ffcu));
                            }
                            uint32_t nb[NCH], e2[NCH];
#pragma unroll
                            for (int j = 0; j < NCH; j++) {
                                // Pointer: lut2 entry base + ext.  lut2 sits at LDS address 0 and
                                // a 13-bit base plus a 15-bit ext stays below 160 KB whatever
                                // the entry holds.  Leaves (nb = 0) all read entry 0 (one
                                // broadcast), which the select drops.
                                nb[j] = __builtin_amdgcn_ubfe(e[j], 6, 4);
                                const uint32_t base = nb[j] ? __builtin_amdgcn_ubfe(e[j], 11, 13) : 0u;
                                const uint32_t i2 = base + __builtin_amdgcn_ubfe(win2[j], kLutBits + 2, nb[j]);
                                e2[j] = s_lut2[i2];
                            }
#pragma unroll
                            for (int j = 0; j < NCH; j++) {
                                asm volatile("" : "+v"(e2[j]));   // read unconditionally: no branch
                                e[j] = nb[j] ? e2[j] : e[j];
                            }
#pragma unroll
                            for (int j = 0; j < NCH; j++) {
                                q[j] += e[j] & 0xffu;            // bits 6-7 of a leaf are 0
                                acc[j] = fmaf(xv[u], __uint_as_float(e[j] & 0xffff0000u), acc[j]);
                            }
                        }
                    }
                } else {
                    for (int i = 0; i < kSub; i++) {
                        const float xv = xr[i ^ xsw];
#pragma unroll
                        for (int j = 0; j < NCH; j++) {
                            const uint32_t q2 = q[j] + 2u;
                            const uint32_t win = window_global(a.words, a.n_words, wbase[j], q2);
                            uint32_t e = s_lut1[win & (kLutSize - 1)];
                            if ((e & 63u) == 0u)
                                e = decode_long<true>(e, win << 2, win, s_lut2, (uint32_t)a.n_lut2,
                                                      a.canon, a.canon_pay);
                            q[j] += e & 63u;
                            acc[j] = fmaf(xv, __uint_as_float(e & 0xffff0000u), acc[j]);
                        }
                    }
                }
#pragma unroll
                for (int j = 0; j < NCH; j++) {
                    const float s = wave_sum(acc[j]);
                    if (b + j < seg_rows && lane == b + j) res += s;
                }
                __builtin_amdgcn_wave_barrier();
            }
        }
        if (lane < seg_rows) out[wid + (int64_t)(seg * 64 + lane) * W] = res;
    }
}

// ---------------------------------------------------------------------------
// Column layout.  Chunk c's 64 sub-blocks are stored side by side: sub-block
// l's bits, LSB-first from bit 0, in words cwords[(row_off[c] + r) * 64 + l]
// for r < rows(c) = max_l ceil(sub_len / 32) (bits past a sub-block's end
// are 0), followed by kColPadRows zero rows.  Every lane of a wave then reads
// its own LDS bank whatever its bit position, the window reads carry no bank
// conflicts, and a lane starts at bit 0 (no scan of sub-block lengths).
// ---------------------------------------------------------------------------
constexpr int kColPadRows = 4;
constexpr int kColSlotRows = kFastSlot / kSub;                // 24 rows per wave slot

// rows[c] = max(1, max_l ceil(sub_len[c*64 + l] / 32)); one wave per chunk.
__global__ __launch_bounds__(256) void col_rows_kernel(const uint16_t *__restrict__ sub_len,
                                                       int64_t n_sub, int64_t n_chunks,
                                                       uint32_t *__restrict__ rows)
{
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int64_t c = (int64_t)blockIdx.x * 4 + threadIdx.x / CBQ_WAVE;
    if (c >= n_chunks) return;                                 // whole waves
    const int64_t sb = c * kSub + lane;
    uint32_t r = ((sb < n_sub ? (uint32_t)sub_len[sb] : 0u) + 31u) >> 5;
    for (int o = CBQ_WAVE >> 1; o > 0; o >>= 1) r = max(r, (uint32_t)__shfl_xor((int)r, o, CBQ_WAVE));
    if (lane == 0) rows[c] = r > 0 ? r : 1u;
}

// One wave per chunk: lane l copies its sub-block's bits into column l.
__global__ __launch_bounds__(256) void columnize_kernel(HuffArgs a,
                                                        const uint32_t *__restrict__ row_off,
                                                        uint32_t *__restrict__ cwords)
{
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int64_t c = (int64_t)blockIdx.x * 4 + threadIdx.x / CBQ_WAVE;
    if (c >= a.n_chunks) return;
    const int64_t sb = c * kSub + lane;
    const uint32_t len = sb < a.n_sub ? a.sub_len[sb] : 0u;
    const uint32_t incl = wave_incl_scan(len);
    const uint64_t start = a.chunk_off[c] + (uint64_t)(incl - len);
    const uint32_t r0 = row_off[c], H = row_off[c + 1] - r0;
    for (uint32_t r = 0; r < H; r++) {
        const uint32_t have = len > 32u * r ? len - 32u * r : 0u;
        uint32_t w = 0u;
        if (have > 0u) {
            const uint64_t b = start + 32ull * r;
            w = window_global(a.words, a.n_words, (int64_t)(b >> 5), (uint32_t)(b & 31u));
            if (have < 32u) w &= (1u << have) - 1u;
        }
        cwords[((size_t)r0 + r) * kSub + lane] = w;
    }
}

// 32 column bits of `lane` from bit pos of its sub-block, from global memory.
__device__ __forceinline__ uint32_t col_window_global(const uint32_t *__restrict__ cwords,
                                                      uint32_t r0, int lane, uint32_t pos)
{
    const size_t w = ((size_t)r0 + (pos >> 5)) * kSub + lane;
    return funnel(cwords[w + kSub], cwords[w], pos);
}

// One matrix of a (possibly grouped) column GEMV launch: blocks
// [block0, block0 + nblocks) of the grid compute out = W x for it.
struct ColSeg {
    HuffArgs a;
    const uint32_t *cwords;
    const uint32_t *row_off;
    float *out;
    int M;
    int block0;
    int nblocks;
};
constexpr int kColMaxSeg = 4;
struct ColSegs {
    ColSeg s[kColMaxSeg];
    int n;
};

// Fused GEMV over the column layout, T = 1, bf16-value payloads, K % 4096 == 0.
// LDS as huff_tile_fast_kernel (lut2 at 0, lut1, swizzled x tile, 16 slots of
// 24 rows); one chunk per wave step.  A grouped launch runs up to four
// matrices that share x (one layer's q/k/v): each block serves one of them
// and stages that matrix's tables.
// XMODE: x is staged as xform_value(XMODE, x, x1, ...) - silu(x) * x1, or
// the RMSNorm of x (+ x1) with the grid's first block storing x + x1 to h_out.
template <int NW, bool UNIFIED, int XMODE = XF_NONE>
__global__ __launch_bounds__(NW * CBQ_WAVE) void huff_col_kernel(const float *__restrict__ x,
                                                                ColSegs segs, int K,
                                                                const float *__restrict__ x1,
                                                                float *__restrict__ h_out,
                                                                float eps)
{
    static_assert(NW <= kFastChains, "one slot per wave");
    int sidx = 0;
#pragma unroll
    for (int i = 1; i < kColMaxSeg; i++)
        if (i < segs.n && (int)blockIdx.x >= segs.s[i].block0) sidx = i;
    const ColSeg &S = segs.s[sidx];
    const HuffArgs a = S.a;
    const uint32_t *__restrict__ cwords = S.cwords;
    const uint32_t *__restrict__ row_off = S.row_off;
    float *__restrict__ out = S.out;
    const int M = S.M;
    const int bid = (int)blockIdx.x - S.block0;             // block within its matrix
    __shared__ __attribute__((aligned(16))) uint32_t s_lds[kFastLdsWords];
    uint32_t *const s_lut2 = s_lds;
    uint32_t *const s_lut1 = s_lds + kFOffLut1;
    float *const s_x = (float *)(s_lds + kFOffX);
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / CBQ_WAVE);
    uint32_t *const s_slot = s_lds + kFOffSlots + wave * kFastSlot;
    // byte address of this lane's column in the slot
    const int lane_addr = __builtin_amdgcn_readfirstlane(4 * (kFOffSlots + wave * kFastSlot)) + 4 * lane;

    // Folded glue: x0 (and x1) into registers while the tables stage.
    GlueTile<NW * CBQ_WAVE, XMODE == XF_SILU ? XF_NONE : XMODE> tile;
    if constexpr (XMODE == XF_ADD_RMS || XMODE == XF_RMS) tile.load(x, x1, K);
    for (int i = wave; i < (kLutSize >> 6); i += NW)
        dma_dword(a.lut1 + (i << 6) + lane, s_lut1 + (i << 6));
    const int n2 = (a.n_lut2 + 63) & ~63;
    for (int i = wave; i < (n2 >> 6); i += NW) {
        const int e = (i << 6) + lane;
        dma_dword(a.lut2 + (e < a.n_lut2 ? e : a.n_lut2 - 1), s_lut2 + (i << 6));
    }
    __syncthreads();
    int unresolved = 0;
    for (int i = threadIdx.x; i < a.n_lut2; i += NW * CBQ_WAVE) unresolved |= s_lut2[i] == 0u;
    {
        const bool wany = __ballot(unresolved) != 0;
        if (lane == 0) ((uint32_t *)s_x)[wave] = wany ? 1u : 0u;
    }
    __syncthreads();
    uint32_t any_unresolved = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) any_unresolved |= ((const uint32_t *)s_x)[w];
    // unified tables hold no unresolved entries (the builder refuses codes
    // beyond 24 bits), and their short-code entries are not leaves
    const bool general = !UNIFIED && any_unresolved != 0;
    float xr_scale = 1.f;
    if constexpr (XMODE == XF_ADD_RMS || XMODE == XF_RMS)
        xr_scale = tile.finish(K, eps, s_x + kFastChains);   // past the flags
    const bool store_h = XMODE == XF_ADD_RMS && blockIdx.x == 0 && h_out != nullptr;

    const int R = K / kChunk;
    const int W = S.nblocks * NW;
    const int wid = bid * NW + wave;
    const int rows = wid < M ? (M - wid + W - 1) / W : 0;
    const int b0 = bid * NW;
    const int rows_max = b0 < M ? (M - b0 + W - 1) / W : 0;
    const int n_seg = (rows_max + 63) >> 6;
    const float *const xr = s_x + lane * 64;
    const int xsw = (lane & 15) << 2;

    for (int seg = 0; seg < n_seg; seg++) {
        float res = 0.f;
        const int seg_rows = min(64, rows - seg * 64);
        for (int p = 0; p < R; p++) {
            __syncthreads();
            if constexpr (XMODE == XF_NONE) {
                for (int r = wave; r < 64; r += NW)
                    dma_dword(x + (size_t)p * kChunk + (r << 6) + (lane ^ ((r & 15) << 2)),
                              s_x + (r << 6));
            } else {
                for (int r = wave; r < 64; r += NW)
                    s_x[(r << 6) + lane] =
                        xform_value(XMODE, x, x1, h_out, store_h,
                                    p * kChunk + (r << 6) + (lane ^ ((r & 15) << 2)), xr_scale);
            }
            __syncthreads();
            for (int b = 0; b < seg_rows; b++) {
                const int64_t row = wid + (int64_t)(seg * 64 + b) * W;
                const int64_t c = __builtin_amdgcn_readfirstlane((int)(row * R + p));
                const uint32_t r0 = row_off[c], H = row_off[c + 1] - r0;
                const bool big = general || H > (uint32_t)(kColSlotRows - 1);
                if (!big)
                    for (uint32_t i = 0; i < H; i += 4)
                        dma_dwordx4(cwords + ((size_t)r0 + i) * kSub + 4 * lane, s_slot + i * kSub);
                __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));   // vmcnt(0)
                uint32_t q = 0xfffffffeu;                  // bit -2: win2 & 0x3ffc = 4 * lut1 index
                float acc = 0.f;
                if (!big && UNIFIED) {
                    // Unified tables: every lut1 entry points into lut2 (a short code at
                    // its own leaf, nb = 0), so the step has no select.
                    for (int i = 0; i < kSub; i += 4) {
                        typedef float f4 __attribute__((ext_vector_type(4)));
                        const f4 xv4 = *(const f4 *)(xr + (i ^ xsw));
                        const float xv[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const int d = __builtin_amdgcn_sbfe((int)q, 5, 27);
                            const char *wp = (const char *)s_lds + lane_addr + d * (4 * kSub);
                            const uint32_t lo = *(const uint32_t *)wp;
                            const uint32_t hi = *(const uint32_t *)(wp + 4 * kSub);
                            const uint32_t win2 = funnel(hi, lo, q);
                            const uint32_t e1 = *(const uint32_t *)((const char *)s_lut1 + (win2 & 0x3ffcu));
                            const uint32_t ext = __builtin_amdgcn_ubfe(win2, kLutBits + 2, e1 & 15u);
                            // byte offset (base + ext) * 4, kept inside lut2 whatever e1 holds
                            const uint32_t off = ((e1 >> 16) + (ext << 2)) & (uint32_t)(4 * kFastLut2 - 4);
                            const uint32_t e = *(const uint32_t *)((const char *)s_lut2 + off);
                            q += e & 0xffu;                    // bits 6-7 of a leaf are 0
                            acc = fmaf(xv[u], __uint_as_float(e & 0xffff0000u), acc);
                        }
                    }
                } else if (!big) {
                    for (int i = 0; i < kSub; i += 4) {
                        typedef float f4 __attribute__((ext_vector_type(4)));
                        const f4 xv4 = *(const f4 *)(xr + (i ^ xsw));
                        const float xv[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const int d = (int)q >> 5;
                            const char *wp = (const char *)s_lds + lane_addr + d * (4 * kSub);
                            const uint32_t lo = *(const uint32_t *)wp;
                            const uint32_t hi = *(const uint32_t *)(wp + 4 * kSub);
                            const uint32_t win2 = funnel(hi, lo, q);
                            uint32_t e = *(const uint32_t *)((const char *)s_lut1 + (win2 & 0x3ffcu));
                            const uint32_t nb = __builtin_amdgcn_ubfe(e, 6, 4);
                            const uint32_t base = nb ? __builtin_amdgcn_ubfe(e, 11, 13) : 0u;
                            uint32_t e2 = s_lut2[base + __builtin_amdgcn_ubfe(win2, kLutBits + 2, nb)];
                            asm volatile("" : "+v"(e2));       // read unconditionally: no branch
                            e = nb ? e2 : e;
                            q += e & 0xffu;                    // bits 6-7 of a leaf are 0
                            acc = fmaf(xv[u], __uint_as_float(e & 0xffff0000u), acc);
                        }
                    }
                } else {
                    for (int i = 0; i < kSub; i++) {
                        const float xv = xr[i ^ xsw];
                        const uint32_t win = col_window_global(cwords, r0, lane, q + 2u);
                        uint32_t e = s_lut1[win & (kLutSize - 1)];
                        if (UNIFIED) {
                            const uint32_t ext = __builtin_amdgcn_ubfe(win, kLutBits, e & 15u);
                            e = s_lut2[((e >> 18) + ext) & (kFastLut2 - 1)];
                        } else if ((e & 63u) == 0u) {
                            e = decode_long<true>(e, win << 2, win, s_lut2, (uint32_t)a.n_lut2,
                                                  a.canon, a.canon_pay);
                        }
                        q += e & 63u;
                        acc = fmaf(xv, __uint_as_float(e & 0xffff0000u), acc);
                    }
                }
                const float s = wave_sum(acc);
                if (lane == b) res += s;
                __builtin_amdgcn_wave_barrier();
            }
        }
        if (lane < seg_rows) out[wid + (int64_t)(seg * 64 + lane) * W] = res;
    }
}

// ---------------------------------------------------------------------------
// Embedding: one wave per requested row (H % 64 == 0)
// ---------------------------------------------------------------------------

template <bool VALUE_MODE>
__global__ __launch_bounds__(kHBlock) void huff_embedding_kernel(
    const int32_t *__restrict__ ids, float *__restrict__ out, HuffArgs a, int T, int vocab,
    int H, int stg_words, int lut2_lds, int n_cb)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t hlds[];
    uint32_t *s_lut1 = hlds;
    uint32_t *s_lut2 = s_lut1 + kLutSize;
    const int lut2_slots = lut2_lds ? ((a.n_lut2 + 3) & ~3) : 0;
    float *s_cb = (float *)(s_lut2 + lut2_slots);
    uint32_t *s_stg = (uint32_t *)(s_cb + ((n_cb + 3) & ~3));
    load_tables(s_lut1, s_lut2, a.lut1, a.lut2, a.n_lut2, lut2_lds, s_cb, a.value_cb, n_cb);
    lds_barrier();

    const Tabs tb{s_lut1, lut2_lds ? s_lut2 : a.lut2, (uint32_t)a.n_lut2, a.canon, a.canon_pay};
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = threadIdx.x / CBQ_WAVE;
    uint32_t *stg = s_stg + wave * stg_words;
    const int KS = H / kSub;                 // sub-blocks per row

    for (int t = blockIdx.x * kHWaves + wave; t < T; t += gridDim.x * kHWaves) {
        int id = ids[t];
        id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
        const int64_t s_first = (int64_t)id * KS;
        for (int r0 = 0; r0 < KS; r0 += CBQ_WAVE) {
            // sub-blocks s_first + r0 + lane lie in at most two chunks: scan both
            const int64_t sA = s_first + r0;
            const int64_t cA = sA / kSub;
            uint32_t lenA, lenB = 0;
            const uint64_t startA = subblock_start(a, cA, lane, lenA);
            const uint64_t startB = cA + 1 < a.n_chunks ? subblock_start(a, cA + 1, lane, lenB) : 0;
            const int64_t s = sA + lane;
            const bool active = (r0 + lane) < KS && s < a.n_sub;
            const int src = (int)(s & (kSub - 1));
            const bool inA = (s / kSub) == cA;
            // every lane takes part in every shuffle (a shuffle reading a lane
            // that skipped it returns nothing useful); select afterwards
            const uint64_t stA = __shfl(startA, src, CBQ_WAVE);
            const uint64_t stB = __shfl(startB, src, CBQ_WAVE);
            const uint32_t lnA = __shfl(lenA, src, CBQ_WAVE);
            const uint32_t lnB = __shfl(lenB, src, CBQ_WAVE);
            const uint64_t my_start = inA ? stA : stB;
            const uint32_t my_len = inA ? lnA : lnB;
            const int n_act = std::min(CBQ_WAVE, KS - r0);
            const uint64_t lo = __shfl(my_start, 0, CBQ_WAVE);
            const uint64_t hi = __shfl(my_start + my_len, n_act - 1, CBQ_WAVE);
            const bool staged = stage_words(stg, stg_words, a.words, a.n_words, lo, hi, lane);
            const int64_t w0 = (int64_t)(lo >> 5);
            uint32_t pos = (uint32_t)(my_start - ((uint64_t)w0 << 5));
            if (active) {
                float *dst = out + (size_t)t * H + (size_t)(r0 + lane) * kSub;
#pragma unroll 4
                for (int i = 0; i < kSub; i += 4) {
                    float v[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const uint32_t w = staged ? window_lds(stg, pos)
                                                  : window_global(a.words, a.n_words, w0, pos);
                        const uint32_t e = decode_entry(w, tb);
                        pos += e & 63u;
                        v[j] = payload_value<VALUE_MODE>(e, s_cb);
                    }
                    __builtin_memcpy(dst + i, v, sizeof(v));
                }
            }
            wave_sync_lds();
        }
    }
}

// ---------------------------------------------------------------------------
// Decode to indices: one wave per chunk (payload = symbol)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kHBlock) void huff_decode_kernel(int32_t *__restrict__ out,
                                                            HuffArgs a, int stg_words,
                                                            int lut2_lds)
{
    extern __shared__ __attribute__((aligned(16))) uint32_t hlds[];
    uint32_t *s_lut1 = hlds;
    uint32_t *s_lut2 = s_lut1 + kLutSize;
    const int lut2_slots = lut2_lds ? ((a.n_lut2 + 3) & ~3) : 0;
    uint32_t *s_stg = s_lut2 + lut2_slots;
    load_tables(s_lut1, s_lut2, a.lut1, a.lut2, a.n_lut2, lut2_lds, nullptr, nullptr, 0);
    lds_barrier();

    const Tabs tb{s_lut1, lut2_lds ? s_lut2 : a.lut2, (uint32_t)a.n_lut2, a.canon, a.canon_pay};
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int wave = threadIdx.x / CBQ_WAVE;
    uint32_t *stg = s_stg + wave * stg_words;
    for (int64_t c = (int64_t)blockIdx.x * kHWaves + wave; c < a.n_chunks;
         c += (int64_t)gridDim.x * kHWaves) {
        uint32_t my_len;
        const uint64_t start = subblock_start(a, c, lane, my_len);
        const uint64_t cbeg = a.chunk_off[c], cend = a.chunk_off[c + 1];
        const bool staged = stage_words(stg, stg_words, a.words, a.n_words, cbeg, cend, lane);
        const int64_t w0 = (int64_t)(cbeg >> 5);
        uint32_t pos = (uint32_t)(start - ((uint64_t)w0 << 5));
        const int64_t sym0 = (c * kSub + lane) * kSub;
        const int nsym = (int)std::max<int64_t>(0, std::min<int64_t>(kSub, a.n_sym - sym0));
        for (int i = 0; i < nsym; i++) {
            const uint32_t w = staged ? window_lds(stg, pos)
                                      : window_global(a.words, a.n_words, w0, pos);
            const uint32_t e = decode_entry(w, tb);
            pos += e & 63u;
            out[sym0 + i] = (int32_t)(e >> 16);
        }
        wave_sync_lds();
    }
}

// ---------------------------------------------------------------------------
// Reference-format kernels (huff_decode_to_i32 & co.)
// ---------------------------------------------------------------------------

// One thread per row over the reference's tables: MSB-first 32-bit peek,
// 12-bit LUT (-1 = miss), then lengths 13..max_len; corrupt -> 0, +1 bit.
__global__ void ref_decode_rows_kernel(const uint8_t *__restrict__ stream,
                                       const int64_t *__restrict__ rbs,
                                       const int32_t *__restrict__ lut_sym,
                                       const int32_t *__restrict__ lut_len,
                                       const int32_t *__restrict__ sl_first,
                                       const int32_t *__restrict__ sl_base,
                                       const int32_t *__restrict__ sl_sym,
                                       int32_t *__restrict__ out, int M, int K, int max_len)
{
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= M) return;
    int64_t pos = rbs[r];
    int32_t *dst = out + (int64_t)r * K;
    for (int k = 0; k < K; k++) {
        // 40-bit big-endian window; the stream carries >= 4 pad bytes, so the
        // 5th byte after the byte holding the symbol's first bit is readable.
        const uint8_t *p = stream + (pos >> 3);
        uint64_t w40 = 0;
        for (int i = 0; i < 5; i++) w40 = (w40 << 8) | p[i];
        const uint32_t w = (uint32_t)(w40 >> (8 - (pos & 7)));   // 32 bits, first in MSB
        const uint32_t key = w >> (32 - kLutBits);
        const int32_t sym = lut_sym[key];
        if (sym != -1) {
            dst[k] = sym;
            pos += lut_len[key];
            continue;
        }
        int32_t out_sym = 0, out_len = 1;
        for (int L = kLutBits + 1; L <= max_len; L++) {
            const int32_t fc = sl_first[L];
            if (fc < 0) continue;
            const int64_t d = (int64_t)(w >> (32 - L)) - fc;
            if (d >= 0 && d < sl_base[L + 1] - sl_base[L]) {
                out_sym = sl_sym[sl_base[L] + d];
                out_len = L;
                break;
            }
        }
        dst[k] = out_sym;
        pos += out_len;
    }
}

__global__ void i32_linear_kernel(const float *__restrict__ x, const int32_t *__restrict__ idx,
                                  const float *__restrict__ cb, float *__restrict__ out, int T,
                                  int M, int K, int C)
{
    const int lane = threadIdx.x & (CBQ_WAVE - 1);
    const int row = blockIdx.x * (blockDim.x / CBQ_WAVE) + threadIdx.x / CBQ_WAVE;
    if (row >= M) return;
    const int32_t *wi = idx + (int64_t)row * K;
    for (int t = 0; t < T; t++) {
        float acc = 0.f;
        for (int k = lane; k < K; k += CBQ_WAVE) {
            int32_t v = wi[k];
            v = (v < 0 || v >= C) ? C - 1 : v;
            acc = fmaf(x[(int64_t)t * K + k], cb[v], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) out[(int64_t)t * M + row] = acc;
    }
}

__global__ void i32_embedding_kernel(const int32_t *__restrict__ ids,
                                     const int32_t *__restrict__ idx,
                                     const float *__restrict__ cb, float *__restrict__ out,
                                     int T, int H, int C)
{
    const int h = blockIdx.x * blockDim.x + threadIdx.x;
    const int t = blockIdx.y;
    if (h >= H || t >= T) return;
    int32_t v = idx[(int64_t)ids[t] * H + h];
    v = (v < 0 || v >= C) ? C - 1 : v;
    out[(int64_t)t * H + h] = cb[v];
}

// ---------------------------------------------------------------------------
// Launch helpers
// ---------------------------------------------------------------------------

bool fill_args(HuffArgs &a, const cbq_huff_stream *hs, int64_t n_sym)
{
    if (!hs || !hs->words || hs->n_words < 2 || !hs->chunk_off || !hs->sub_len || !hs->lut1 ||
        !hs->lut2 || hs->n_lut2 < 1 || !hs->canon || !hs->canon_pay || n_sym <= 0)
        return false;
    a.words = hs->words; a.n_words = hs->n_words; a.chunk_off = hs->chunk_off;
    a.sub_len = hs->sub_len; a.lut1 = hs->lut1; a.lut2 = hs->lut2; a.n_lut2 = hs->n_lut2;
    a.canon = hs->canon; a.canon_pay = hs->canon_pay; a.value_cb = hs->value_cb; a.C = hs->C;
    a.n_sym = n_sym;
    a.n_chunks = (n_sym + kChunk - 1) / kChunk;
    a.n_sub = (n_sym + kSub - 1) / kSub;
    return true;
}

int stage_words_of(const cbq_huff_stream *hs)
{
    int w = hs->stage_words > 0 ? hs->stage_words : 1536;
    return std::max(8, std::min(w, kStageMaxWords));
}

struct LdsPlan {
    size_t bytes;
    int lut2_lds;
    int stg_words;
    int n_cb;
};

// Staging slot size: from the chunk sizes known at load we only know the cap
// here, so use the cap that keeps two blocks per CU when possible.
LdsPlan plan_lds(int n_lut2, int n_cb, int stg_words)
{
    LdsPlan p;
    p.lut2_lds = n_lut2 <= kLut2LdsMax;
    p.n_cb = n_cb;
    p.stg_words = stg_words;
    p.bytes = (size_t)kLutSize * 4 + (p.lut2_lds ? (size_t)((n_lut2 + 3) & ~3) * 4 : 0) +
              (size_t)((n_cb + 3) & ~3) * 4 + (size_t)kHWaves * stg_words * 4;
    return p;
}

template <int TMAX, bool VM>
int launch_gemv(const float *x, float *out, const HuffArgs &a, int T, int M, int K, int RW,
                int SPL, const LdsPlan &p, hipStream_t st)
{
    const int64_t n_groups = ((int64_t)M + RW - 1) / RW;
    const int per_cu = std::max(1, std::min(2, (int)(160 * 1024 / p.bytes)));
    const int64_t want = (n_groups + kHWaves - 1) / kHWaves;
    const int blocks = (int)std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)cbq_num_cus() * per_cu));
    hipLaunchKernelGGL((huff_gemv_kernel<TMAX, VM>), dim3(blocks), dim3(kHBlock), p.bytes, st, x,
                       out, a, T, M, K, RW, SPL, p.stg_words, p.lut2_lds, p.n_cb);
    return cbq_launch_status("huff_gemv_kernel");
}

int64_t gcd64(int64_t a, int64_t b) { while (b) { int64_t t = a % b; a = b; b = t; } return a; }

// k-tiled kernel (K % 4096 == 0, T == 1).  Returns -1 when the LDS plan does
// not leave room for useful word slots (the caller then uses huff_gemv_kernel).
constexpr size_t kTileLds = 160 * 1024;

template <int NCH>
int launch_tile_n(const float *x, float *out, const HuffArgs &a, int M, int K, int n_cb,
                  int slot_cap, int waves, hipStream_t st)
{
    const bool value_mode = a.value_cb == nullptr;
    const size_t lut2_bytes = (size_t)((a.n_lut2 + 63) & ~63) * 4;
    const size_t cb_bytes = value_mode ? 0 : (size_t)((n_cb + 63) & ~63) * 4;
    const size_t fixed_nol2 = (size_t)kLutSize * 4 + cb_bytes + 64 * kXRun * 4;
    const bool lut2_lds = fixed_nol2 + lut2_bytes + (size_t)waves * NCH * 1536 * 4 <= kTileLds;
    const size_t fixed = fixed_nol2 + (lut2_lds ? lut2_bytes : 0);
    if (fixed >= kTileLds) return -1;
    int slot = (int)((kTileLds - fixed) / ((size_t)waves * NCH * 4));
    if (slot < 1024) return -1;
    // The descriptor's stage_words caps the slot.  This kernel stages whole
    // 256-word DMA steps from a 16-byte aligned start, so the cap is widened
    // by that rounding; larger chunks decode from global memory.
    const int cap = (slot_cap + 4 + 255) & ~255;
    slot = std::min({slot, 2048, cap}) & ~255;
    const size_t dyn = fixed - (size_t)kLutSize * 4 + (size_t)waves * NCH * slot * 4;
    const int blocks = std::max(1, std::min(cbq_num_cus(), (M + waves - 1) / waves));
#define CBQ_TILE_LAUNCH(VM, L2)                                                                \
    hipLaunchKernelGGL((huff_tile_kernel<NCH, VM, L2>), dim3(blocks), dim3(waves * CBQ_WAVE), \
                       dyn, st, x, out, a, M, K, slot, n_cb)
    if (value_mode) {
        if (lut2_lds) CBQ_TILE_LAUNCH(true, true); else CBQ_TILE_LAUNCH(true, false);
    } else {
        if (lut2_lds) CBQ_TILE_LAUNCH(false, true); else CBQ_TILE_LAUNCH(false, false);
    }
#undef CBQ_TILE_LAUNCH
    return cbq_launch_status("huff_tile_kernel");
}

int launch_tile(const float *x, float *out, const HuffArgs &a, int M, int K, int n_cb,
                int slot_cap, hipStream_t st)
{
    if (a.value_cb == nullptr && a.n_lut2 <= kFastLut2 && a.n_words >= 4) {
        const int cap = std::min(kFastSlot, (slot_cap + 4 + 255) & ~255) & ~255;
        // 16 waves x 1 chain measured 45 us for 4096 -> 12288 on MI355X (8 x 2: 52 us);
        // the step is bound by LDS bank conflicts of the window and lut1 reads.
        const int blocks = std::max(1, std::min(cbq_num_cus(), (M + 15) / 16));
        hipLaunchKernelGGL((huff_tile_fast_kernel<16, 1>), dim3(blocks), dim3(16 * CBQ_WAVE), 0, st,
                           x, out, a, M, K, cap);
        return cbq_launch_status("huff_tile_fast_kernel");
    }
    // 8 waves x 2 chains: LDS holds lut1 + lut2 + x tile + 16 word slots.
    // Measured on MI355X, 4096 -> 12288: 56 us; 8x1 74 us, 4x4 76 us, 6x3
    // (lut2 pushed out of LDS) 126 us.
    return launch_tile_n<2>(x, out, a, M, K, n_cb, slot_cap, kTWaves, st);
}

}  // namespace

extern "C" {

int cbq_huff_linear_f32(const float *x, const cbq_huff_stream *hs, float *out, int T, int M,
                        int K, hipStream_t stream)
{
    if (!x || !out || T <= 0 || T > 16 || M <= 0 || K <= 0 || K % kSub != 0) return CK_ERR_ARG;
    HuffArgs a;
    if (!fill_args(a, hs, (int64_t)M * K)) return CK_ERR_ARG;
    const bool value_mode = a.value_cb == nullptr;
    const int n_cb = value_mode ? 0 : a.C;
    if (!value_mode && (a.C <= 0 || a.C > 16384)) return CK_ERR_ARG;
    const int64_t L = (int64_t)K / gcd64(K, kChunk) * kChunk;      // lcm(K, 4096)
    const int64_t RW = L / K, SPL = L / kChunk;
    if (RW > (1 << 20) || SPL > (1 << 20)) return CK_ERR_ARG;
    if (T == 1 && K % kChunk == 0) {
        const int cap = hs->stage_words > 0 ? hs->stage_words : 2048;
        const int rc = launch_tile(x, out, a, M, K, n_cb, cap, stream);
        if (rc >= 0) return rc;
    }
    const LdsPlan p = plan_lds(a.n_lut2, n_cb, stage_words_of(hs));
    if (p.bytes > 160 * 1024) return CK_ERR_ARG;
    if (T == 1)
        return value_mode ? launch_gemv<1, true>(x, out, a, T, M, K, (int)RW, (int)SPL, p, stream)
                          : launch_gemv<1, false>(x, out, a, T, M, K, (int)RW, (int)SPL, p, stream);
    if (T <= 4)
        return value_mode ? launch_gemv<4, true>(x, out, a, T, M, K, (int)RW, (int)SPL, p, stream)
                          : launch_gemv<4, false>(x, out, a, T, M, K, (int)RW, (int)SPL, p, stream);
    return value_mode ? launch_gemv<16, true>(x, out, a, T, M, K, (int)RW, (int)SPL, p, stream)
                      : launch_gemv<16, false>(x, out, a, T, M, K, (int)RW, (int)SPL, p, stream);
}

int cbq_huff_column_rows(const cbq_huff_stream *hs, int64_t n_symbols, uint32_t *rows,
                         hipStream_t stream)
{
    if (!hs || !hs->sub_len || !rows || n_symbols <= 0) return CK_ERR_ARG;
    const int64_t n_chunks = (n_symbols + kChunk - 1) / kChunk;
    const int64_t n_sub = (n_symbols + kSub - 1) / kSub;
    const int64_t blocks = (n_chunks + 3) / 4;
    if (blocks > INT32_MAX) return CK_ERR_ARG;
    hipLaunchKernelGGL(col_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, hs->sub_len,
                       n_sub, n_chunks, rows);
    return cbq_launch_status("col_rows_kernel");
}

int cbq_huff_columnize(const cbq_huff_stream *hs, int64_t n_symbols, const uint32_t *row_off,
                       uint32_t *cwords, hipStream_t stream)
{
    HuffArgs a;
    if (!fill_args(a, hs, n_symbols) || !row_off || !cwords) return CK_ERR_ARG;
    const int64_t blocks = (a.n_chunks + 3) / 4;
    if (blocks > INT32_MAX) return CK_ERR_ARG;
    hipLaunchKernelGGL(columnize_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a, row_off,
                       cwords);
    return cbq_launch_status("columnize_kernel");
}

int cbq_huff_linear_col_xform_f32(const float *x, const float *x1, float *h_out, int mode,
                                  float eps, int n, const cbq_huff_stream *const *hs,
                                  const cbq_huff_columns *const *cols, float *const *outs,
                                  const int *Ms, int K, hipStream_t stream)
{
    if (!x || n < 1 || n > kColMaxSeg || !hs || !cols || !outs || !Ms || K <= 0 ||
        K % kChunk != 0)
        return CK_ERR_ARG;
    if (mode < XF_NONE || mode > XF_RMS || ((mode == XF_SILU || mode == XF_ADD_RMS) && !x1) ||
        (mode >= XF_ADD_RMS && K > 16384))
        return CK_ERR_ARG;
    ColSegs segs = {};
    segs.n = n;
    bool unified = true;
    int m_max = 0;
    for (int i = 0; i < n; i++) {
        const cbq_huff_stream *h = hs[i];
        const cbq_huff_columns *c = cols[i];
        const int M = Ms[i];
        if (!h || !c || !outs[i] || M <= 0) return CK_ERR_ARG;
        if (!h->lut1 || !h->lut2 || h->n_lut2 < 1 || h->n_lut2 > kFastLut2 || !h->canon ||
            !h->canon_pay || h->value_cb != nullptr)
            return CK_ERR_ARG;
        if (!c->cwords || !c->row_off || c->n_chunks != (int64_t)M * K / kChunk) return CK_ERR_ARG;
        unified = unified && c->ulut1 && c->ulut2 && c->n_ulut2 >= 1 && c->n_ulut2 <= kFastLut2;
        m_max = std::max(m_max, M);
    }
    // Waves per block (one block per CU: the LDS is static): 16 when every CU
    // gets >= 16 rows of the largest matrix, else fewer so that small matrices
    // still reach all CUs.  MI355X, 1024 x 4096: 16 waves 14.7 us, 4 waves
    // 13.7 us; 4096 x 4096: 16 waves 17.9 us, 8 waves 23.4 us.  A step is a
    // chain of three dependent LDS reads (~440 cycles), so throughput scales
    // with resident waves.
    const int per = m_max / cbq_num_cus();
    const int nw = per >= 16 ? 16 : per >= 8 ? 8 : 4;
    int blocks = 0;
    for (int i = 0; i < n; i++) {
        ColSeg &g = segs.s[i];
        const int M = Ms[i];
        HuffArgs &a = g.a;
        a = HuffArgs{};
        if (unified) {
            a.lut1 = cols[i]->ulut1; a.lut2 = cols[i]->ulut2; a.n_lut2 = cols[i]->n_ulut2;
        } else {
            a.lut1 = hs[i]->lut1; a.lut2 = hs[i]->lut2; a.n_lut2 = hs[i]->n_lut2;
        }
        a.canon = hs[i]->canon; a.canon_pay = hs[i]->canon_pay; a.C = hs[i]->C;
        a.n_sym = (int64_t)M * K; a.n_chunks = cols[i]->n_chunks; a.n_sub = a.n_sym / kSub;
        g.cwords = cols[i]->cwords; g.row_off = cols[i]->row_off; g.out = outs[i]; g.M = M;
        g.block0 = blocks;
        g.nblocks = std::max(1, std::min(cbq_num_cus(), (M + nw - 1) / nw));
        blocks += g.nblocks;
    }
    if (mode != XF_NONE && !unified) return CK_ERR_ARG;   // transforms need unified tables
#define CBQ_COL_XF(NWV, MODE)                                                                  \
    hipLaunchKernelGGL((huff_col_kernel<NWV, true, MODE>), dim3(blocks), dim3(NWV * CBQ_WAVE),  \
                       0, stream, x, segs, K, x1, h_out, eps)
#define CBQ_COL_LAUNCH(NWV)                                                                    \
    do {                                                                                       \
        if (mode == XF_SILU) CBQ_COL_XF(NWV, XF_SILU);                                         \
        else if (mode == XF_ADD_RMS) CBQ_COL_XF(NWV, XF_ADD_RMS);                              \
        else if (mode == XF_RMS) CBQ_COL_XF(NWV, XF_RMS);                                      \
        else if (unified) CBQ_COL_XF(NWV, XF_NONE);                                            \
        else                                                                                   \
            hipLaunchKernelGGL((huff_col_kernel<NWV, false>), dim3(blocks),                    \
                               dim3(NWV * CBQ_WAVE), 0, stream, x, segs, K,                    \
                               (const float *)nullptr, (float *)nullptr, 0.f);                  \
    } while (0)
    if (nw == 4) CBQ_COL_LAUNCH(4);
    else if (nw == 8) CBQ_COL_LAUNCH(8);
    else CBQ_COL_LAUNCH(16);
#undef CBQ_COL_LAUNCH
#undef CBQ_COL_XF
    return cbq_launch_status("huff_col_kernel");
}

int cbq_huff_linear_col_multi_f32(const float *x, int n, const cbq_huff_stream *const *hs,
                                  const cbq_huff_columns *const *cols, float *const *outs,
                                  const int *Ms, int K, hipStream_t stream)
{
    return cbq_huff_linear_col_xform_f32(x, nullptr, nullptr, XF_NONE, 0.f, n, hs, cols, outs, Ms,
                                         K, stream);
}

int cbq_huff_linear_col_f32(const float *x, const cbq_huff_stream *hs,
                            const cbq_huff_columns *cols, float *out, int M, int K,
                            hipStream_t stream)
{
    return cbq_huff_linear_col_multi_f32(x, 1, &hs, &cols, &out, &M, K, stream);
}

int cbq_huff_embedding_f32(const int32_t *token_ids, const cbq_huff_stream *hs, float *out,
                           int T, int vocab, int H, hipStream_t stream)
{
    if (!token_ids || !out || T <= 0 || vocab <= 0 || H <= 0 || H % kSub != 0) return CK_ERR_ARG;
    HuffArgs a;
    if (!fill_args(a, hs, (int64_t)vocab * H)) return CK_ERR_ARG;
    const bool value_mode = a.value_cb == nullptr;
    const int n_cb = value_mode ? 0 : a.C;
    if (!value_mode && (a.C <= 0 || a.C > 16384)) return CK_ERR_ARG;
    const LdsPlan p = plan_lds(a.n_lut2, n_cb, stage_words_of(hs));
    if (p.bytes > 160 * 1024) return CK_ERR_ARG;
    const int blocks = std::max(1, std::min((T + kHWaves - 1) / kHWaves, cbq_num_cus()));
    if (value_mode)
        hipLaunchKernelGGL((huff_embedding_kernel<true>), dim3(blocks), dim3(kHBlock), p.bytes,
                           stream, token_ids, out, a, T, vocab, H, p.stg_words, p.lut2_lds, 0);
    else
        hipLaunchKernelGGL((huff_embedding_kernel<false>), dim3(blocks), dim3(kHBlock), p.bytes,
                           stream, token_ids, out, a, T, vocab, H, p.stg_words, p.lut2_lds, n_cb);
    return cbq_launch_status("huff_embedding_kernel");
}

int cbq_huff_decode_indices(const cbq_huff_stream *hs, int32_t *out, int64_t n_symbols,
                            hipStream_t stream)
{
    if (!out) return CK_ERR_ARG;
    HuffArgs a;
    if (!fill_args(a, hs, n_symbols)) return CK_ERR_ARG;
    const LdsPlan p = plan_lds(a.n_lut2, 0, stage_words_of(hs));
    if (p.bytes > 160 * 1024) return CK_ERR_ARG;
    const int64_t want = (a.n_chunks + kHWaves - 1) / kHWaves;
    const int blocks = (int)std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)cbq_num_cus() * 2));
    hipLaunchKernelGGL(huff_decode_kernel, dim3(blocks), dim3(kHBlock), p.bytes, stream, out, a,
                       p.stg_words, p.lut2_lds);
    return cbq_launch_status("huff_decode_kernel");
}

int huff_decode_to_i32(const void *stream, const void *row_bit_start, const void *lut_sym,
                       const void *lut_len, const void *sl_first_code,
                       const void *sl_base_offset, const void *sl_sym, void *out, int M, int K,
                       int max_code_len, hipStream_t stream_h)
{
    if (!stream || !row_bit_start || !lut_sym || !lut_len || !sl_first_code ||
        !sl_base_offset || !sl_sym || !out)
        return HK_ERR_ARG;
    if (M <= 0 || K <= 0 || max_code_len > 32) return HK_ERR_ARG;
    const int blk = 64;
    hipLaunchKernelGGL(ref_decode_rows_kernel, dim3((M + blk - 1) / blk), dim3(blk), 0, stream_h,
                       (const uint8_t *)stream, (const int64_t *)row_bit_start,
                       (const int32_t *)lut_sym, (const int32_t *)lut_len,
                       (const int32_t *)sl_first_code, (const int32_t *)sl_base_offset,
                       (const int32_t *)sl_sym, (int32_t *)out, M, K, max_code_len);
    return cbq_launch_status("ref_decode_rows_kernel");
}

int huff_i32_linear_f32(const void *x, const void *i32_indices, const void *codebook, void *out,
                        int T, int M, int K, int C, hipStream_t stream_h)
{
    if (!x || !i32_indices || !codebook || !out) return HK_ERR_ARG;
    if (T <= 0 || M <= 0 || K <= 0 || C <= 0) return HK_ERR_ARG;
    const int wpb = 4;
    hipLaunchKernelGGL(i32_linear_kernel, dim3((M + wpb - 1) / wpb), dim3(wpb * CBQ_WAVE), 0,
                       stream_h, (const float *)x, (const int32_t *)i32_indices,
                       (const float *)codebook, (float *)out, T, M, K, C);
    return cbq_launch_status("i32_linear_kernel");
}

int huff_i32_embedding_f32(const void *token_ids, const void *i32_indices, const void *codebook,
                           void *out, int T, int H, int C, hipStream_t stream_h)
{
    if (!token_ids || !i32_indices || !codebook || !out) return HK_ERR_ARG;
    if (T <= 0 || H <= 0 || C <= 0 || T > 65535) return HK_ERR_ARG;
    const int blk = 128;
    hipLaunchKernelGGL(i32_embedding_kernel, dim3((H + blk - 1) / blk, T), dim3(blk), 0,
                       stream_h, (const int32_t *)token_ids, (const int32_t *)i32_indices,
                       (const float *)codebook, (float *)out, T, H, C);
    return cbq_launch_status("i32_embedding_kernel");
}

}  // extern "C"
