// Split-exponent device format and its one-token GEMV, for gfx950.
//
// The canonical-Huffman index stream of the reference
// (src/huffman_codebook.py:126-226) spends ~10.5 bits per weight, and its
// decode is a chain of three dependent table reads per symbol.  When every
// codebook value is a bf16 number (the lossless direct-codebook mode), the
// same weights can be held instead as
//
//   raw   one byte per weight: sign (bit 7) | the 7 mantissa bits;
//   exp   the 8-bit exponent, Huffman-coded with codes of at most 7 bits
//         (~2.6 bits per weight on N(0, sigma) weights),
//
// ~10.6 bits per weight, built once at load from the decoded indices.  The
// exponent codes of each 64-weight sub-block form an LSB-first bit stream
// stored in the column layout: chunk c (4096 weights, 64 sub-blocks) owns
// rows row_off[c] .. row_off[c+1]-1 of 64 words, word l of a row belonging
// to sub-block l, so a wave reads a row with one conflict-free LDS access.
// A 128-entry table maps the next 7 stream bits to (exp << 23) | len, and
// the weight is ((sign|mantissa byte, placed by v_perm) & 0x807fffff) |
// (entry & 0x7f800000): one table read and ~7 VALU operations per weight.
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
constexpr int kSMaxLen = 7;                       // exponent code length limit
constexpr int kSLut = 1 << kSMaxLen;              // 128 table entries
// A chunk has at most ceil(64 * 7 / 32) = 14 rows; the slot holds one more,
// since the window of a sub-block's last codes reads the row after them.
constexpr int kSRows = 15;
constexpr int kSSlotWords = kSRows * kSSub;       // one wave's chunk slot
constexpr int kSMaxSeg = 4;

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
// sub-block and its exponent-code words (rows 0 .. H-1 of the chunk).
struct SplitItem {
    uint32_t raw[16];
    uint32_t ew[kSRows];
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
    const uint32_t *wp = S.cwords + (size_t)r0 * kSSub + lane;
#pragma unroll
    for (int r = 0; r < kSRows; r++) it.ew[r] = r < (int)H ? wp[(size_t)r * kSSub] : 0u;
}

// Decodes the 64 weights of this lane's sub-block against the staged x and
// returns the dot product.  slot: this wave's LDS rows (already written);
// lane_addr: byte address of the lane's column in row 0 of the slot.
__device__ __forceinline__ float split_decode(const uint32_t (&raw)[16], const uint32_t *s_lds,
                                              int lane_addr, const float *xr, int xsw)
{
    float acc = 0.f;
    uint32_t q = 0;
#pragma unroll
    for (int g = 0; g < 16; g++) {
        const f4 xv4 = *(const f4 *)(xr + ((4 * g) ^ xsw));
        const float xv[4] = {xv4.x, xv4.y, xv4.z, xv4.w};
        // 30 stream bits from bit q on, in bits 2..31 (bits 0-1: the two before)
        const int qm = (int)q - 2;
        const int d = qm >> 5;
        const char *wp = (const char *)s_lds + lane_addr + d * (4 * kSSub);
        const uint32_t lo = *(const uint32_t *)wp;
        const uint32_t hi = *(const uint32_t *)(wp + 4 * kSSub);
        uint32_t w = __builtin_amdgcn_alignbit(hi, lo, (uint32_t)qm);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t e = *(const uint32_t *)((const char *)s_lds + (w & (4u * kSLut - 4u)));
            // raw byte u in bytes 3 and 2: sign lands in bit 31, mantissa in 16..22
            const uint32_t sel = (uint32_t)(u << 24) | (uint32_t)(u << 16) | 0x0c0cu;
            const uint32_t R = __builtin_amdgcn_perm(raw[g], raw[g], sel);
            const uint32_t v = (R & 0x807fffffu) | (e & 0x7f800000u);
            acc = fmaf(xv[u], __uint_as_float(v), acc);
            w >>= (e & 31u);
            q += e & 0xffu;
        }
    }
    return acc;
}

template <int NW, int XMODE>
__global__ __launch_bounds__(NW * CBQ_WAVE) void split_gemv_kernel(const float *__restrict__ x,
                                                                   SplitSegs segs, int K,
                                                                   const float *__restrict__ x1,
                                                                   float *__restrict__ h_out,
                                                                   float eps)
{
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
    uint32_t *const s_slot = s_lds + kSLut + kSChunk + wave * kSSlotWords;
    const int lane_addr =
        __builtin_amdgcn_readfirstlane(4 * (kSLut + kSChunk + wave * kSSlotWords)) + 4 * lane;

    GlueTile<NW * CBQ_WAVE, XMODE == XF_SILU ? XF_NONE : XMODE> tile;
    if constexpr (XMODE == XF_ADD_RMS || XMODE == XF_RMS) tile.load(x, x1, K);
    if (threadIdx.x < kSLut) s_lds[threadIdx.x] = S.lut[threadIdx.x];
    float xr_scale = 1.f;
    if constexpr (XMODE == XF_ADD_RMS || XMODE == XF_RMS)
        xr_scale = tile.finish(K, eps, s_x);      // s_x is staged after the next barrier
    const bool store_h = XMODE == XF_ADD_RMS && blockIdx.x == 0 && h_out != nullptr;

    const int R = K / kSChunk;
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
                for (int r = wave; r < 64; r += NW) {
                    const float v = x[(size_t)p * kSChunk + (r << 6) + (lane ^ ((r & 15) << 2))];
                    s_x[(r << 6) + lane] = v;
                }
            } else {
                for (int r = wave; r < 64; r += NW)
                    s_x[(r << 6) + lane] =
                        xform_value(XMODE, x, x1, h_out, store_h,
                                    p * kSChunk + (r << 6) + (lane ^ ((r & 15) << 2)), xr_scale);
            }
            __syncthreads();
            auto chunk_of = [&](int b, uint32_t &r0, uint32_t &H) {
                const int64_t row = wid + (int64_t)(seg * 64 + b) * W;
                const int64_t c = __builtin_amdgcn_readfirstlane((int)(row * R + p));
                r0 = S.row_off[c];
                H = S.row_off[c + 1] - r0;
                H = H < (uint32_t)kSRows ? H : (uint32_t)kSRows;
                return c;
            };
            // Two items in flight: the next one's loads go out before this
            // one is decoded.  The slot is rewritten only after the previous
            // item's reads (LDS operations of a wave complete in order).
            SplitItem A, B;
            uint32_t rA = 0, hA = 0, rB = 0, hB = 0;
            if (seg_rows > 0) {
                const int64_t c = chunk_of(0, rA, hA);
                split_load(A, S, c, rA, hA, lane);
            }
            for (int b = 0; b < seg_rows; b += 2) {
                if (b + 1 < seg_rows) {
                    const int64_t c = chunk_of(b + 1, rB, hB);
                    split_load(B, S, c, rB, hB, lane);
                }
#pragma unroll
                for (int r = 0; r < kSRows; r++)
                    if (r < (int)hA) s_slot[r * kSSub + lane] = A.ew[r];
                {
                    const float s = wave_sum(split_decode(A.raw, s_lds, lane_addr, xr, xsw));
                    if (lane == b) res += s;
                }
                if (b + 1 >= seg_rows) break;
                if (b + 2 < seg_rows) {
                    const int64_t c = chunk_of(b + 2, rA, hA);
                    split_load(A, S, c, rA, hA, lane);
                }
#pragma unroll
                for (int r = 0; r < kSRows; r++)
                    if (r < (int)hB) s_slot[r * kSSub + lane] = B.ew[r];
                {
                    const float s = wave_sum(split_decode(B.raw, s_lds, lane_addr, xr, xsw));
                    if (lane == b + 1) res += s;
                }
            }
        }
        if (lane < seg_rows) S.out[wid + (int64_t)(seg * 64 + lane) * W] = res;
    }
}

// ---- build ------------------------------------------------------------------

// sym_code[i]: bit-reversed exponent code | len << 24 of symbol i.
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

}  // namespace

extern "C" {

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

int cbq_split_linear_f32(const float *x, const float *x1, float *h_out, int mode, float eps, int n,
                         const cbq_split_matrix *const *mats, float *const *outs, const int *Ms,
                         int K, hipStream_t stream)
{
    if (!x || n < 1 || n > kSMaxSeg || !mats || !outs || !Ms || K <= 0 || K % kSChunk != 0)
        return CK_ERR_ARG;
    if (mode < XF_NONE || mode > XF_RMS || ((mode == XF_SILU || mode == XF_ADD_RMS) && !x1) ||
        (mode >= XF_ADD_RMS && K > 16384))
        return CK_ERR_ARG;
    SplitSegs segs = {};
    segs.n = n;
    int m_max = 0;
    for (int i = 0; i < n; i++) {
        const cbq_split_matrix *m = mats[i];
        if (!m || !m->cwords || !m->row_off || !m->raw || !m->lut || !outs[i] || Ms[i] <= 0)
            return CK_ERR_ARG;
        if (m->n_chunks != (int64_t)Ms[i] * (K / kSChunk)) return CK_ERR_ARG;
        if (((uintptr_t)m->raw & 15) != 0) return CK_ERR_ARG;
        SplitSeg &g = segs.s[i];
        g.cwords = m->cwords;
        g.row_off = m->row_off;
        g.raw = m->raw;
        g.lut = m->lut;
        g.out = outs[i];
        g.M = Ms[i];
        m_max = std::max(m_max, Ms[i]);
    }
    // waves per block: 16 unless that leaves CUs idle
    const int per = m_max / cbq_num_cus();
    const int nw = per >= 16 ? 16 : per >= 8 ? 8 : 4;
    int blocks = 0;
    for (int i = 0; i < n; i++) {
        SplitSeg &g = segs.s[i];
        g.block0 = blocks;
        g.nblocks = std::max(1, std::min(cbq_num_cus(), (g.M + nw - 1) / nw));
        blocks += g.nblocks;
    }
#define CBQ_SPLIT(NWV, MODE)                                                                      \
    hipLaunchKernelGGL((split_gemv_kernel<NWV, MODE>), dim3(blocks), dim3(NWV * CBQ_WAVE), 0,     \
                       stream, x, segs, K, x1, h_out, eps)
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
    return cbq_launch_status("split_gemv_kernel");
}

}  // extern "C"
