/*
 * cbq_oracle.c -- CPU restatement of the reference compressed-matmul kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in codebook-quantization_amd/csrc.  Only tests/, the smoke() entry
 * and the cpu_baseline leg of bench.py may load it; the product path never
 * links or calls it.
 *
 * Each function restates one routine of the reference file
 * /root/reference/src/compressed_matmul.c with the same arithmetic order:
 *   - fixed-width index read          : compressed_matmul.c:334-354
 *   - fixed-width GEMV (row range)    : compressed_matmul.c:416-450
 *   - fixed-width GEMV (serial)       : compressed_matmul.c:376-405
 *   - MSB-first bit peek              : compressed_matmul.c:121-131
 *   - one Huffman symbol (LUT + slow) : compressed_matmul.c:146-186
 *   - Huffman GEMV (row range)        : compressed_matmul.c:208-239
 *   - Huffman embedding rows          : compressed_matmul.c:253-281
 *   - Huffman decode to weights       : compressed_matmul.c:296-322
 * plus the GPU embedding closed form of rocm/compressed_kernel.hip:103-120.
 *
 * Accumulation is fp32, k ascending, token loop innermost, exactly as the
 * reference; it is compiled with the reference wrapper's flags
 * (-O3 -march=native -funroll-loops -fopenmp, compressed_matmul_cpu.py:88-91)
 * except that -march=native becomes -march=x86-64-v3 (AVX2 + FMA), so the
 * library also runs on other x86 hosts; gcc makes the same multiply-add
 * contraction choices either way.
 */
#include <stdint.h>
#include <string.h>

/* ---- fixed-width indices (LSB-first bitstream) --------------------------- */

/* Index `elem` of a b-bit LSB-first stream: a little-endian 32-bit window
 * read at byte elem*b/8, shifted by elem*b mod 8 (compressed_matmul.c:334-347).
 * Needs 3 readable bytes past the byte holding the index's first bit. */
static inline int oracle_index_at(const uint8_t *packed, int64_t elem, int bits)
{
    const int64_t first_bit = elem * (int64_t)bits;
    const uint8_t *p = packed + (first_bit >> 3);
    uint32_t window = (uint32_t)p[0] | ((uint32_t)p[1] << 8) |
                      ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    return (int)((window >> (first_bit & 7)) & ((1u << bits) - 1u));
}

void oracle_unpack_indices(const uint8_t *packed, int64_t n, int bits,
                           int32_t *out)
{
    for (int64_t i = 0; i < n; i++)
        out[i] = bits == 8 ? (int32_t)packed[i] : oracle_index_at(packed, i, bits);
}

/* Rows [r_start, r_end) of out[t*M + r] += x[t*K + k] * cb[min(idx, C-1)].
 * out is accumulated, so the caller zeroes it (compressed_matmul.c:416-450). */
void oracle_fixed_gemv_rows(const float *x, const uint8_t *packed,
                            const float *cb, float *out,
                            int T, int M, int K, int C, int bits,
                            int r_start, int r_end)
{
    if (r_end > M) r_end = M;
    #pragma omp parallel for schedule(dynamic, 64)
    for (int r = r_start; r < r_end; r++) {
        const int64_t row0 = (int64_t)r * K;
        for (int k = 0; k < K; k++) {
            int idx = bits == 8 ? (int)packed[row0 + k]
                                : oracle_index_at(packed, row0 + k, bits);
            if (idx >= C) idx = C - 1;
            const float w = cb[idx];
            for (int t = 0; t < T; t++)
                out[t * M + r] += x[t * K + k] * w;
        }
    }
}

/* Single-threaded whole-matrix variant (compressed_matmul.c:376-405). */
void oracle_fixed_gemv_serial(const float *x, const uint8_t *packed,
                              const float *cb, float *out,
                              int T, int M, int K, int C, int bits)
{
    for (int r = 0; r < M; r++) {
        const int64_t row0 = (int64_t)r * K;
        for (int k = 0; k < K; k++) {
            int idx = bits == 8 ? (int)packed[row0 + k]
                                : oracle_index_at(packed, row0 + k, bits);
            if (idx >= C) idx = C - 1;
            const float w = cb[idx];
            for (int t = 0; t < T; t++)
                out[t * M + r] += x[t * K + k] * w;
        }
    }
}

/* out[t, h] = cb[min(idx[ids[t]*H + h], C-1)]  (rocm/compressed_kernel.hip:103-120). */
void oracle_fixed_embedding(const int32_t *ids, const uint8_t *packed,
                            const float *cb, float *out,
                            int T, int H, int C, int bits)
{
    for (int t = 0; t < T; t++) {
        const int64_t row0 = (int64_t)ids[t] * H;
        for (int h = 0; h < H; h++) {
            int idx = bits == 8 ? (int)packed[row0 + h]
                                : oracle_index_at(packed, row0 + h, bits);
            if (idx >= C) idx = C - 1;
            out[(int64_t)t * H + h] = cb[idx];
        }
    }
}

/* ---- canonical Huffman (MSB-first bitstream) ----------------------------- */

#define ORACLE_LUT_BITS 12

/* n (<= 25) bits at bit_pos, first stream bit in the result's bit n-1
 * (compressed_matmul.c:121-131).  Needs 4 readable bytes from bit_pos/8. */
static inline uint32_t oracle_peek_msb(const uint8_t *s, int64_t bit_pos, int n)
{
    const uint8_t *p = s + (bit_pos >> 3);
    uint32_t w = ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) |
                 ((uint32_t)p[2] << 8) | (uint32_t)p[3];
    return (w << (bit_pos & 7)) >> (32 - n);
}

/* One symbol at *bit_pos (compressed_matmul.c:148-186): 12-bit table when
 * lut_len[key] > 0, else extend one bit at a time for L = 13..max_len testing
 * 0 <= code - first[L] < base[L+1] - base[L]; no match -> symbol 0, +1 bit. */
static inline int oracle_next_symbol(const uint8_t *s, int64_t *bit_pos,
                                     const uint16_t *lut_sym, const uint8_t *lut_len,
                                     const int64_t *sl_first, const int32_t *sl_base,
                                     const uint16_t *sl_sym, int max_len)
{
    const uint32_t key = oracle_peek_msb(s, *bit_pos, ORACLE_LUT_BITS);
    const int len = (int)lut_len[key];
    if (len > 0) {
        *bit_pos += len;
        return (int)lut_sym[key];
    }
    uint32_t code = key;
    for (int L = ORACLE_LUT_BITS + 1; L <= max_len; L++) {
        code = (code << 1) | oracle_peek_msb(s, *bit_pos + (L - 1), 1);
        const int64_t first = sl_first[L];
        if (first < 0) continue;
        const int64_t delta = (int64_t)code - first;
        if (delta >= 0 && delta < (int64_t)(sl_base[L + 1] - sl_base[L])) {
            *bit_pos += L;
            return (int)sl_sym[sl_base[L] + (int)delta];
        }
    }
    *bit_pos += 1;
    return 0;
}

/* Rows [r_start, r_end): decode K symbols from row_bit_starts[r], clamp to
 * C-1, accumulate like the fixed-width kernel (compressed_matmul.c:208-239). */
void oracle_huff_gemv_rows(const float *x, const uint8_t *stream,
                           const uint16_t *lut_sym, const uint8_t *lut_len,
                           const int64_t *sl_first, const int32_t *sl_base,
                           const uint16_t *sl_sym, const int64_t *row_bit_starts,
                           const float *cb, float *out,
                           int T, int M, int K, int C,
                           int r_start, int r_end, int max_len)
{
    if (r_end > M) r_end = M;
    #pragma omp parallel for schedule(dynamic, 64)
    for (int r = r_start; r < r_end; r++) {
        int64_t pos = row_bit_starts[r];
        for (int k = 0; k < K; k++) {
            int sym = oracle_next_symbol(stream, &pos, lut_sym, lut_len,
                                         sl_first, sl_base, sl_sym, max_len);
            if (sym >= C) sym = C - 1;
            const float w = cb[sym];
            for (int t = 0; t < T; t++)
                out[t * M + r] += x[t * K + k] * w;
        }
    }
}

/* out[t, :] = cb[decode(row ids[t])], overwritten (compressed_matmul.c:253-281). */
void oracle_huff_embedding_rows(const int32_t *ids, const uint8_t *stream,
                                const uint16_t *lut_sym, const uint8_t *lut_len,
                                const int64_t *sl_first, const int32_t *sl_base,
                                const uint16_t *sl_sym, const int64_t *row_bit_starts,
                                const float *cb, float *out,
                                int T, int H, int C, int max_len)
{
    #pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++) {
        int64_t pos = row_bit_starts[(int64_t)ids[t]];
        float *dst = out + (int64_t)t * H;
        for (int h = 0; h < H; h++) {
            int sym = oracle_next_symbol(stream, &pos, lut_sym, lut_len,
                                         sl_first, sl_base, sl_sym, max_len);
            if (sym >= C) sym = C - 1;
            dst[h] = cb[sym];
        }
    }
}

/* W[r, k] = cb[decode], overwritten (compressed_matmul.c:296-322).  With
 * cb[i] = i this returns the decoded indices exactly (i < 2^24). */
void oracle_huff_decode_weights(const uint8_t *stream,
                                const uint16_t *lut_sym, const uint8_t *lut_len,
                                const int64_t *sl_first, const int32_t *sl_base,
                                const uint16_t *sl_sym, const int64_t *row_bit_starts,
                                const float *cb, float *out,
                                int M, int K, int C, int max_len)
{
    #pragma omp parallel for schedule(dynamic, 64)
    for (int r = 0; r < M; r++) {
        int64_t pos = row_bit_starts[r];
        float *dst = out + (int64_t)r * K;
        for (int k = 0; k < K; k++) {
            int sym = oracle_next_symbol(stream, &pos, lut_sym, lut_len,
                                         sl_first, sl_base, sl_sym, max_len);
            if (sym >= C) sym = C - 1;
            dst[k] = cb[sym];
        }
    }
}

/* Decoded symbol indices of rows [0, M) without the codebook clamp: the
 * bit-exact index oracle used against the GPU decoder. */
void oracle_huff_decode_indices(const uint8_t *stream,
                                const uint16_t *lut_sym, const uint8_t *lut_len,
                                const int64_t *sl_first, const int32_t *sl_base,
                                const uint16_t *sl_sym, const int64_t *row_bit_starts,
                                int32_t *out, int M, int K, int max_len)
{
    #pragma omp parallel for schedule(dynamic, 64)
    for (int r = 0; r < M; r++) {
        int64_t pos = row_bit_starts[r];
        int32_t *dst = out + (int64_t)r * K;
        for (int k = 0; k < K; k++)
            dst[k] = oracle_next_symbol(stream, &pos, lut_sym, lut_len,
                                        sl_first, sl_base, sl_sym, max_len);
    }
}
