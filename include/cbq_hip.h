/*
 * cbq_hip.h -- C ABI of the MI355X (gfx950) always-compressed matmul library
 * (libcbq_hip.so, built from codebook-quantization_amd/csrc).
 *
 * Weights stay as codebook indices in HBM: fixed-width b-bit indices
 * (LSB-first bitstream, index i at bits [i*b, (i+1)*b)) or canonical-Huffman
 * codes.  Every entry point takes plain device pointers and sizes, runs
 * asynchronously on `stream` (NULL = default stream), never synchronises and
 * never allocates device memory (the two upload helpers aside).  Return codes follow the reference
 * (rocm/compressed_kernel.h:37-41, rocm/huffman_kernel.h:26-28):
 *   0 success, 1 HIP runtime error (message on stderr), 2 invalid argument.
 * Kernel faults surface asynchronously, as with any HIP launch.
 *
 * Layouts: W is [M = out, K = in] row-major, x is [T, K], out is [T, M];
 * accumulation is always float32.  Outputs are written, never accumulated,
 * so callers need not zero them.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CK_SUCCESS  0
#define CK_ERR_HIP  1
#define CK_ERR_ARG  2
#define HK_SUCCESS  CK_SUCCESS
#define HK_ERR_HIP  CK_ERR_HIP
#define HK_ERR_ARG  CK_ERR_ARG

/* Human-readable text for a return code.
 * Replaces ck_error_string (rocm/compressed_kernel.h:41). */
const char *ck_error_string(int err);

/* ==== fixed-width codebook GEMV / skinny GEMM ============================ */

/* out[t, m] = sum_k x[t, k] * codebook[min(idx[m*K + k], C-1)], float32 x/out.
 * packed: ceil(M*K*bits/8) bytes + >= 4 pad bytes; 1 <= bits <= 16.
 * Replaces ck_linear_f32 (rocm/compressed_kernel.h:52-59); same arguments.
 * Any T >= 1 (T > 16 runs as successive 16-token tiles). */
int ck_linear_f32(const float *x, const uint8_t *packed, const float *codebook,
                  float *out, int T, int M, int K, int C, int bits,
                  hipStream_t stream);

/* Workspace bytes cbq_linear_f32_ws splits K with for a T x M x K product
 * (0: no split).  No counterpart in the reference. */
size_t cbq_linear_f32_workspace(int T, int M, int K);

/* ck_linear_f32 with a caller workspace: for T >= 64 on the fp32 MFMA path
 * (widths 8 and 10..13), grids under two blocks per CU split K across
 * blocks that write fp32 partials to `workspace` (>= cbq_linear_f32_workspace
 * bytes, 16-byte aligned), summed in split order by a second kernel.  With a
 * smaller workspace it is ck_linear_f32.  No counterpart in the reference:
 * batched fp32 tokens through GPUAcceleratedLinear
 * (src/gpu_accelerated_functions.py:928-950), e.g. a prompt prefill. */
int cbq_linear_f32_ws(const float *x, const uint8_t *packed, const float *codebook, float *out,
                      int T, int M, int K, int C, int bits, void *workspace, size_t ws_bytes,
                      hipStream_t stream);

/* Fixed-width GEMV with an implicit (affine) codebook: index i stands for
 * the bf16 value with bit pattern lo + i (i < w), 0x8000 + lo + i - w
 * (w <= i < 2w), and 0.0 for i >= 2w.  This is the load-time re-indexed
 * form of a lossless bf16 codebook whose nonzero magnitudes all lie in
 * [lo, lo + w) (every frequency-sorted codebook of normally distributed
 * weights qualifies); the decoded weights are the codebook's values
 * bit-for-bit, without an LDS table gather.  float32 x/out, any T (tiles of
 * 16); K % 32 == 0; x and packed 4-byte aligned; 1 <= lo, lo + w <= 0x8000,
 * 2w <= 2^bits, bits in {8, 10..14}.  No counterpart in the reference: an
 * alternative resident form behind ck_linear_f32's interface. */
int cbq_linear_affine_f32(const float *x, const uint8_t *packed, uint32_t lo, uint32_t w,
                          float *out, int T, int M, int K, int bits, hipStream_t stream);

/* Same with bfloat16 x and out (raw uint16 bf16 bit patterns; out rounded to
 * nearest even).  Replaces ck_linear_bf16 (rocm/compressed_kernel.h:66-73). */
int ck_linear_bf16(const void *x_bf16, const uint8_t *packed, const float *codebook,
                   void *out_bf16, int T, int M, int K, int C, int bits,
                   hipStream_t stream);

/* Workspace bytes of cbq_linear_bf16_ws for a T x M x K product: room for a
 * copy of x in MFMA fragment order, plus fp32 partials when K is split (0:
 * the shape does not take the MFMA path).  No counterpart in the reference. */
size_t cbq_linear_bf16_workspace(int T, int M, int K);

/* ck_linear_bf16 with a caller workspace (>= cbq_linear_bf16_workspace
 * bytes, 256-byte aligned).  For T >= 64 on the MFMA path x is first copied
 * to fragment order in the workspace (each wave's operand loads are then
 * contiguous), and when the output tiles alone would leave CUs idle, K is
 * split across blocks that write fp32 partials there too, summed in split
 * order by a second kernel.  With a smaller workspace it is ck_linear_bf16.
 * No counterpart in the reference: the prefill of GPUAcceleratedLinear
 * (src/gpu_accelerated_functions.py:928-950) for batched tokens. */
int cbq_linear_bf16_ws(const void *x_bf16, const uint8_t *packed, const float *codebook,
                       void *out_bf16, int T, int M, int K, int C, int bits, void *workspace,
                       size_t ws_bytes, hipStream_t stream);

/* ==== compressed embedding gather ======================================== */

/* out[t, h] = codebook[min(idx[ids[t]*H + h], C-1)], float32 out.  ids are
 * trusted, as in the reference.
 * Replaces ck_embedding_f32 (rocm/compressed_kernel.h:83-90). */
int ck_embedding_f32(const int32_t *token_ids, const uint8_t *packed,
                     const float *codebook, float *out, int T, int H, int C,
                     int bits, hipStream_t stream);

/* As ck_embedding_f32 with the table's row count: ids outside [0, vocab)
 * are clamped into range instead of read out of bounds.
 * Backs GPUAcceleratedEmbedding.__call__
 * (src/gpu_accelerated_functions.py:1005-1029). */
int cbq_embedding_f32(const int32_t *token_ids, const uint8_t *packed,
                      const float *codebook, float *out, int T, int vocab, int H,
                      int C, int bits, hipStream_t stream);

/* ==== canonical Huffman: reference-format entry points ==================== */

/* Decode a row-indexed MSB-first Huffman stream into int32 indices [M*K] with
 * the reference's tables (12-bit int32 LUT, -1 = no short code; int32
 * slow-path tables; corrupt prefix -> symbol 0, +1 bit).
 * Replaces huff_decode_to_i32 (rocm/huffman_kernel.h:57-67). */
int huff_decode_to_i32(const void *stream, const void *row_bit_start,
                       const void *lut_sym, const void *lut_len,
                       const void *sl_first_code, const void *sl_base_offset,
                       const void *sl_sym, void *out, int M, int K,
                       int max_code_len, hipStream_t stream_h);

/* GEMV over int32 indices (clamped to [0, C-1]).
 * Replaces huff_i32_linear_f32 (rocm/huffman_kernel.h:81-87). */
int huff_i32_linear_f32(const void *x, const void *i32_indices, const void *codebook,
                        void *out, int T, int M, int K, int C, hipStream_t stream_h);

/* Gather over int32 indices.
 * Replaces huff_i32_embedding_f32 (rocm/huffman_kernel.h:101-107). */
int huff_i32_embedding_f32(const void *token_ids, const void *i32_indices,
                           const void *codebook, void *out, int T, int H, int C,
                           hipStream_t stream_h);

/* ==== canonical Huffman: fused chunk-parallel path ========================= *
 *
 * Device stream format ("chunked Huffman"):
 *   words     uint32, the reference's MSB-first byte stream with the bits of
 *             every byte reversed, read as little-endian words, so stream bit
 *             j is bit j%32 of word j/32; >= 2 zero words of padding.
 *   chunk_off uint64[n_chunks + 1]: bit offset of flat symbol c*4096.
 *   sub_len   uint16[ceil(N/64)]: bits taken by symbols [64s, 64s+64).
 *   lut1      uint32[4096] and lut2 uint32[n_lut2]: decode tables built by
 *             cbq_huff_build_luts from the code lengths and the codebook.
 *   canon     int32[3*33] + canon_sym: per-length first code / count / base
 *             and symbols in canonical order, for codes beyond 24 bits.
 * Decoding is bit-exact with the reference decoder (compressed_matmul.c:
 * 146-186) for every bit pattern, including corrupt ones.
 */

/* Device-resident chunked-Huffman stream: plain device pointers + sizes. */
typedef struct cbq_huff_stream {
    const uint32_t *words;      /* LSB-first stream words (+ >= 2 zero words)   */
    int64_t n_words;            /* length of `words`                             */
    const uint64_t *chunk_off;  /* [ceil(N/4096) + 1] bit offsets                */
    const uint16_t *sub_len;    /* [ceil(N/64)] sub-block bit lengths            */
    const uint32_t *lut1;       /* [4096]                                        */
    const uint32_t *lut2;       /* [n_lut2]                                      */
    int32_t n_lut2;
    const int32_t *canon;       /* [100]: first[33] count[33] base[33] invalid   */
    const int32_t *canon_pay;   /* payloads in canonical symbol order            */
    const float *value_cb;      /* NULL: payloads are bf16 values; else float32
                                   codebook[C] indexed by the (clamped) symbol   */
    int32_t C;
    int32_t stage_words;        /* LDS words staged per wave (0 = default 1536);
                                   larger chunks decode from global memory       */
} cbq_huff_stream;

/* Table builder (host only, no GPU needed).  payload_is_value != 0 stores
 * the bf16 bits of codebook[min(sym, C-1)] (valid only when every codebook
 * value is exactly a bf16); 0 stores the symbol (clamped to C-1 when
 * clamp_to != 0, else raw).  With lut1 or lut2 NULL only *n_lut2 (and canon
 * / canon_pay when non-NULL) are written.  canon_pay needs one slot per used
 * symbol.  Returns CK_ERR_ARG on invalid lengths (Kraft sum > 1, > 32 bits).
 * Tables follow the reference's build_gpu_lut / _build_slow_path_tables
 * (src/huffman_codebook.py:353-423) in meaning, not layout. */
int cbq_huff_build_luts(const uint8_t *lengths, int n_alpha, const float *codebook,
                        int C, int payload_is_value, int clamp_to,
                        uint32_t *lut1, uint32_t *lut2, int *n_lut2,
                        int32_t *canon, int32_t *canon_pay);

/* Host indexer: decode the reference-format MSB-first stream once (up to
 * `threads` threads, split at row starts) and write chunk_off[ceil(N/4096)+1]
 * and sub_len[ceil(N/64)] for N = M*K.  row_bit_starts[M] may be NULL (one
 * thread).  Returns CK_ERR_ARG when the row starts disagree with the stream.
 * Derived from huff_row_bit_starts (src/huffman_codebook.py:210-215). */
int cbq_huff_index_stream(const uint8_t *stream_msb, int64_t stream_bytes,
                          const uint8_t *lengths, int n_alpha,
                          const int64_t *row_bit_starts, int M, int K,
                          uint64_t *chunk_off, uint16_t *sub_len, int threads);

/* Fused Huffman GEMV: out[t, m] = sum_k x[t, k] * codebook[decode(m*K + k)],
 * decoded chunk-parallel straight into the dot product; no index or weight
 * buffer.  Requires K % 64 == 0 and 1 <= T <= 16.
 * Replaces the decode + GEMV pair of HuffmanCodebookLinear.__call__
 * (src/gpu_huffman_functions.py:834-855) and huffman_matmul_f32_chunk
 * (src/compressed_matmul.c:208-239). */
int cbq_huff_linear_f32(const float *x, const cbq_huff_stream *hs, float *out,
                        int T, int M, int K, hipStream_t stream);

/* Fused Huffman embedding: out[t, h] = codebook[decode(ids[t]*H + h)]; only
 * the requested rows are decoded (ids clamped to [0, vocab)).  H % 64 == 0.
 * Replaces HuffmanCodebookEmbedding.__call__
 * (src/gpu_huffman_functions.py:961-979) and huffman_embedding_f32_rows
 * (src/compressed_matmul.c:253-281). */
int cbq_huff_embedding_f32(const int32_t *token_ids, const cbq_huff_stream *hs,
                           float *out, int T, int vocab, int H, hipStream_t stream);

/* Column layout of a chunked stream, built on the device by
 * cbq_huff_column_rows + cbq_huff_columnize: chunk c's 64 sub-blocks side by
 * side, sub-block l's bits LSB-first in cwords[(row_off[c] + r) * 64 + l],
 * r < rows(c) = max_l ceil(sub_len / 32); bits past a sub-block are 0 and
 * 4 zero rows follow the last chunk.  No counterpart in the reference: a
 * load-time re-layout of its stream (same codes, ~6% more bytes) so that the
 * GEMV's window reads are free of LDS bank conflicts. */
typedef struct cbq_huff_columns {
    const uint32_t *cwords;     /* [(row_off[n_chunks] + 4) * 64]                */
    const uint32_t *row_off;    /* [n_chunks + 1], row_off[0] = 0               */
    int64_t n_chunks;           /* ceil(n_symbols / 4096)                        */
    const uint32_t *ulut1;      /* optional unified tables (cbq_huff_build_ulut) */
    const uint32_t *ulut2;      /*   replacing hs->lut1 / lut2 in the GEMV; NULL */
    int32_t n_ulut2;            /*   = use hs's tables                           */
} cbq_huff_columns;

/* Unified decode tables for bf16-value payloads of codes <= 24 bits (host
 * only): every ulut1[4096] entry is (base << 18) | nb and the code's leaf is
 * ulut2[base + next nb stream bits] (short codes: nb = 0, one leaf per
 * symbol), so the GEMV step needs no leaf/pointer select.  Leaves as lut2's.
 * With ulut1 or ulut2 NULL only *n_ulut2 is written.  CK_ERR_ARG for
 * invalid lengths, codes beyond 24 bits or more than 16383 entries. */
int cbq_huff_build_ulut(const uint8_t *lengths, int n_alpha, const float *codebook, int C,
                        uint32_t *ulut1, uint32_t *ulut2, int *n_ulut2);

/* rows[c] = max(1, max_l ceil(sub_len[64 c + l] / 32)) for every chunk; the
 * caller's exclusive prefix sum of rows is row_off.  Needs hs->sub_len. */
int cbq_huff_column_rows(const cbq_huff_stream *hs, int64_t n_symbols, uint32_t *rows,
                         hipStream_t stream);

/* Fill cwords (zeroed by the caller, (row_off[n_chunks] + 4) * 64 words)
 * from the stream's words / chunk_off / sub_len. */
int cbq_huff_columnize(const cbq_huff_stream *hs, int64_t n_symbols, const uint32_t *row_off,
                       uint32_t *cwords, hipStream_t stream);

/* cbq_huff_linear_f32 for T = 1 over the column layout: out[m] =
 * sum_k x[k] * value(decode(m*K + k)).  Uses hs's tables only (bf16-value
 * payloads, value_cb NULL, n_lut2 <= 8192); K % 4096 == 0.  Same result as
 * cbq_huff_linear_f32 (same per-lane accumulation order). */
int cbq_huff_linear_col_f32(const float *x, const cbq_huff_stream *hs,
                            const cbq_huff_columns *cols, float *out, int M, int K,
                            hipStream_t stream);

/* One launch of cbq_huff_linear_col_f32 for n <= 4 matrices that share x
 * and K (a layer's q/k/v, each with its own Huffman code): outs[i] =
 * W_i x, W_i [Ms[i], K] described by hs[i] / cols[i] (host arrays of
 * pointers).  Each block of the grid serves one matrix, so small matrices
 * run side by side instead of one after another.  No counterpart in the
 * reference.  Results equal n single calls bit for bit. */
int cbq_huff_linear_col_multi_f32(const float *x, int n, const cbq_huff_stream *const *hs,
                                  const cbq_huff_columns *const *cols, float *const *outs,
                                  const int *Ms, int K, hipStream_t stream);

/* Activation transforms a single-token GEMV applies while staging x, which
 * replace the decoder's separate glue launches (include/cbq_decode.h):
 *   CBQ_XF_SILU     x = silu(x0) * x1                 (the down projection)
 *   CBQ_XF_ADD_RMS  h = x0 + x1, x = rmsnorm(h); one block stores h to
 *                   h_out (NULL: not stored)          (a layer's first GEMVs)
 *   CBQ_XF_RMS      x = rmsnorm(x0)
 * RMSNorm has unit weight and the reduction order of cbq_add_rmsnorm_f32,
 * and every step rounds as the separate kernels do, so fused and unfused
 * decoders produce identical values.  K <= 16384 in every mode.  No
 * counterpart in the reference (its glue is HF PyTorch code). */
#define CBQ_XF_SILU    1
#define CBQ_XF_ADD_RMS 2
#define CBQ_XF_RMS     3

/* ck_linear_f32 for T = 1 with x = transform(x0, x1) (mode above); fixed
 * width widths {8, 10..14}, K % 32 == 0, C <= 16384, packed 4-byte aligned;
 * CK_ERR_ARG otherwise (use the plain entry point and the glue kernels). */
int cbq_linear_xform_f32(const float *x0, const float *x1, float *h_out, int mode, float eps,
                         const uint8_t *packed, const float *codebook, float *out, int M, int K,
                         int C, int bits, hipStream_t stream);

/* The gated MLP's gate and up projections in one launch, with the SiLU
 * product in the epilogue: packed holds 2M rows, gate_proj's M rows then
 * up_proj's (the row-stacked [gate; up] matrix ck_linear_f32 takes), and
 * out[j] = silu(gate_j . x) * (up_j . x) for j < M, with x =
 * transform(x0, x1) (mode 0, CBQ_XF_ADD_RMS or CBQ_XF_RMS).  Each product
 * sums as in cbq_linear_xform_f32 and the SiLU product rounds as
 * cbq_silu_mul_f32, so out equals those two calls bit for bit.  Same widths
 * and limits as cbq_linear_xform_f32.  Replaces the reference's separate
 * gate_proj / up_proj module calls and HF's act_fn(gate) * up
 * (src/compressed_modules.py:77-490 modules inside HF's Qwen3MLP). */
int cbq_linear_xform_glu_f32(const float *x0, const float *x1, float *h_out, int mode,
                             float eps, const uint8_t *packed, const float *codebook, float *out,
                             int M, int K, int C, int bits, hipStream_t stream);

/* cbq_huff_linear_col_multi_f32 with x = transform(x0, x1) (mode above, or
 * 0 for none); modes other than 0 need every matrix's unified tables. */
int cbq_huff_linear_col_xform_f32(const float *x0, const float *x1, float *h_out, int mode,
                                  float eps, int n, const cbq_huff_stream *const *hs,
                                  const cbq_huff_columns *const *cols, float *const *outs,
                                  const int *Ms, int K, hipStream_t stream);

/* ---- Split device format (no counterpart in the reference) ----------------
 * A load-time re-encoding of a Huffman-coded matrix whose codebook values are
 * all bf16 numbers, for the single-token GEMV that HuffmanCodebookLinear
 * runs for T = 1 (src/gpu_huffman_functions.py:834-855): one raw byte per
 * weight (the low byte of its bf16 bits, natural order) and the high byte
 * (sign, exponent bits 7..1) Huffman-coded with codes of at most 7 bits,
 * LSB-first per 64-weight sub-block, stored in the column layout (chunk c =
 * 4096 weights owns rows row_off[c] .. row_off[c+1]-1 of 64 words, at most
 * 14).  lut[j] for the next 14 stream bits j (always two whole codes) is
 * hi1 << 24 | hi2 << 16 | (len1 + len2).  n_symbols % 4096 == 0. */
typedef struct cbq_split_matrix {
    const uint32_t *cwords;   /* total rows x 64 words, then 3 readable rows, 16-byte aligned */
    const uint32_t *row_off;  /* [n_chunks + 1] */
    const uint8_t *raw;       /* [n_chunks * 4096] low bytes, 16-byte aligned */
    const uint32_t *lut;      /* [16384], 16-byte aligned */
    int64_t n_chunks;
} cbq_split_matrix;

/* Build, step 1: sub_bits[s] = code bits of sub-block s (64 symbols) of the
 * decoded indices; sym_code[i] = bit-reversed high-byte code of symbol i |
 * len << 24 (indices clamp to [0, n_sym)).  The caller derives row_off:
 * rows(c) = max(1, ceil(max over the chunk's 64 sub_bits / 32)). */
int cbq_split_bits(const int32_t *indices, int64_t n_symbols, const uint32_t *sym_code, int n_sym,
                   uint32_t *sub_bits, hipStream_t stream);

/* Build, step 2: writes the column words (every row of every chunk) and the
 * raw bytes (sym_raw[i]: the low byte of symbol i's bf16 value). */
int cbq_split_pack(const int32_t *indices, int64_t n_symbols, const uint32_t *sym_code,
                   const uint8_t *sym_raw, int n_sym, const uint32_t *row_off, uint32_t *cwords,
                   uint8_t *raw, hipStream_t stream);

/* y_i[M_i] = W_i @ x for up to four split-format matrices sharing x (T = 1,
 * K % 1024 == 0, M_i * K % 4096 == 0), with x = transform(x0, x1) as
 * cbq_linear_xform_f32 (mode 0: x0 itself).  With K % 4096 == 0 the outputs
 * equal cbq_huff_linear_col_f32's on the same weights bit for bit; other K
 * walk groups of 4096 / gcd(K, 4096) rows (whole chunks).  Replaces the
 * T = 1 decode + GEMV of HuffmanCodebookLinear.__call__
 * (src/gpu_huffman_functions.py:834-855). */
int cbq_split_linear_f32(const float *x0, const float *x1, float *h_out, int mode, float eps, int n,
                         const cbq_split_matrix *const *mats, float *const *outs, const int *Ms,
                         int K, hipStream_t stream);

/* The gated MLP's gate and up projections in one launch over the split
 * format, with the SiLU product in the epilogue: m holds 2M rows, gate_proj's
 * M rows then up_proj's, coded with one shared table (the two matrices share
 * their category codebook), and out[j] = silu(gate_j . x) * (up_j . x) for
 * j < M, x = transform(x0, x1) (mode 0, CBQ_XF_ADD_RMS or CBQ_XF_RMS).  Each
 * product sums as cbq_split_linear_f32 does and the SiLU product rounds as
 * cbq_silu_mul_f32, so out equals those calls bit for bit.  K % 4096 == 0;
 * K <= 16384 for the norms.  Replaces the reference's separate gate_proj /
 * up_proj Huffman module calls and HF's act_fn(gate) * up
 * (src/gpu_huffman_functions.py:834-855 inside HF's Qwen3MLP). */
int cbq_split_linear_glu_f32(const float *x0, const float *x1, float *h_out, int mode, float eps,
                             const cbq_split_matrix *m, float *out, int M, int K,
                             hipStream_t stream);

/* Decode flat symbols [0, n_symbols) to int32 with the chunked kernel (lut
 * payloads must be raw symbols).  The bit-exact check of the fused decoder;
 * the equivalent of huffman_decode_to_weights_f32 with an identity codebook
 * (src/compressed_matmul.c:296-322). */
int cbq_huff_decode_indices(const cbq_huff_stream *hs, int32_t *out,
                            int64_t n_symbols, hipStream_t stream);

/* Packs n int32 indices (n % 32 == 0, clamped to [0, 2^bits - 1]) into the
 * reference's LSB-first fixed-width stream (src/bitpack.py:32-95), bits in
 * {8, 10, 11, 12, 13}; packed 4-byte aligned, n * bits / 8 bytes.  No
 * counterpart on the GPU in the reference: the batched-token (prefill) path
 * of a Huffman module decodes its stream with cbq_huff_decode_indices, packs
 * it here and runs ck_linear_f32's matrix-core GEMM on the transient copy. */
int cbq_pack_indices(const int32_t *indices, int64_t n, int bits, uint8_t *packed,
                     hipStream_t stream);

/* Decodes a split-format matrix (cbq_split_matrix, n_chunks chunks of 4096
 * weights) straight to the LSB-first fixed-width stream of its codebook
 * indices, bits in {8, 10, 11, 12, 13, 16, 32} (16: little-endian uint16,
 * 32: int32 indices): inv maps every bf16 bit pattern of the codebook to an
 * index holding that value (65536 uint16 entries); packed (4-byte aligned)
 * receives n_chunks * 4096 * bits / 8 bytes.  No counterpart in the
 * reference: the batched-token path of a Huffman module whose split format
 * exists (one table read per two weights instead of the stream decode to
 * int32 and cbq_pack_indices), and, with bits = 32, its index decode
 * (huffman_decode_to_weights_f32 with an identity codebook,
 * src/compressed_matmul.c:296-322) when the codebook's values are distinct. */
int cbq_split_to_packed(const cbq_split_matrix *m, const uint16_t *inv, int bits,
                        uint8_t *packed, hipStream_t stream);

/* y_i[T, M_i] = x[T, K] @ W_i^T for up to four split-format matrices sharing
 * x (one launch), any T >= 1 (fp32 x and outputs, 16-byte aligned x), in
 * launches of up to 16 tokens: every weight is decoded once per launch into
 * LDS and multiplied on the bf16 matrix cores (x split exactly into three
 * bf16 parts), never written out.  K % 4096 == 0, or K % 1024 == 0 with
 * the rows of a 4096-weight chunk group tiling 16 waves (K = 1024, 2048,
 * 3072, 5120, 6144, 7168; M_i a multiple of 4096 / gcd(K, 4096)); M_i * K a
 * whole number of chunks; other shapes return CK_ERR_ARG.  ws (16-byte
 * aligned, at least cbq_split_fewtok_ws_bytes(K) bytes, or NULL): x's three
 * bf16 parts are written there once per 16 tokens in fragment order and
 * read ready-made, instead of every lane splitting its x in the GEMM; the
 * shapes whose row tiles need two MFMA passes per phase (K = 3072, 5120,
 * 6144, 7168) require it.  Never allocates.
 * Replaces, for Huffman
 * modules whose split format exists, the batched-token path of
 * huffman_matmul (src/compressed_matmul.c:208-239 over several rows of x,
 * src/gpu_huffman_functions.py:834-855), which decodes to a transient index
 * buffer first (rocm/huffman_kernel.hip:61-156). */
int cbq_split_linear_fewtok_f32(const float *x, int T, int n, const cbq_split_matrix *const *mats,
                                float *const *outs, const int *Ms, int K, void *ws,
                                size_t ws_bytes, hipStream_t stream);

/* Workspace bytes cbq_split_linear_fewtok_f32 uses at this K (96 K); no
 * counterpart in the reference. */
size_t cbq_split_fewtok_ws_bytes(int K);

/* ==== upload helpers ===================================================== */

/* Allocate device memory (hipMalloc) and copy `nbytes` host bytes into it
 * synchronously; NULL on failure (message on stderr) or when the source is
 * NULL / empty.  The caller hipFree()s the pointer.  These two are the only
 * entry points that allocate.  ck_upload_packed takes the packed stream as
 * the caller has it: ceil(M*K*bits/8) bytes plus the >= 4 pad bytes
 * ck_linear_f32 requires.
 * Replace ck_upload_packed / ck_upload_codebook
 * (rocm/compressed_kernel.h:153-161); same arguments and ownership. */
uint8_t *ck_upload_packed(const uint8_t *host_packed, size_t nbytes);
float *ck_upload_codebook(const float *host_codebook, int C);

/* ==== library introspection ============================================== */

/* Version string of the library build. */
const char *cbq_version(void);

/* Diagnostics: in a library built with -DCBQ_TIMELINE
 * (build_native.py --timeline), copies the per-wave timeline of the last
 * one-token fixed-width streaming launch: 4096 waves x 6 uint64 (clock at
 * entry, after staging, after the first ring of items, after the loop, at
 * exit, in 10 ns ticks of s_memrealtime; then the wave's item count) to
 * host memory.  CK_ERR_ARG in the normal build or when dst_bytes <
 * 4096 * 6 * 8.  No counterpart in the reference. */
int cbq_timeline_read(void *dst, size_t dst_bytes);

/* Diagnostics: in a -DCBQ_TIMELINE library, copies the per-wave timeline of
 * the last bf16 prefill GEMM launch (ck_linear_bf16 / cbq_linear_bf16_ws with
 * T >= 64): 4096 waves x 6 uint64 (clock at entry, after the codebook
 * staging, after the K loop's prologue, after the K loop, at exit, in 10 ns
 * ticks; then the wave's K steps), wave w of grid block b at index
 * 8 b + w.  CK_ERR_ARG in the normal build or when dst_bytes <
 * 4096 * 6 * 8.  No counterpart in the reference. */
int cbq_prefill_timeline_read(void *dst, size_t dst_bytes);

/* Diagnostics: in a -DCBQ_TIMELINE library, copies the per-wave timeline of
 * the last split-format row-walk GEMV launch (one token,
 * cbq_split_linear_f32 / cbq_split_linear_glu_f32): 4096 waves x 6 uint64
 * (clock at entry, after the first barrier, after the wave's first chunk,
 * after its row loop, at exit, in 10 ns ticks; then its rows), wave w of
 * block b at index 16 b + w for 16-wave blocks.  CK_ERR_ARG in the normal
 * build or when dst_bytes < 4096 * 6 * 8.  No counterpart in the
 * reference. */
int cbq_split_timeline_read(void *dst, size_t dst_bytes);

/* ---- lm_head GEMV with the greedy pick fused ------------------------------
 * The one-token GEMV of the decoder's last matrix (vocabulary rows) and the
 * greedy pick of the next token in two launches: the GEMV's epilogue reduces
 * each block's rows to one (max, first index) pair in `workspace`
 * (>= CBQ_ARGMAX_WORKSPACE bytes, 4-byte aligned, overwritten by every
 * call), and one merge block picks the token: ids32[0] = tok;
 * toks[pos[0] - first] = tok when that index lies in [0, n_toks);
 * pos[0] += 1.  Order as torch.argmax: first maximum, NaN highest.  out
 * (the logits) is written when not NULL.  No counterpart in the reference,
 * whose HF generate loop reads the logits back for the pick
 * (chat.py:264-315); the logits never make a second trip through HBM and
 * the separate reduction launch of cbq_argmax_step is saved.
 * cbq_linear_xform_argmax_f32: fixed width, x = transform(x0, x1) as
 * cbq_linear_xform_f32 (mode 0: x0 itself).
 * cbq_split_linear_argmax_f32: one split-format matrix (Huffman), as
 * cbq_split_linear_f32 with n = 1. */
#define CBQ_ARGMAX_WORKSPACE 8192
int cbq_linear_xform_argmax_f32(const float *x0, const float *x1, float *h_out, int mode,
                                float eps, const uint8_t *packed, const float *codebook,
                                float *out, int M, int K, int C, int bits, void *workspace,
                                size_t workspace_bytes, int32_t *ids32, int64_t *toks,
                                int64_t *pos, int64_t first, int64_t n_toks, hipStream_t stream);
int cbq_split_linear_argmax_f32(const float *x0, const float *x1, float *h_out, int mode,
                                float eps, const cbq_split_matrix *m, float *out, int M, int K,
                                void *workspace, size_t workspace_bytes, int32_t *ids32,
                                int64_t *toks, int64_t *pos, int64_t first, int64_t n_toks,
                                hipStream_t stream);

/* ==== direct-to-device load ============================================== */

/* One byte range of a file and its device destination. */
typedef struct cbq_upload_part {
    int64_t file_offset;
    int64_t nbytes;
    void *dst;                   /* device memory, >= nbytes */
} cbq_upload_part;

/* Copy every part's bytes from the file at `path` to its device
 * destination and return when all copies have completed.  n_threads reader
 * threads (1..64) pread pieces of chunk_bytes (4 KiB .. 1 GiB) into two
 * pinned host buffers each and hand each piece to the device with
 * hipMemcpyAsync on the thread's own stream, so reads and copies overlap.
 * The staging buffers and streams live for the call only; no device memory
 * is allocated.  Destinations must not be in use by pending device work.
 * CK_ERR_ARG for bad arguments, a file that cannot be opened or a range
 * past its end (message on stderr), CK_ERR_HIP for runtime errors.
 * No counterpart in the reference: it replaces the gzip .npz thread-pool
 * preload (src/compressor.py:347-361) and the .idx mmap
 * (src/compressed_matmul_cpu.py:23-63) on the way to the device. */
int cbq_file_upload(const char *path, const cbq_upload_part *parts, int n_parts,
                    size_t chunk_bytes, int n_threads);

#ifdef __cplusplus
}
#endif
