// Host code of the library and the CPU oracle under AddressSanitizer and
// UndefinedBehaviorSanitizer (built by `make -C tests/native sanitize`, run
// by tests/test_sanitize_host.py on the CPU).  Test infrastructure.
//
// Library host code that takes file-borne input (csrc/cbq_huff_host.cpp,
// csrc/cbq_io.cpp):
//   - cbq_huff_index_stream on streams this program encodes (canonical codes
//     from random complete and incomplete length sets, up to 32-bit codes):
//     chunk offsets and sub-block lengths must equal the encoder's own bit
//     positions; then the same call on tampered input -- bit flips,
//     truncated byte counts, negative / out-of-range / shuffled row starts,
//     over-full or over-long code lengths -- must return without touching
//     memory outside its arguments (CK_SUCCESS or CK_ERR_ARG);
//   - cbq_huff_build_luts / cbq_huff_build_ulut over valid and random length
//     sets, tables sized exactly as the size query reports;
//   - cbq_file_upload's argument and file checks (missing file, ranges past
//     the end, negative offsets, bad chunk and thread counts), which return
//     before any HIP call.
// Oracle (oracle/cbq_oracle.c), on inputs of exactly the size the reference
// format guarantees (packed stream + 4 pad bytes; Huffman stream + 4 pad
// bytes): fixed-width unpack / GEMV / embedding at widths 1..16, and the
// Huffman decode and GEMV against the encoder's symbols.
//
// Exit status 0 when every case passes; the sanitizers abort on the first
// error they find.
#include "../../include/cbq_hip.h"

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <vector>

extern "C" {
void oracle_unpack_indices(const uint8_t *packed, int64_t n, int bits, int32_t *out);
void oracle_fixed_gemv_serial(const float *x, const uint8_t *packed, const float *cb, float *out,
                              int T, int M, int K, int C, int bits);
void oracle_fixed_embedding(const int32_t *ids, const uint8_t *packed, const float *cb,
                            float *out, int T, int H, int C, int bits);
void oracle_huff_decode_indices(const uint8_t *stream, const uint16_t *lut_sym,
                                const uint8_t *lut_len, const int64_t *sl_first,
                                const int32_t *sl_base, const uint16_t *sl_sym,
                                const int64_t *row_bit_starts, int32_t *out, int M, int K,
                                int max_len);
void oracle_huff_gemv_rows(const float *x, const uint8_t *stream, const uint16_t *lut_sym,
                           const uint8_t *lut_len, const int64_t *sl_first, const int32_t *sl_base,
                           const uint16_t *sl_sym, const int64_t *row_bit_starts, const float *cb,
                           float *out, int T, int M, int K, int C, int r_start, int r_end,
                           int max_len);
}

static int g_fail = 0;
static int g_cases = 0;

#define CHECK(cond, ...)                                                                       \
    do {                                                                                       \
        if (!(cond)) {                                                                         \
            printf("FAIL  " __VA_ARGS__);                                                      \
            printf("  (%s:%d)\n", __FILE__, __LINE__);                                         \
            g_fail++;                                                                          \
        }                                                                                      \
    } while (0)

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
    uint64_t next()
    {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    int below(int n) { return (int)(next() % (uint64_t)n); }
};

// ---- a canonical-Huffman encoder of its own (RFC 1951 section 3.2.2) -------

// Lengths of a complete prefix code with n symbols: split random leaves of a
// one-leaf tree until there are n, none deeper than max_len.  With
// `incomplete` one leaf is dropped again (Kraft sum < 1).
static std::vector<uint8_t> random_lengths(Rng &r, int n, int max_len, bool incomplete)
{
    std::vector<uint8_t> leaves(1, 0);
    while ((int)leaves.size() < n + (incomplete ? 1 : 0)) {
        int i = r.below((int)leaves.size());
        for (int tries = 0; leaves[i] >= max_len && tries < 64; tries++)
            i = r.below((int)leaves.size());
        if (leaves[i] >= max_len) break;
        const uint8_t d = (uint8_t)(leaves[i] + 1);
        leaves[i] = d;
        leaves.push_back(d);
    }
    if (incomplete && leaves.size() > 1) leaves.pop_back();
    if (leaves.size() == 1) leaves[0] = 1;                 // one symbol: one 1-bit code
    for (size_t i = leaves.size(); i > 1; i--) std::swap(leaves[i - 1], leaves[r.below((int)i)]);
    // a few symbols without a code (length 0), as unused codebook entries
    std::vector<uint8_t> out;
    for (uint8_t L : leaves) {
        if (r.below(16) == 0) out.push_back(0);
        out.push_back(L);
    }
    return out;
}

struct Code {
    std::vector<uint32_t> code;
    std::vector<int> len;
    int max_len = 0;
};

static Code canonical(const std::vector<uint8_t> &lengths)
{
    Code c;
    int count[40] = {0};
    for (uint8_t L : lengths) {
        if (L) count[L]++;
        c.max_len = std::max(c.max_len, (int)L);
    }
    uint64_t next[40] = {0}, code = 0;
    for (int L = 1; L < 40; L++) {
        code = (code + count[L - 1] * (L > 1)) << 1;
        next[L] = code;
    }
    c.code.resize(lengths.size());
    c.len.resize(lengths.size());
    for (size_t s = 0; s < lengths.size(); s++) {
        c.len[s] = lengths[s];
        if (lengths[s]) c.code[s] = (uint32_t)next[lengths[s]]++;
    }
    return c;
}

struct Encoded {
    std::vector<uint8_t> stream;        // MSB-first, + 4 zero pad bytes
    std::vector<int64_t> row_start;     // bit offset of each row
    std::vector<int64_t> sym_pos;       // bit offset of every symbol, + the end
    std::vector<int32_t> syms;
};

static Encoded encode(const Code &c, int M, int K, Rng &r)
{
    std::vector<int> used;
    for (size_t s = 0; s < c.len.size(); s++)
        if (c.len[s]) used.push_back((int)s);
    Encoded e;
    e.syms.resize((size_t)M * K);
    int64_t bit = 0;
    std::vector<uint8_t> bits;
    for (int64_t i = 0; i < (int64_t)M * K; i++) {
        if (i % K == 0) e.row_start.push_back(bit);
        const int s = used[r.below((int)used.size())];
        e.syms[i] = s;
        e.sym_pos.push_back(bit);
        for (int b = c.len[s] - 1; b >= 0; b--) bits.push_back((uint8_t)((c.code[s] >> b) & 1u));
        bit += c.len[s];
    }
    e.sym_pos.push_back(bit);
    e.stream.assign((bits.size() + 7) / 8 + 4, 0);
    for (size_t i = 0; i < bits.size(); i++)
        if (bits[i]) e.stream[i >> 3] |= (uint8_t)(0x80u >> (i & 7));
    return e;
}

// ---- the library's stream indexer ------------------------------------------

static void check_index(const std::vector<uint8_t> &lengths, const Encoded &e, int M, int K,
                        int threads)
{
    const int64_t N = (int64_t)M * K;
    std::vector<uint64_t> chunk((N + 4095) / 4096 + 1);
    std::vector<uint16_t> sub((N + 63) / 64);
    const int rc = cbq_huff_index_stream(e.stream.data(), (int64_t)e.stream.size(),
                                         lengths.data(), (int)lengths.size(),
                                         threads > 1 ? e.row_start.data() : nullptr, M, K,
                                         chunk.data(), sub.data(), threads);
    g_cases++;
    CHECK(rc == CK_SUCCESS, "index_stream M=%d K=%d threads=%d: rc %d\n", M, K, threads, rc);
    if (rc != CK_SUCCESS) return;
    bool ok = true;
    for (size_t c = 0; c + 1 < chunk.size(); c++)
        ok &= chunk[c] == (uint64_t)e.sym_pos[c * 4096];
    ok &= chunk.back() == (uint64_t)e.sym_pos[N];
    for (size_t s = 0; s < sub.size(); s++) {
        const int64_t end = e.sym_pos[std::min<int64_t>((int64_t)(s + 1) * 64, N)];
        ok &= sub[s] == (uint16_t)(end - e.sym_pos[s * 64]);
    }
    CHECK(ok, "index_stream M=%d K=%d threads=%d: offsets differ from the encoder's\n", M, K,
          threads);
}

// Tampered input: the call must return (SUCCESS or ARG), never fault.
static void tamper_index(const std::vector<uint8_t> &lengths, const Encoded &e, int M, int K,
                         Rng &r)
{
    const int64_t N = (int64_t)M * K;
    std::vector<uint64_t> chunk((N + 4095) / 4096 + 1);
    std::vector<uint16_t> sub((N + 63) / 64);
    for (int t = 0; t < 24; t++) {
        std::vector<uint8_t> s = e.stream;
        std::vector<int64_t> rows = e.row_start;
        std::vector<uint8_t> lens = lengths;
        int64_t nbytes = (int64_t)s.size();
        switch (t % 6) {
        case 0:                                             // flipped bits
            for (int k = 0; k < 1 + r.below(32); k++) s[r.below((int)s.size())] ^= (uint8_t)(1u << r.below(8));
            break;
        case 1:                                             // stream cut short
            nbytes = 1 + r.below((int)std::max<int64_t>(1, nbytes - 1));
            break;
        case 2:                                             // row starts out of range
            rows[r.below(M)] = (r.below(2) ? -1 : 1) * (int64_t)(r.next() >> (r.below(40) + 2));
            break;
        case 3:                                             // row starts shuffled
            for (size_t i = rows.size(); i > 1; i--) std::swap(rows[i - 1], rows[r.below((int)i)]);
            break;
        case 4:                                             // random code lengths
            for (auto &L : lens) L = (uint8_t)r.below(40);
            break;
        default:                                            // every byte random
            for (auto &b : s) b = (uint8_t)r.next();
            break;
        }
        std::vector<uint8_t> exact(s.begin(), s.begin() + nbytes);  // no slack past nbytes
        const int rc = cbq_huff_index_stream(exact.data(), nbytes, lens.data(), (int)lens.size(),
                                             rows.data(), M, K, chunk.data(), sub.data(),
                                             1 + r.below(4));
        g_cases++;
        CHECK(rc == CK_SUCCESS || rc == CK_ERR_ARG, "tampered index_stream: rc %d\n", rc);
    }
}

// ---- the library's table builders -----------------------------------------

static void check_tables(const std::vector<uint8_t> &lengths, Rng &r)
{
    const int n = (int)lengths.size();
    std::vector<float> cb(n);
    for (int i = 0; i < n; i++) {
        const uint32_t u = (uint32_t)(0x3c00u + (uint32_t)r.below(0x800)) << 16;
        memcpy(&cb[i], &u, 4);
    }
    for (int value = 0; value < 2; value++) {
        int n2 = 0;
        int rc = cbq_huff_build_luts(lengths.data(), n, value ? cb.data() : nullptr,
                                     value ? n : 0, value, 0, nullptr, nullptr, &n2, nullptr,
                                     nullptr);
        g_cases++;
        if (rc != CK_SUCCESS) {
            CHECK(rc == CK_ERR_ARG, "build_luts size query: rc %d\n", rc);
            continue;
        }
        int used = 0;
        for (uint8_t L : lengths) used += L != 0;
        std::vector<uint32_t> l1(4096), l2((size_t)n2);
        std::vector<int32_t> canon(3 * 33 + 1), pay(std::max(1, used));
        rc = cbq_huff_build_luts(lengths.data(), n, value ? cb.data() : nullptr, value ? n : 0,
                                 value, 0, l1.data(), l2.data(), &n2, canon.data(), pay.data());
        CHECK(rc == CK_SUCCESS, "build_luts: rc %d\n", rc);
    }
    int nu = 0;
    int rc = cbq_huff_build_ulut(lengths.data(), n, cb.data(), n, nullptr, nullptr, &nu);
    g_cases++;
    if (rc == CK_SUCCESS) {
        std::vector<uint32_t> u1(4096), u2((size_t)nu);
        rc = cbq_huff_build_ulut(lengths.data(), n, cb.data(), n, u1.data(), u2.data(), &nu);
        CHECK(rc == CK_SUCCESS, "build_ulut: rc %d\n", rc);
    } else {
        CHECK(rc == CK_ERR_ARG, "build_ulut size query: rc %d\n", rc);
    }
}

// ---- the oracle's reference-format tables ----------------------------------

struct RefTables {
    std::vector<uint16_t> lut_sym;
    std::vector<uint8_t> lut_len;
    std::vector<int64_t> first;   // [max_len + 2]
    std::vector<int32_t> base;    // [max_len + 2]
    std::vector<uint16_t> sym;    // canonical order
};

// 12-bit table for codes <= 12 bits; per-length first code, base index and
// symbols in canonical order for the longer ones (the reference's
// build_gpu_lut / _build_slow_path_tables, src/huffman_codebook.py:353-423).
static RefTables ref_tables(const std::vector<uint8_t> &lengths, const Code &c)
{
    RefTables t;
    t.lut_sym.assign(4096, 0);
    t.lut_len.assign(4096, 0);
    for (size_t s = 0; s < lengths.size(); s++) {
        const int L = lengths[s];
        if (!L || L > 12) continue;
        const uint32_t lo = c.code[s] << (12 - L);
        for (uint32_t i = 0; i < (1u << (12 - L)); i++) {
            t.lut_sym[lo + i] = (uint16_t)s;
            t.lut_len[lo + i] = (uint8_t)L;
        }
    }
    t.first.assign(c.max_len + 2, -1);
    t.base.assign(c.max_len + 2, 0);
    std::vector<int> count(c.max_len + 2, 0);
    for (uint8_t L : lengths)
        if (L) count[L]++;
    int acc = 0;
    for (int L = 1; L <= c.max_len + 1; L++) {
        t.base[L] = acc;
        if (L <= c.max_len) acc += count[L];
    }
    t.sym.assign(std::max(acc, 1), 0);
    std::vector<int> fill(t.base);
    for (int L = 1; L <= c.max_len; L++)
        for (size_t s = 0; s < lengths.size(); s++)
            if (lengths[s] == L) {
                if (t.first[L] < 0) t.first[L] = c.code[s];
                t.sym[fill[L]++] = (uint16_t)s;
            }
    return t;
}

static void check_oracle_huffman(const std::vector<uint8_t> &lengths, const Code &c,
                                 const Encoded &e, int M, int K)
{
    const RefTables t = ref_tables(lengths, c);
    std::vector<uint8_t> exact(e.stream);      // stream + the 4 pad bytes, nothing more
    std::vector<int32_t> dec((size_t)M * K);
    oracle_huff_decode_indices(exact.data(), t.lut_sym.data(), t.lut_len.data(), t.first.data(),
                               t.base.data(), t.sym.data(), e.row_start.data(), dec.data(), M, K,
                               c.max_len);
    g_cases++;
    CHECK(dec == e.syms, "oracle Huffman decode M=%d K=%d max_len=%d: symbols differ\n", M, K,
          c.max_len);
    const int C = (int)lengths.size();
    std::vector<float> cb(C), x(K), out(M, 0.f), ref(M, 0.f);
    for (int i = 0; i < C; i++) cb[i] = 0.001f * (float)((i * 37) % 101 - 50);
    for (int k = 0; k < K; k++) x[k] = 0.01f * (float)((k * 13) % 23 - 11);
    oracle_huff_gemv_rows(x.data(), exact.data(), t.lut_sym.data(), t.lut_len.data(),
                          t.first.data(), t.base.data(), t.sym.data(), e.row_start.data(),
                          cb.data(), out.data(), 1, M, K, C, 0, M, c.max_len);
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++) ref[m] += x[k] * cb[e.syms[(size_t)m * K + k]];
    g_cases++;
    CHECK(out == ref, "oracle Huffman GEMV M=%d K=%d: differs from the sequential sum\n", M, K);
}

static void check_oracle_fixed(Rng &r)
{
    for (int bits = 1; bits <= 16; bits++) {
        const int M = 1 + r.below(9), K = 1 + r.below(70), T = 1 + r.below(3);
        const int C = 1 + r.below(1 << bits);
        const int64_t n = (int64_t)M * K;
        std::vector<int32_t> idx(n), got(n);
        std::vector<uint8_t> packed((n * bits + 7) / 8 + 4, 0);   // the reference's 4 pad bytes
        for (int64_t i = 0; i < n; i++) {
            idx[i] = (int32_t)(r.next() & ((1u << bits) - 1u));
            for (int b = 0; b < bits; b++)
                if ((idx[i] >> b) & 1) packed[(i * bits + b) >> 3] |= (uint8_t)(1u << ((i * bits + b) & 7));
        }
        oracle_unpack_indices(packed.data(), n, bits, got.data());
        g_cases++;
        CHECK(got == idx, "oracle unpack bits=%d n=%lld\n", bits, (long long)n);
        std::vector<float> cb(C), x((size_t)T * K), out((size_t)T * M, 0.f), ref((size_t)T * M, 0.f);
        for (int i = 0; i < C; i++) cb[i] = (float)(i % 7) - 3.f;
        for (auto &v : x) v = (float)r.below(5) - 2.f;
        oracle_fixed_gemv_serial(x.data(), packed.data(), cb.data(), out.data(), T, M, K, C, bits);
        for (int t = 0; t < T; t++)
            for (int m = 0; m < M; m++)
                for (int k = 0; k < K; k++)
                    ref[(size_t)t * M + m] += x[(size_t)t * K + k] * cb[std::min(idx[(size_t)m * K + k], C - 1)];
        g_cases++;
        CHECK(out == ref, "oracle fixed GEMV bits=%d\n", bits);
        std::vector<int32_t> ids(T);
        for (auto &v : ids) v = r.below(M);
        std::vector<float> emb((size_t)T * K);
        oracle_fixed_embedding(ids.data(), packed.data(), cb.data(), emb.data(), T, K, C, bits);
        bool ok = true;
        for (int t = 0; t < T; t++)
            for (int k = 0; k < K; k++)
                ok &= emb[(size_t)t * K + k] == cb[std::min(idx[(size_t)ids[t] * K + k], C - 1)];
        g_cases++;
        CHECK(ok, "oracle fixed embedding bits=%d\n", bits);
    }
}

// ---- the library's file upload: checks before any HIP call ----------------

static void check_upload_args()
{
    char path[] = "/tmp/cbq_sanitize_XXXXXX";
    const int fd = mkstemp(path);
    CHECK(fd >= 0, "mkstemp\n");
    if (fd < 0) return;
    char buf[8192];
    memset(buf, 7, sizeof(buf));
    CHECK(write(fd, buf, sizeof(buf)) == (ssize_t)sizeof(buf), "write\n");
    close(fd);
    char dst[64];
    cbq_upload_part p = {0, 64, dst};
    struct Case {
        const char *path;
        cbq_upload_part part;
        int n;
        size_t chunk;
        int threads;
    } cases[] = {
        {"/nonexistent/cbq.img", p, 1, 1 << 20, 2},
        {path, {8192 - 32, 64, dst}, 1, 1 << 20, 2},     // range past the end of the file
        {path, {-1, 64, dst}, 1, 1 << 20, 2},            // negative offset
        {path, {0, -8, dst}, 1, 1 << 20, 2},             // negative size
        {path, {0, 64, nullptr}, 1, 1 << 20, 2},         // no destination
        {path, p, 1, 100, 2},                            // chunk below 4 KiB
        {path, p, 1, (size_t)1 << 40, 2},                // chunk above 1 GiB
        {path, p, 1, 1 << 20, 0},                        // no threads
        {path, p, 1, 1 << 20, 65},                       // too many threads
        {nullptr, p, 1, 1 << 20, 2},                     // no path
    };
    for (const Case &c : cases) {
        const int rc = cbq_file_upload(c.path, &c.part, c.n, c.chunk, c.threads);
        g_cases++;
        CHECK(rc == CK_ERR_ARG, "cbq_file_upload bad request: rc %d\n", rc);
    }
    g_cases++;
    CHECK(cbq_file_upload(path, &p, 0, 1 << 20, 2) == CK_SUCCESS, "cbq_file_upload no parts\n");
    unlink(path);
}

int main()
{
    Rng r(2024);
    check_oracle_fixed(r);
    check_upload_args();
    struct Shape {
        int n_alpha, max_len, M, K;
        bool incomplete;
    } shapes[] = {
        {1, 1, 3, 64, false},      {2, 2, 4, 100, false},     {300, 12, 6, 1000, false},
        {4556, 24, 8, 4096, false}, {4556, 24, 8, 4096, true}, {3000, 32, 5, 4160, false},
        {65, 30, 40, 130, true},   {12000, 28, 3, 8192, false},
    };
    for (const Shape &sh : shapes) {
        std::vector<uint8_t> lengths = random_lengths(r, sh.n_alpha, sh.max_len, sh.incomplete);
        const Code c = canonical(lengths);
        const Encoded e = encode(c, sh.M, sh.K, r);
        for (int threads : {1, 3, 8}) check_index(lengths, e, sh.M, sh.K, threads);
        tamper_index(lengths, e, sh.M, sh.K, r);
        check_tables(lengths, r);
        check_oracle_huffman(lengths, c, e, sh.M, sh.K);
    }
    // length sets no code has: over-full, longer than 32 bits, all zero
    for (int t = 0; t < 40; t++) {
        std::vector<uint8_t> lengths(1 + r.below(3000));
        for (auto &L : lengths) L = (uint8_t)r.below(t < 20 ? 12 : 48);
        check_tables(lengths, r);
    }
    printf("%d cases\n", g_cases);
    if (g_fail) {
        printf("%d case(s) failed\n", g_fail);
        return 1;
    }
    printf("all cases passed\n");
    return 0;
}
