// Host side of the canonical-Huffman format (no device code): canonical code
// assignment, the device decode tables (cbq_huff_build_luts,
// cbq_huff_build_ulut) and the stream indexer (cbq_huff_index_stream) that
// turns a reference-format MSB-first stream into the chunk offsets and
// sub-block lengths the GPU decoder starts from.  Every input may come from a
// file: lengths, stream bytes and row starts are validated and never
// dereferenced out of range.  Plain C++ (compiled by the host compiler into
// libcbq_hip.so, and with address / undefined-behaviour sanitizers by the
// CPU test build).
#include "../../include/cbq_hip.h"
#include "cbq_huff_format.h"

#include <stdint.h>

#include <algorithm>
#include <thread>
#include <vector>

namespace {

using namespace cbq_huff;

// ---------------------------------------------------------------------------
// Host: canonical codes and tables
// ---------------------------------------------------------------------------

uint32_t bitrev(uint32_t v, int n)
{
    uint32_t r = 0;
    for (int i = 0; i < n; i++) r |= ((v >> i) & 1u) << (n - 1 - i);
    return r;
}

struct Canon {
    int max_len = 0;
    int64_t first[kMaxLen + 2];
    int32_t count[kMaxLen + 2];
    int32_t base[kMaxLen + 2];
    std::vector<uint32_t> code;     // per symbol
    std::vector<int32_t> order;     // symbols in canonical order
};

// RFC 1951 section 3.2.2 code assignment; false when the lengths over-fill
// the code space (Kraft sum > 1) or exceed 32.
bool make_canon(const uint8_t *lengths, int n, Canon &cn)
{
    for (int L = 0; L <= kMaxLen + 1; L++) { cn.first[L] = -1; cn.count[L] = 0; cn.base[L] = 0; }
    uint64_t kraft = 0;
    for (int s = 0; s < n; s++) {
        int L = lengths[s];
        if (L > kMaxLen) return false;
        if (L) { cn.count[L]++; kraft += 1ull << (kMaxLen - L); cn.max_len = std::max(cn.max_len, L); }
    }
    if (kraft > (1ull << kMaxLen)) return false;
    int64_t next[kMaxLen + 2];
    int64_t code = 0;
    next[0] = 0;
    for (int L = 1; L <= kMaxLen; L++) {
        code = (code + (L > 1 ? cn.count[L - 1] : 0)) << 1;
        next[L] = code;
        if (cn.count[L]) cn.first[L] = code;
    }
    int acc = 0;
    for (int L = 1; L <= kMaxLen; L++) { cn.base[L] = acc; acc += cn.count[L]; }
    cn.base[kMaxLen + 1] = acc;
    cn.code.assign(n, 0);
    cn.order.assign(acc, 0);
    int fill[kMaxLen + 2];
    for (int L = 0; L <= kMaxLen + 1; L++) fill[L] = cn.base[L];
    for (int s = 0; s < n; s++) {
        int L = lengths[s];
        if (!L) continue;
        cn.code[s] = (uint32_t)next[L]++;
        cn.order[fill[L]++] = s;
    }
    return true;
}

inline uint32_t leaf(int len, uint32_t payload) { return (uint32_t)len | (payload << 16); }

// ---------------------------------------------------------------------------
// Host: decoder used by the indexer (MSB-first, reference semantics)
// ---------------------------------------------------------------------------

struct HostDecoder {
    Canon cn;
    uint8_t lut_len[kLutSize];      // 0: no code of <= 12 bits has this prefix

    bool init(const uint8_t *lengths, int n)
    {
        if (!make_canon(lengths, n, cn)) return false;
        std::fill(lut_len, lut_len + kLutSize, 0);
        for (int s = 0; s < n; s++) {
            int L = lengths[s];
            if (!L || L > kLutBits) continue;
            uint32_t lo = cn.code[s] << (kLutBits - L), cnt = 1u << (kLutBits - L);
            for (uint32_t i = 0; i < cnt; i++) lut_len[lo + i] = (uint8_t)L;
        }
        return true;
    }

    // 32 stream bits at `pos`, first one in the MSB (stream has >= 4 pad bytes
    // beyond the last code byte; reads at most 5 bytes).
    static uint32_t peek32(const uint8_t *s, int64_t nbytes, int64_t pos)
    {
        int64_t b = pos >> 3;
        uint64_t w = 0;
        for (int i = 0; i < 5; i++) w = (w << 8) | (b + i >= 0 && b + i < nbytes ? s[b + i] : 0);
        return (uint32_t)(w >> (8 - (pos & 7)));
    }

    int length_at(const uint8_t *s, int64_t nbytes, int64_t pos) const
    {
        uint32_t w = peek32(s, nbytes, pos);
        int L = lut_len[w >> (32 - kLutBits)];
        if (L) return L;
        for (L = kLutBits + 1; L <= cn.max_len; L++) {
            if (!cn.count[L]) continue;
            int64_t d = (int64_t)(w >> (32 - L)) - cn.first[L];
            if (d >= 0 && d < cn.count[L]) return L;
        }
        return 1;   // corrupt prefix: symbol 0, one bit
    }
};

}  // namespace

extern "C" {

int cbq_huff_build_luts(const uint8_t *lengths, int n_alpha, const float *codebook, int C,
                        int payload_is_value, int clamp_to, uint32_t *lut1, uint32_t *lut2,
                        int *n_lut2, int32_t *canon, int32_t *canon_pay)
{
    if (!lengths || n_alpha <= 0 || n_alpha > 65536 || !n_lut2) return CK_ERR_ARG;
    if (payload_is_value && (!codebook || C <= 0)) return CK_ERR_ARG;
    if (clamp_to && C <= 0) return CK_ERR_ARG;
    Canon cn;
    if (!make_canon(lengths, n_alpha, cn)) return CK_ERR_ARG;

    auto payload = [&](int sym) -> uint32_t {
        int s = sym;
        if (payload_is_value || clamp_to) s = std::min(s, C - 1);
        if (payload_is_value) {
            uint32_t u;
            __builtin_memcpy(&u, &codebook[s], 4);
            return u >> 16;
        }
        return (uint32_t)s;
    };
    const uint32_t invalid = leaf(1, payload(0));

    // Long-code prefixes: key = reversed first 12 code bits; subtable width.
    std::vector<int> maxlen(kLutSize, 0);
    for (int s = 0; s < n_alpha; s++) {
        int L = lengths[s];
        if (L <= kLutBits) continue;
        uint32_t key = bitrev(cn.code[s] >> (L - kLutBits), kLutBits);
        maxlen[key] = std::max(maxlen[key], L);
    }
    std::vector<uint32_t> base(kLutSize, 0), nbits(kLutSize, 0);
    int64_t total = 0;
    for (int k = 0; k < kLutSize; k++) {
        if (!maxlen[k]) continue;
        nbits[k] = (uint32_t)std::min(maxlen[k] - kLutBits, kLutBits);
        base[k] = (uint32_t)total;
        total += 1ll << nbits[k];
    }
    if (total == 0) total = 1;     // keep one (unused) entry so the array is never empty
    if (total >= (1 << 21)) return CK_ERR_ARG;
    *n_lut2 = (int)total;
    if (canon) {
        for (int L = 0; L <= kMaxLen; L++) {
            canon[L] = (int32_t)cn.first[L];
            canon[(kMaxLen + 1) + L] = cn.count[L];
            canon[2 * (kMaxLen + 1) + L] = cn.base[L];
        }
        canon[3 * (kMaxLen + 1)] = (int32_t)payload(0);
    }
    if (canon_pay)
        for (size_t i = 0; i < cn.order.size(); i++) canon_pay[i] = (int32_t)payload(cn.order[i]);
    if (!lut1 || !lut2) return CK_SUCCESS;

    for (int k = 0; k < kLutSize; k++) lut1[k] = invalid;
    for (int64_t i = 0; i < total; i++) lut2[i] = invalid;
    for (int k = 0; k < kLutSize; k++) {
        if (!maxlen[k]) continue;
        lut1[k] = (nbits[k] << 6) | (base[k] << 11);
        if (maxlen[k] > 2 * kLutBits)   // codes beyond 24 bits: unresolved -> canon stage
            for (uint32_t i = 0; i < (1u << nbits[k]); i++) lut2[base[k] + i] = 0u;
    }
    for (int s = 0; s < n_alpha; s++) {
        const int L = lengths[s];
        if (!L) continue;
        const uint32_t e = leaf(L, payload(s));
        if (L <= kLutBits) {
            const uint32_t r = bitrev(cn.code[s], L);
            for (uint32_t hi = 0; hi < (1u << (kLutBits - L)); hi++) lut1[r | (hi << L)] = e;
        } else {
            const uint32_t key = bitrev(cn.code[s] >> (L - kLutBits), kLutBits);
            const int rest = L - kLutBits;
            if (rest > (int)nbits[key]) continue;     // resolved by the canon stage
            const uint32_t suf = bitrev(cn.code[s] & ((1u << rest) - 1u), rest);
            for (uint32_t hi = 0; hi < (1u << (nbits[key] - rest)); hi++)
                lut2[base[key] + (suf | (hi << rest))] = e;
        }
    }
    return CK_SUCCESS;
}

int cbq_huff_build_ulut(const uint8_t *lengths, int n_alpha, const float *codebook, int C,
                        uint32_t *ulut1, uint32_t *ulut2, int *n_ulut2)
{
    if (!lengths || n_alpha <= 0 || n_alpha > 65536 || !codebook || C <= 0 || !n_ulut2)
        return CK_ERR_ARG;
    Canon cn;
    if (!make_canon(lengths, n_alpha, cn) || cn.max_len > 2 * kLutBits) return CK_ERR_ARG;
    auto payload = [&](int sym) -> uint32_t {
        uint32_t u;
        __builtin_memcpy(&u, &codebook[std::min(sym, C - 1)], 4);
        return u >> 16;
    };
    // entry 0: the "no code" leaf (symbol 0, one bit); then one leaf per short
    // code; then the per-prefix subtables of the long codes
    std::vector<int> maxlen(kLutSize, 0);
    int n_short = 0;
    for (int sy = 0; sy < n_alpha; sy++) {
        const int L = lengths[sy];
        if (!L) continue;
        if (L <= kLutBits) { n_short++; continue; }
        const uint32_t key = bitrev(cn.code[sy] >> (L - kLutBits), kLutBits);
        maxlen[key] = std::max(maxlen[key], L);
    }
    std::vector<uint32_t> base(kLutSize, 0), nbits(kLutSize, 0);
    int64_t total = 1 + n_short;
    for (int k = 0; k < kLutSize; k++) {
        if (!maxlen[k]) continue;
        nbits[k] = (uint32_t)(maxlen[k] - kLutBits);
        base[k] = (uint32_t)total;
        total += 1ll << nbits[k];
    }
    if (total >= (1 << 14)) return CK_ERR_ARG;           // base * 4 must fit 16 bits
    *n_ulut2 = (int)total;
    if (!ulut1 || !ulut2) return CK_SUCCESS;
    const uint32_t invalid = leaf(1, payload(0));
    for (int64_t i = 0; i < total; i++) ulut2[i] = invalid;
    for (int k = 0; k < kLutSize; k++) ulut1[k] = maxlen[k] ? (base[k] << 18) | nbits[k] : 0u;
    int next = 1;
    for (int sy = 0; sy < n_alpha; sy++) {
        const int L = lengths[sy];
        if (!L) continue;
        const uint32_t e = leaf(L, payload(sy));
        if (L <= kLutBits) {
            ulut2[next] = e;
            const uint32_t r = bitrev(cn.code[sy], L);
            for (uint32_t hi = 0; hi < (1u << (kLutBits - L)); hi++)
                ulut1[r | (hi << L)] = (uint32_t)next << 18;
            next++;
        } else {
            const uint32_t key = bitrev(cn.code[sy] >> (L - kLutBits), kLutBits);
            const int rest = L - kLutBits;
            const uint32_t suf = bitrev(cn.code[sy] & ((1u << rest) - 1u), rest);
            for (uint32_t hi = 0; hi < (1u << (nbits[key] - rest)); hi++)
                ulut2[base[key] + (suf | (hi << rest))] = e;
        }
    }
    return CK_SUCCESS;
}

int cbq_huff_index_stream(const uint8_t *stream_msb, int64_t stream_bytes,
                          const uint8_t *lengths, int n_alpha, const int64_t *row_bit_starts,
                          int M, int K, uint64_t *chunk_off, uint16_t *sub_len, int threads)
{
    if (!stream_msb || stream_bytes <= 0 || !lengths || n_alpha <= 0 || M <= 0 || K <= 0 ||
        !chunk_off || !sub_len)
        return CK_ERR_ARG;
    HostDecoder dec;
    if (!dec.init(lengths, n_alpha)) return CK_ERR_ARG;
    const int64_t N = (int64_t)M * K;
    const int64_t n_sub = (N + kSub - 1) / kSub;
    const int64_t n_chunks = (N + kChunk - 1) / kChunk;
    std::vector<int64_t> sub_start(n_sub + 1, -1);
    const int64_t total_bits = stream_bytes * 8;
    if (!row_bit_starts) threads = 1;
    threads = std::max(1, std::min(threads, M));
    std::vector<int> ok(threads, 1);
    std::vector<int64_t> end_pos(threads, 0);

    auto work = [&](int ti) {
        const int ra = (int)((int64_t)M * ti / threads), rb = (int)((int64_t)M * (ti + 1) / threads);
        int64_t pos = ti == 0 ? 0 : row_bit_starts[ra];
        // row starts come from the file: out-of-range ones fail here
        if (pos < 0 || pos > total_bits || (row_bit_starts && row_bit_starts[ra] != pos)) {
            ok[ti] = 0;
            return;
        }
        int64_t sym = (int64_t)ra * K, sym_end = (int64_t)rb * K;
        // own the sub-blocks whose first symbol lies in [ra*K, rb*K)
        while (sym < sym_end || (sym % kSub) != 0) {
            if (sym >= N) break;
            if (sym % kSub == 0) sub_start[sym / kSub] = pos;
            if (row_bit_starts && sym % K == 0 && sym < sym_end && row_bit_starts[sym / K] != pos) {
                ok[ti] = 0;
                return;
            }
            if (pos >= total_bits) { ok[ti] = 0; return; }
            pos += dec.length_at(stream_msb, stream_bytes, pos);
            sym++;
        }
        end_pos[ti] = pos;
    };
    if (threads == 1) {
        work(0);
    } else {
        std::vector<std::thread> pool;
        for (int ti = 0; ti < threads; ti++) pool.emplace_back(work, ti);
        for (auto &th : pool) th.join();
    }
    for (int ti = 0; ti < threads; ti++)
        if (!ok[ti]) return CK_ERR_ARG;
    int64_t last_end = 0;
    // the thread that decoded symbol N-1 reports the stream end
    for (int ti = 0; ti < threads; ti++) last_end = std::max(last_end, end_pos[ti]);
    sub_start[n_sub] = last_end;
    for (int64_t s = 0; s < n_sub; s++) {
        const int64_t len = sub_start[s + 1] - sub_start[s];
        if (sub_start[s] < 0 || len < 0 || len > 65535) return CK_ERR_ARG;
        sub_len[s] = (uint16_t)len;
    }
    for (int64_t c = 0; c < n_chunks; c++) chunk_off[c] = (uint64_t)sub_start[c * (kChunk / kSub)];
    chunk_off[n_chunks] = (uint64_t)last_end;
    return CK_SUCCESS;
}

}  // extern "C"
