// Native test of libcbq_hip.so's C ABI, in the manner of the reference's own
// rocm/test_kernel.cpp (built and run by rocm/Makefile:62): host arrays are
// packed here, uploaded with ck_upload_codebook / ck_upload_packed, run
// through ck_linear_f32 / ck_linear_bf16 / ck_embedding_f32 and compared with
// the CPU oracle (oracle/libcbq_oracle.so, the C restatement of
// src/compressed_matmul.c), plus the argument checks of each entry point.
// Test infrastructure: it links the oracle as the checker.
//
// Exit status 0 when every case passes; one line per case on stdout.
#include "../../include/cbq_hip.h"

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

extern "C" {
void oracle_fixed_gemv_serial(const float *x, const uint8_t *packed, const float *cb, float *out,
                              int T, int M, int K, int C, int bits);
void oracle_fixed_embedding(const int32_t *ids, const uint8_t *packed, const float *cb,
                            float *out, int T, int H, int C, int bits);
}

static int g_fail = 0;

#define REQUIRE(cond, ...)                                                                     \
    do {                                                                                       \
        if (!(cond)) {                                                                         \
            printf("FAIL  " __VA_ARGS__);                                                      \
            printf("  (%s:%d)\n", __FILE__, __LINE__);                                         \
            g_fail++;                                                                          \
            return;                                                                            \
        }                                                                                      \
    } while (0)

// splitmix64: a seeded stream shared by every case
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next()
    {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    float uniform() { return (float)((next() >> 40) * (1.0 / 16777216.0)); }   // [0, 1)
    float normal()
    {
        const float u1 = uniform() + 1e-7f, u2 = uniform();
        return sqrtf(-2.f * logf(u1)) * cosf(6.2831853f * u2);
    }
};

static uint16_t bf16_bits(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);             // round to nearest even
    return (uint16_t)(u >> 16);
}

static float bf16_value(uint16_t b)
{
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// LSB-first fixed-width stream of n indices (src/bitpack.py:32-95) with the
// reference's 4 pad bytes (rocm/test_kernel.cpp:91).
static std::vector<uint8_t> pack_lsb(const std::vector<uint32_t> &idx, int bits)
{
    const size_t n = idx.size();
    std::vector<uint8_t> out((n * bits + 7) / 8 + 4, 0);
    for (size_t i = 0; i < n; i++) {
        const uint64_t bit = (uint64_t)i * bits;
        for (int b = 0; b < bits; b++)
            if ((idx[i] >> b) & 1u) out[(bit + b) >> 3] |= (uint8_t)(1u << ((bit + b) & 7));
    }
    return out;
}

// Codebook of C (<= 5376) distinct bf16 values, random sign and mantissa,
// magnitudes in [2^-23, 2^-2), and M*K indices, a few of them >= C (the
// reference clamps those to C - 1).
struct Matrix {
    std::vector<float> cb;
    std::vector<uint32_t> idx;
    std::vector<uint8_t> packed;
};

static Matrix make_matrix(int M, int K, int C, int bits, uint64_t seed)
{
    Rng r(seed);
    Matrix m;
    std::vector<uint8_t> seen(65536, 0);
    while ((int)m.cb.size() < C) {
        const uint64_t z = r.next();
        const uint16_t b = (uint16_t)((z & 0x807fu) | ((0x68u + (uint32_t)((z >> 16) % 21u)) << 7));
        if (!seen[b]) {
            seen[b] = 1;
            m.cb.push_back(bf16_value(b));
        }
    }
    const uint32_t top = (1u << bits) - 1u;
    m.idx.resize((size_t)M * K);
    for (auto &v : m.idx) {
        const uint64_t z = r.next();
        v = (z & 1023u) == 7u ? top - (uint32_t)((z >> 10) % 3u) : (uint32_t)((z >> 12) % (uint64_t)C);
        if (v > top) v = top;
    }
    m.packed = pack_lsb(m.idx, bits);
    return m;
}

static double rel_l2(const float *a, const float *b, size_t n)
{
    double num = 0, den = 0;
    for (size_t i = 0; i < n; i++) {
        num += ((double)a[i] - b[i]) * ((double)a[i] - b[i]);
        den += (double)b[i] * b[i];
    }
    return den > 0 ? sqrt(num / den) : sqrt(num);
}

static bool hip_ok(hipError_t e, const char *what)
{
    if (e != hipSuccess) {
        printf("FAIL  %s: %s\n", what, hipGetErrorString(e));
        g_fail++;
        return false;
    }
    return true;
}

static void test_linear_f32(int T, int M, int K, int C, int bits, uint64_t seed)
{
    const Matrix m = make_matrix(M, K, C, bits, seed);
    Rng r(seed ^ 0x5bd1e995u);
    std::vector<float> x((size_t)T * K), ref((size_t)T * M, 0.f), got((size_t)T * M);
    for (auto &v : x) v = r.normal();
    oracle_fixed_gemv_serial(x.data(), m.packed.data(), m.cb.data(), ref.data(), T, M, K, C, bits);

    float *d_cb = ck_upload_codebook(m.cb.data(), C);
    uint8_t *d_pk = ck_upload_packed(m.packed.data(), m.packed.size());
    REQUIRE(d_cb && d_pk, "linear_f32: upload helpers returned NULL");
    float *d_x = nullptr, *d_out = nullptr;
    if (!hip_ok(hipMalloc(&d_x, x.size() * 4), "hipMalloc x") ||
        !hip_ok(hipMalloc(&d_out, got.size() * 4), "hipMalloc out"))
        return;
    hip_ok(hipMemcpy(d_x, x.data(), x.size() * 4, hipMemcpyHostToDevice), "copy x");
    const int rc = ck_linear_f32(d_x, d_pk, d_cb, d_out, T, M, K, C, bits, 0);
    hip_ok(hipDeviceSynchronize(), "sync");
    hip_ok(hipMemcpy(got.data(), d_out, got.size() * 4, hipMemcpyDeviceToHost), "copy out");
    (void)hipFree(d_x);
    (void)hipFree(d_out);
    (void)hipFree(d_cb);
    (void)hipFree(d_pk);
    const double e = rel_l2(got.data(), ref.data(), got.size());
    // fp32 accumulate: rel-L2 <= 1e-5; T >= 64 runs the fp32 MFMA path, same bar
    REQUIRE(rc == CK_SUCCESS && e <= 1e-5, "ck_linear_f32 T=%d M=%d K=%d C=%d bits=%d: rc %d rel-L2 %.3e",
            T, M, K, C, bits, rc, e);
    printf("PASS  ck_linear_f32 T=%d M=%d K=%d C=%d bits=%d rel-L2 %.2e\n", T, M, K, C, bits, e);
}

static void test_linear_bf16(int T, int M, int K, int C, int bits, uint64_t seed)
{
    const Matrix m = make_matrix(M, K, C, bits, seed);
    Rng r(seed ^ 0x27d4eb2fu);
    std::vector<uint16_t> xb((size_t)T * K), got((size_t)T * M);
    std::vector<float> xf((size_t)T * K), ref((size_t)T * M, 0.f);
    for (size_t i = 0; i < xb.size(); i++) {
        xb[i] = bf16_bits(r.normal());
        xf[i] = bf16_value(xb[i]);
    }
    oracle_fixed_gemv_serial(xf.data(), m.packed.data(), m.cb.data(), ref.data(), T, M, K, C,
                             bits);
    float *d_cb = ck_upload_codebook(m.cb.data(), C);
    uint8_t *d_pk = ck_upload_packed(m.packed.data(), m.packed.size());
    REQUIRE(d_cb && d_pk, "linear_bf16: upload helpers returned NULL");
    void *d_x = nullptr, *d_out = nullptr;
    if (!hip_ok(hipMalloc(&d_x, xb.size() * 2), "hipMalloc x") ||
        !hip_ok(hipMalloc(&d_out, got.size() * 2), "hipMalloc out"))
        return;
    hip_ok(hipMemcpy(d_x, xb.data(), xb.size() * 2, hipMemcpyHostToDevice), "copy x");
    const int rc = ck_linear_bf16(d_x, d_pk, d_cb, d_out, T, M, K, C, bits, 0);
    hip_ok(hipDeviceSynchronize(), "sync");
    hip_ok(hipMemcpy(got.data(), d_out, got.size() * 2, hipMemcpyDeviceToHost), "copy out");
    (void)hipFree(d_x);
    (void)hipFree(d_out);
    (void)hipFree(d_cb);
    (void)hipFree(d_pk);
    std::vector<float> gf(got.size());
    for (size_t i = 0; i < got.size(); i++) gf[i] = bf16_value(got[i]);
    const double e = rel_l2(gf.data(), ref.data(), gf.size());
    // bf16 output (and bf16 MFMA at T >= 64): rel-L2 <= 2e-3
    REQUIRE(rc == CK_SUCCESS && e <= 2e-3, "ck_linear_bf16 T=%d M=%d K=%d C=%d bits=%d: rc %d rel-L2 %.3e",
            T, M, K, C, bits, rc, e);
    printf("PASS  ck_linear_bf16 T=%d M=%d K=%d C=%d bits=%d rel-L2 %.2e\n", T, M, K, C, bits, e);
}

static void test_embedding(int T, int vocab, int H, int C, int bits, uint64_t seed)
{
    const Matrix m = make_matrix(vocab, H, C, bits, seed);
    Rng r(seed ^ 0x85ebca6bu);
    std::vector<int32_t> ids(T);
    for (auto &v : ids) v = (int32_t)(r.next() % (uint64_t)vocab);
    ids[0] = vocab - 1;                                // last row: the stream's tail
    std::vector<float> ref((size_t)T * H), got((size_t)T * H);
    oracle_fixed_embedding(ids.data(), m.packed.data(), m.cb.data(), ref.data(), T, H, C, bits);
    float *d_cb = ck_upload_codebook(m.cb.data(), C);
    uint8_t *d_pk = ck_upload_packed(m.packed.data(), m.packed.size());
    REQUIRE(d_cb && d_pk, "embedding: upload helpers returned NULL");
    int32_t *d_ids = nullptr;
    float *d_out = nullptr;
    if (!hip_ok(hipMalloc(&d_ids, ids.size() * 4), "hipMalloc ids") ||
        !hip_ok(hipMalloc(&d_out, got.size() * 4), "hipMalloc out"))
        return;
    hip_ok(hipMemcpy(d_ids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice), "copy ids");
    const int rc = ck_embedding_f32(d_ids, d_pk, d_cb, d_out, T, H, C, bits, 0);
    hip_ok(hipDeviceSynchronize(), "sync");
    hip_ok(hipMemcpy(got.data(), d_out, got.size() * 4, hipMemcpyDeviceToHost), "copy out");
    (void)hipFree(d_ids);
    (void)hipFree(d_out);
    (void)hipFree(d_cb);
    (void)hipFree(d_pk);
    REQUIRE(rc == CK_SUCCESS && memcmp(got.data(), ref.data(), got.size() * 4) == 0,
            "ck_embedding_f32 T=%d vocab=%d H=%d bits=%d: rc %d, rows differ", T, vocab, H, bits, rc);
    printf("PASS  ck_embedding_f32 T=%d vocab=%d H=%d C=%d bits=%d bit-exact\n", T, vocab, H, C,
           bits);
}

static void test_arguments()
{
    const float cb[4] = {0.f, 1.f, 2.f, 3.f};
    // the upload helpers refuse empty / NULL sources
    REQUIRE(ck_upload_packed(nullptr, 16) == nullptr, "ck_upload_packed(NULL) not NULL");
    REQUIRE(ck_upload_packed((const uint8_t *)cb, 0) == nullptr, "ck_upload_packed(n=0) not NULL");
    REQUIRE(ck_upload_codebook(cb, 0) == nullptr, "ck_upload_codebook(C=0) not NULL");
    float *d_cb = ck_upload_codebook(cb, 4);
    REQUIRE(d_cb != nullptr, "ck_upload_codebook(C=4) NULL");
    float back[4] = {0};
    hip_ok(hipMemcpy(back, d_cb, sizeof(back), hipMemcpyDeviceToHost), "copy back");
    REQUIRE(memcmp(back, cb, sizeof(cb)) == 0, "ck_upload_codebook bytes differ");
    uint8_t *d_pk = ck_upload_packed((const uint8_t *)cb, sizeof(cb));
    REQUIRE(d_pk != nullptr, "ck_upload_packed NULL");
    float *d_x = nullptr;
    hip_ok(hipMalloc(&d_x, 64 * sizeof(float)), "hipMalloc x");
    // invalid arguments return CK_ERR_ARG before any launch
    REQUIRE(ck_linear_f32(nullptr, d_pk, d_cb, d_x, 1, 1, 32, 4, 2, 0) == CK_ERR_ARG,
            "ck_linear_f32(x=NULL)");
    REQUIRE(ck_linear_f32(d_x, d_pk, d_cb, d_x, 1, 1, 32, 4, 17, 0) == CK_ERR_ARG,
            "ck_linear_f32(bits=17)");
    REQUIRE(ck_linear_f32(d_x, d_pk, d_cb, d_x, 0, 1, 32, 4, 2, 0) == CK_ERR_ARG,
            "ck_linear_f32(T=0)");
    REQUIRE(ck_linear_bf16(d_x, d_pk, nullptr, d_x, 1, 1, 32, 4, 2, 0) == CK_ERR_ARG,
            "ck_linear_bf16(codebook=NULL)");
    REQUIRE(ck_embedding_f32(nullptr, d_pk, d_cb, d_x, 1, 32, 4, 2, 0) == CK_ERR_ARG,
            "ck_embedding_f32(ids=NULL)");
    REQUIRE(ck_embedding_f32((const int32_t *)d_x, d_pk, d_cb, d_x, 1, 32, 0, 2, 0) == CK_ERR_ARG,
            "ck_embedding_f32(C=0)");
    REQUIRE(strcmp(ck_error_string(CK_ERR_ARG), "invalid argument") == 0, "ck_error_string");
    (void)hipFree(d_x);
    (void)hipFree(d_pk);
    (void)hipFree(d_cb);
    printf("PASS  argument checks and upload helpers\n");
}

int main()
{
    printf("%s\n", cbq_version());
    fflush(stdout);
    test_arguments();
    // config 1's shape: 2048 -> 6144 at 13 bits (4556-entry lossless codebook)
    test_linear_f32(1, 6144, 2048, 4556, 13, 1);
    test_linear_f32(4, 384, 1024, 1000, 10, 2);
    test_linear_f32(16, 200, 512, 255, 8, 3);
    test_linear_f32(3, 70, 100, 3000, 12, 4);          // K % 32 != 0: per-element path
    test_linear_f32(64, 256, 512, 4000, 12, 5);        // fp32 MFMA path
    test_linear_f32(2, 64, 256, 4556, 16, 6);          // 16-bit indices
    test_linear_bf16(1, 512, 2048, 4556, 13, 7);
    test_linear_bf16(5, 128, 512, 300, 9, 8);
    test_linear_bf16(64, 256, 1024, 4556, 13, 9);      // bf16 MFMA path
    test_embedding(5, 300, 256, 1000, 10, 10);
    test_embedding(4, 77, 100, 90, 7, 11);             // H % 32 != 0
    test_embedding(3, 64, 512, 4556, 13, 12);
    fflush(stdout);
    if (g_fail) {
        printf("%d case(s) failed\n", g_fail);
        return 1;
    }
    printf("all cases passed\n");
    return 0;
}
