// Torch operator binding of libcbq_hip.so: the compressed entry points
// registered with torch's dispatcher as torch.ops.cbq.*, so that module
// code calls them like any ATen op (eagerly, under torch.cuda.graph capture,
// with torch's caching allocator for outputs and workspaces and its current
// HIP stream).  Host code only: every op checks its tensors, resolves the
// stream and calls the C ABI of include/cbq_hip.h, which launches the gfx950
// kernels.  It replaces the reference's load_inline extension
// (src/gpu_accelerated_functions.py:805-858) and its ctypes calls
// (src/gpu_accelerated_functions.py:415-543).
//
//   linear(x, packed, codebook, M, bits) -> out          ck_linear_f32 / ck_linear_bf16
//   embedding(ids, packed, codebook, vocab, bits, H) -> out     cbq_embedding_f32
//   split_linear(x, cwords, row_off, raw, lut, M) -> out         cbq_split_linear_f32
//   huff_linear(x, words, chunk_off, sub_len, lut1, lut2, canon, canon_pay,
//               value_cb, C, stage_words, M) -> out               cbq_huff_linear_f32
//   huff_embedding(ids, words, ..., vocab, H) -> out              cbq_huff_embedding_f32
//
// Outputs are new tensors on the inputs' device; fp32 unless x is bf16
// (linear only).  A HIP library error raises RuntimeError with the entry
// point's name and return code.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "../../include/cbq_hip.h"

namespace {

hipStream_t current_stream(const at::Tensor &t)
{
    return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_rc(int rc, const char *what)
{
    TORCH_CHECK(rc == CK_SUCCESS, what, " returned ", rc, " (", ck_error_string(rc), ")");
}

void check_dev(const at::Tensor &t, const at::Tensor &ref, const char *name)
{
    TORCH_CHECK(t.device() == ref.device(), name, " is on ", t.device(), ", expected ",
                ref.device());
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

template <typename P> const P *cptr(const at::Tensor &t) { return (const P *)t.data_ptr(); }

at::Tensor linear(const at::Tensor &x, const at::Tensor &packed, const at::Tensor &codebook,
                  int64_t M, int64_t bits)
{
    TORCH_CHECK(x.is_cuda(), "cbq::linear: x must be a device tensor");
    TORCH_CHECK(x.dim() == 2, "cbq::linear: x must be [T, K]");
    TORCH_CHECK(x.scalar_type() == at::kFloat || x.scalar_type() == at::kBFloat16,
                "cbq::linear: x must be float32 or bfloat16");
    TORCH_CHECK(packed.scalar_type() == at::kByte, "cbq::linear: packed must be uint8");
    TORCH_CHECK(codebook.scalar_type() == at::kFloat, "cbq::linear: codebook must be float32");
    check_dev(x, x, "x");
    check_dev(packed, x, "packed");
    check_dev(codebook, x, "codebook");
    const int64_t T = x.size(0), K = x.size(1), C = codebook.numel();
    TORCH_CHECK(M > 0 && M < (1ll << 31) && K < (1ll << 31) && T < (1ll << 31) && bits >= 1 &&
                    bits <= 16 && C > 0,
                "cbq::linear: bad sizes");
    TORCH_CHECK(packed.numel() >= (M * K * bits + 7) / 8 + 4,
                "cbq::linear: packed holds ", packed.numel(), " bytes, ",
                (M * K * bits + 7) / 8 + 4, " needed");
    c10::DeviceGuard guard(x.device());
    at::Tensor out = at::empty({T, M}, x.options());
    if (T == 0) return out;
    const hipStream_t st = current_stream(x);
    const bool bf16 = x.scalar_type() == at::kBFloat16;
    // batched tokens: MFMA path with its workspace from torch's allocator
    const size_t nws = T < 64 ? 0
                       : bf16 ? cbq_linear_bf16_workspace((int)T, (int)M, (int)K)
                              : cbq_linear_f32_workspace((int)T, (int)M, (int)K);
    at::Tensor ws;
    if (nws) ws = at::empty({(int64_t)((nws + 255) / 256 * 256)}, x.options().dtype(at::kByte));
    int rc;
    if (bf16)
        rc = cbq_linear_bf16_ws(x.data_ptr(), cptr<uint8_t>(packed), cptr<float>(codebook),
                                out.data_ptr(), (int)T, (int)M, (int)K, (int)C, (int)bits,
                                nws ? ws.data_ptr() : nullptr, nws, st);
    else
        rc = cbq_linear_f32_ws(cptr<float>(x), cptr<uint8_t>(packed), cptr<float>(codebook),
                               (float *)out.data_ptr(), (int)T, (int)M, (int)K, (int)C, (int)bits,
                               nws ? ws.data_ptr() : nullptr, nws, st);
    check_rc(rc, bf16 ? "cbq_linear_bf16_ws" : "cbq_linear_f32_ws");
    return out;
}

at::Tensor embedding(const at::Tensor &ids, const at::Tensor &packed, const at::Tensor &codebook,
                     int64_t vocab, int64_t bits, int64_t H)
{
    TORCH_CHECK(ids.is_cuda() && ids.scalar_type() == at::kInt && ids.dim() == 1,
                "cbq::embedding: ids must be a 1-D int32 device tensor");
    TORCH_CHECK(packed.scalar_type() == at::kByte && codebook.scalar_type() == at::kFloat,
                "cbq::embedding: packed uint8, codebook float32");
    check_dev(ids, ids, "ids");
    check_dev(packed, ids, "packed");
    check_dev(codebook, ids, "codebook");
    TORCH_CHECK(vocab > 0 && H > 0 && bits >= 1 && bits <= 16 && ids.numel() <= 65535,
                "cbq::embedding: bad sizes");
    TORCH_CHECK(packed.numel() >= (vocab * H * bits + 7) / 8 + 4, "cbq::embedding: packed short");
    c10::DeviceGuard guard(ids.device());
    const int64_t T = ids.numel();
    at::Tensor out = at::empty({T, H}, codebook.options());
    if (T == 0) return out;
    check_rc(cbq_embedding_f32(cptr<int32_t>(ids), cptr<uint8_t>(packed), cptr<float>(codebook),
                               (float *)out.data_ptr(), (int)T, (int)vocab, (int)H,
                               (int)codebook.numel(), (int)bits, current_stream(ids)),
             "cbq_embedding_f32");
    return out;
}

// T = 1: the one-token GEMV (cbq_split_linear_f32).  T >= 2: the fused
// few-token kernel (cbq_split_linear_fewtok_f32, 16 tokens a launch), which
// takes K % 1024 == 0 shapes whose row-group tile fits (it refuses the rest
// with an error here); x's bf16 parts go to a workspace from torch's
// allocator from 5 tokens on and for the shapes with two MFMA passes per
// phase (K % 4096 != 0 other than 1024 and 2048), as the Python wrapper
// split_fewtok does.
at::Tensor split_linear(const at::Tensor &x, const at::Tensor &cwords, const at::Tensor &row_off,
                        const at::Tensor &raw, const at::Tensor &lut, int64_t M)
{
    TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kFloat && x.dim() == 2 && x.size(0) >= 1 &&
                    x.is_contiguous(),
                "cbq::split_linear: x must be a contiguous [T, K] float32 device tensor");
    for (const auto &p : {std::make_pair(&cwords, "cwords"), std::make_pair(&row_off, "row_off"),
                          std::make_pair(&raw, "raw"), std::make_pair(&lut, "lut")})
        check_dev(*p.first, x, p.second);
    const int64_t K = x.size(1);
    TORCH_CHECK(M > 0 && (M * K) % 4096 == 0 && row_off.numel() == M * K / 4096 + 1 &&
                    raw.numel() == M * K && lut.numel() == 16384,
                "cbq::split_linear: tensors do not describe a ", M, "x", K, " split matrix");
    c10::DeviceGuard guard(x.device());
    const int64_t T = x.size(0);
    at::Tensor out = at::empty({T, M}, x.options());
    cbq_split_matrix m;
    m.cwords = cptr<uint32_t>(cwords);
    m.row_off = cptr<uint32_t>(row_off);
    m.raw = cptr<uint8_t>(raw);
    m.lut = cptr<uint32_t>(lut);
    m.n_chunks = M * K / 4096;
    const cbq_split_matrix *mats[1] = {&m};
    float *outs[1] = {(float *)out.data_ptr()};
    const int Ms[1] = {(int)M};
    if (T == 1) {
        check_rc(cbq_split_linear_f32(cptr<float>(x), nullptr, nullptr, 0, 0.f, 1, mats, outs,
                                      Ms, (int)K, current_stream(x)),
                 "cbq_split_linear_f32");
        return out;
    }
    TORCH_CHECK(T <= (int64_t)1 << 24, "cbq::split_linear: too many tokens");
    const bool two_pass = K % 4096 != 0 && K != 1024 && K != 2048;
    at::Tensor ws;
    size_t wsb = 0;
    if (T > 4 || two_pass) {
        wsb = cbq_split_fewtok_ws_bytes((int)K);
        ws = at::empty({(int64_t)wsb}, x.options().dtype(at::kByte));
    }
    const int rc = cbq_split_linear_fewtok_f32(cptr<float>(x), (int)T, 1, mats, outs, Ms, (int)K,
                                               wsb ? ws.data_ptr() : nullptr, wsb,
                                               current_stream(x));
    TORCH_CHECK(rc != CK_ERR_ARG, "cbq::split_linear: the few-token kernel does not take K = ", K,
                " (or x is not 16-byte aligned)");
    check_rc(rc, "cbq_split_linear_fewtok_f32");
    return out;
}

cbq_huff_stream stream_desc(const at::Tensor &ref, const at::Tensor &words,
                            const at::Tensor &chunk_off, const at::Tensor &sub_len,
                            const at::Tensor &lut1, const at::Tensor &lut2,
                            const at::Tensor &canon, const at::Tensor &canon_pay,
                            const c10::optional<at::Tensor> &value_cb, int64_t C,
                            int64_t stage_words)
{
    check_dev(words, ref, "words");
    check_dev(chunk_off, ref, "chunk_off");
    check_dev(sub_len, ref, "sub_len");
    check_dev(lut1, ref, "lut1");
    check_dev(lut2, ref, "lut2");
    check_dev(canon, ref, "canon");
    check_dev(canon_pay, ref, "canon_pay");
    TORCH_CHECK(lut1.numel() == 4096 && canon.numel() >= 100, "cbq: bad Huffman tables");
    cbq_huff_stream hs;
    hs.words = cptr<uint32_t>(words);
    hs.n_words = words.numel();
    hs.chunk_off = cptr<uint64_t>(chunk_off);
    hs.sub_len = cptr<uint16_t>(sub_len);
    hs.lut1 = cptr<uint32_t>(lut1);
    hs.lut2 = cptr<uint32_t>(lut2);
    hs.n_lut2 = (int32_t)lut2.numel();
    hs.canon = cptr<int32_t>(canon);
    hs.canon_pay = cptr<int32_t>(canon_pay);
    hs.value_cb = nullptr;
    if (value_cb.has_value() && value_cb->defined()) {
        check_dev(*value_cb, ref, "value_cb");
        hs.value_cb = cptr<float>(*value_cb);
    }
    hs.C = (int32_t)C;
    hs.stage_words = (int32_t)stage_words;
    return hs;
}

at::Tensor huff_linear(const at::Tensor &x, const at::Tensor &words, const at::Tensor &chunk_off,
                       const at::Tensor &sub_len, const at::Tensor &lut1, const at::Tensor &lut2,
                       const at::Tensor &canon, const at::Tensor &canon_pay,
                       const c10::optional<at::Tensor> &value_cb, int64_t C, int64_t stage_words,
                       int64_t M)
{
    TORCH_CHECK(x.is_cuda() && x.scalar_type() == at::kFloat && x.dim() == 2,
                "cbq::huff_linear: x must be a [T, K] float32 device tensor");
    check_dev(x, x, "x");
    const int64_t T = x.size(0), K = x.size(1);
    TORCH_CHECK(M > 0 && chunk_off.numel() == (M * K + 4095) / 4096 + 1 &&
                    sub_len.numel() == (M * K + 63) / 64,
                "cbq::huff_linear: the chunk index does not describe ", M, "x", K, " symbols");
    const cbq_huff_stream hs = stream_desc(x, words, chunk_off, sub_len, lut1, lut2, canon,
                                           canon_pay, value_cb, C, stage_words);
    c10::DeviceGuard guard(x.device());
    at::Tensor out = at::empty({T, M}, x.options());
    const hipStream_t st = current_stream(x);
    for (int64_t t0 = 0; t0 < T; t0 += 16) {                 // 16-token tiles
        const int64_t tt = std::min<int64_t>(16, T - t0);
        check_rc(cbq_huff_linear_f32(cptr<float>(x) + t0 * K, &hs,
                                     (float *)out.data_ptr() + t0 * M, (int)tt, (int)M, (int)K,
                                     st),
                 "cbq_huff_linear_f32");
    }
    return out;
}

at::Tensor huff_embedding(const at::Tensor &ids, const at::Tensor &words,
                          const at::Tensor &chunk_off, const at::Tensor &sub_len,
                          const at::Tensor &lut1, const at::Tensor &lut2, const at::Tensor &canon,
                          const at::Tensor &canon_pay, const c10::optional<at::Tensor> &value_cb,
                          int64_t C, int64_t stage_words, int64_t vocab, int64_t H)
{
    TORCH_CHECK(ids.is_cuda() && ids.scalar_type() == at::kInt && ids.dim() == 1,
                "cbq::huff_embedding: ids must be a 1-D int32 device tensor");
    check_dev(ids, ids, "ids");
    TORCH_CHECK(vocab > 0 && H > 0 && chunk_off.numel() == (vocab * H + 4095) / 4096 + 1,
                "cbq::huff_embedding: the chunk index does not describe ", vocab, "x", H);
    const cbq_huff_stream hs = stream_desc(ids, words, chunk_off, sub_len, lut1, lut2, canon,
                                           canon_pay, value_cb, C, stage_words);
    c10::DeviceGuard guard(ids.device());
    const int64_t T = ids.numel();
    at::Tensor out = at::empty({T, H}, ids.options().dtype(at::kFloat));
    if (T == 0) return out;
    check_rc(cbq_huff_embedding_f32(cptr<int32_t>(ids), &hs, (float *)out.data_ptr(), (int)T,
                                    (int)vocab, (int)H, current_stream(ids)),
             "cbq_huff_embedding_f32");
    return out;
}

// Shape functions for tracing (meta tensors): same output shapes and dtypes.
at::Tensor linear_meta(const at::Tensor &x, const at::Tensor &, const at::Tensor &, int64_t M,
                       int64_t)
{
    return at::empty({x.size(0), M}, x.options());
}

at::Tensor embedding_meta(const at::Tensor &ids, const at::Tensor &, const at::Tensor &codebook,
                          int64_t, int64_t, int64_t H)
{
    return at::empty({ids.size(0), H}, ids.options().dtype(codebook.scalar_type()));
}

}  // namespace

TORCH_LIBRARY(cbq, m)
{
    m.def("linear(Tensor x, Tensor packed, Tensor codebook, int M, int bits) -> Tensor");
    m.def("embedding(Tensor ids, Tensor packed, Tensor codebook, int vocab, int bits, int H) "
          "-> Tensor");
    m.def("split_linear(Tensor x, Tensor cwords, Tensor row_off, Tensor raw, Tensor lut, "
          "int M) -> Tensor");
    m.def("huff_linear(Tensor x, Tensor words, Tensor chunk_off, Tensor sub_len, Tensor lut1, "
          "Tensor lut2, Tensor canon, Tensor canon_pay, Tensor? value_cb, int C, "
          "int stage_words, int M) -> Tensor");
    m.def("huff_embedding(Tensor ids, Tensor words, Tensor chunk_off, Tensor sub_len, "
          "Tensor lut1, Tensor lut2, Tensor canon, Tensor canon_pay, Tensor? value_cb, int C, "
          "int stage_words, int vocab, int H) -> Tensor");
}

// torch registers ROCm devices under its "CUDA" dispatch key
TORCH_LIBRARY_IMPL(cbq, CUDA, m)
{
    m.impl("linear", &linear);
    m.impl("embedding", &embedding);
    m.impl("split_linear", &split_linear);
    m.impl("huff_linear", &huff_linear);
    m.impl("huff_embedding", &huff_embedding);
}

TORCH_LIBRARY_IMPL(cbq, Meta, m)
{
    m.impl("linear", &linear_meta);
    m.impl("embedding", &embedding_meta);
}
