"""Huffman decode / GEMV / embedding on the GPU vs the oracle.

Decoded indices must be bit-exact (the chunked decoder and the reference-
format row decoder); GEMV outputs within rel-L2 1e-5 of the oracle's
huffman_matmul; embedding rows bit-exact.
"""
import ctypes

import numpy as np
import pytest
import torch

import codebook_builder as cbb
import huffman_codebook as hc
from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _lin(enc, cb, M, K, **over):
    from gpu_huffman_functions import HuffmanCodebookLinear
    kw = {k: enc.get(k) for k in ("huff_row_bit_starts", "huff_lut_sym", "huff_lut_len",
                                  "huff_sl_first_code", "huff_sl_base_offset", "huff_sl_sym",
                                  "huff_chunk_offsets", "huff_sub_lens")}
    kw.update(over)
    return HuffmanCodebookLinear("t", enc["huff_stream"], enc["huff_lengths"],
                                 int(np.asarray(enc["huff_n"])[0]), torch.from_numpy(cb),
                                 (M, K), cbb.bits_for(len(cb)), **kw)


def test_golden_cases(cuda, golden):
    from gpu_huffman_functions import HuffmanCodebookEmbedding
    for name, c in golden["huffman"].items():
        M, K = int(c["M"]), int(c["K"])
        enc = {k: c[k] for k in c if k.startswith("huff_")}
        lin = _lin(enc, c["cb"], M, K)
        y = lin(torch.from_numpy(c["x"]).to(cuda)).cpu().numpy()
        print(name, rel_l2(y, c["y"]), flush=True)
        assert rel_l2(y, c["y"]) <= TOL, name
        dec = lin.decode_indices().cpu().numpy()
        assert np.array_equal(dec, c["dec"]), name
        emb = HuffmanCodebookEmbedding("e", enc["huff_stream"], enc["huff_lengths"],
                                       int(enc["huff_n"][0]), torch.from_numpy(c["cb"]), (M, K),
                                       13, huff_row_bit_starts=enc["huff_row_bit_starts"])
        e = emb(torch.from_numpy(c["ids"]).to(cuda)).cpu().numpy()
        assert np.array_equal(e, c["emb"]), name


@pytest.mark.parametrize("M,K", [(2048, 2048), (1024, 2048), (6144, 2048), (2048, 6144),
                                 (512, 12288), (256, 4096), (96, 1024), (40, 192)])
def test_config3_shapes(cuda, oracle, M, K):
    """Config 3: bf16 N(0, 0.02) weights, frequency-sorted codebook, 24-bit
    limited canonical Huffman with 4096-symbol chunks; T = 1."""
    w = cbb.bf16_round(np.random.default_rng(M + K).standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = _lin(enc, cb, M, K)
    dec = lin.decode_indices().cpu().numpy().reshape(-1)
    assert np.array_equal(dec, idx.astype(np.int32))
    x = np.random.default_rng(1).standard_normal((1, K)).astype(np.float32)
    y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
    ref = oracle.huff_gemv(x, enc, cb, M, K, chunk_rows=None)
    assert rel_l2(y, ref) <= TOL


@pytest.mark.parametrize("T", [2, 4, 9, 16, 33])
def test_multi_token(cuda, oracle, T):
    M, K = 300, 2048
    w = cbb.bf16_round(np.random.default_rng(T).standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    x = np.random.default_rng(2).standard_normal((T, K)).astype(np.float32)
    y = _lin(enc, cb, M, K)(torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert rel_l2(y, oracle.huff_gemv(x, enc, cb, M, K, chunk_rows=None)) <= TOL


def test_symbol_payload_fp32_codebook(cuda, oracle):
    """Codebook values that are not bf16 -> symbol payload + LDS codebook."""
    rng = np.random.default_rng(3)
    M, K, C = 128, 1024, 3000
    f = np.ones(C)
    f[:100] = rng.uniform(100, 9000, 100)
    idx = rng.choice(C, size=M * K, p=f / f.sum())
    cb = rng.standard_normal(C).astype(np.float32)         # not bf16-exact
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = _lin(enc, cb, M, K)
    assert not lin.dev.value_payload
    x = rng.standard_normal((2, K)).astype(np.float32)
    y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert rel_l2(y, oracle.huff_gemv(x, enc, cb, M, K)) <= TOL


def test_codebook_shorter_than_alphabet_clamps(cuda, oracle, golden):
    c = golden["huffman"]["clamp"]
    enc = {k: c[k] for k in c if k.startswith("huff_")}
    M, K = int(c["M"]), int(c["K"])
    assert int(c["idx"].max()) >= len(c["cb"])
    y = _lin(enc, c["cb"], M, K)(torch.from_numpy(c["x"]).to(cuda)).cpu().numpy()
    assert rel_l2(y, c["y"]) <= TOL


def test_global_window_fallback(cuda, oracle):
    """Chunks larger than the LDS staging slot decode from global memory."""
    M, K = 256, 4096
    w = cbb.bf16_round(np.random.default_rng(9).standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = _lin(enc, cb, M, K, layout="stream")
    x = torch.randn(1, K, device=cuda)
    y_staged = lin(x)
    lin.dev.desc.stage_words = 64              # smaller than every chunk
    y_global = lin(x)
    assert torch.equal(y_staged, y_global)
    ref = oracle.huff_gemv(x.cpu().numpy(), enc, cb, M, K, chunk_rows=None)
    assert rel_l2(y_global.cpu().numpy(), ref) <= TOL


def test_codes_longer_than_24_bits(cuda, oracle):
    """Reference-style unlimited lengths (here up to 30 bits) resolve through
    the canonical stage and still decode bit-exactly."""
    rng = np.random.default_rng(5)
    lengths = np.array(list(range(1, 31)) + [30], np.uint8)
    M, K = 64, 256
    idx = rng.integers(0, 31, size=M * K)
    enc = oracle.huffman_encode(idx, shape=(M, K), lengths=lengths)
    cb = (rng.standard_normal(31) * 0.02).astype(np.float32)
    lin = _lin(enc, cb, M, K)
    assert np.array_equal(lin.decode_indices().cpu().numpy().reshape(-1), idx)
    x = rng.standard_normal((1, K)).astype(np.float32)
    y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert rel_l2(y, oracle.huff_gemv(x, enc, cb, M, K)) <= TOL


def test_reference_format_entry_points(cuda, oracle, golden):
    """huff_decode_to_i32 / huff_i32_linear_f32 / huff_i32_embedding_f32 with
    the reference's own int32 tables (src/gpu_huffman_functions.py:534-632)."""
    import cbq_native as nat
    lib = nat.load()
    st = nat.stream_ptr(cuda)
    for name, c in golden["huffman"].items():
        M, K, C = int(c["M"]), int(c["K"]), int(c["C"])
        t = {k: torch.from_numpy(np.asarray(c[k]).astype(np.int32)).to(cuda)
             for k in ("huff_lut_sym", "huff_lut_len", "huff_sl_first_code",
                       "huff_sl_base_offset", "huff_sl_sym")}
        stream = torch.from_numpy(np.concatenate([c["huff_stream"], np.zeros(8, np.uint8)])).to(cuda)
        rbs = torch.from_numpy(c["huff_row_bit_starts"].astype(np.int64)).to(cuda)
        out = torch.empty(M * K, dtype=torch.int32, device=cuda)
        mx = int(c["huff_lengths"].max())
        rc = lib.huff_decode_to_i32(stream.data_ptr(), rbs.data_ptr(), t["huff_lut_sym"].data_ptr(),
                                    t["huff_lut_len"].data_ptr(), t["huff_sl_first_code"].data_ptr(),
                                    t["huff_sl_base_offset"].data_ptr(), t["huff_sl_sym"].data_ptr(),
                                    out.data_ptr(), M, K, mx, st)
        nat.check(rc, "huff_decode_to_i32")
        assert np.array_equal(out.cpu().numpy().reshape(M, K), c["dec"]), name
        x = torch.from_numpy(c["x"]).to(cuda)
        cb = torch.from_numpy(c["cb"]).to(cuda)
        y = torch.empty(x.shape[0], M, device=cuda)
        nat.check(lib.huff_i32_linear_f32(x.data_ptr(), out.data_ptr(), cb.data_ptr(), y.data_ptr(),
                                          x.shape[0], M, K, C, st), "huff_i32_linear_f32")
        assert rel_l2(y.cpu().numpy(), c["y"]) <= TOL, name
        ids = torch.from_numpy(c["ids"]).to(cuda)
        e = torch.empty(len(c["ids"]), K, device=cuda)
        nat.check(lib.huff_i32_embedding_f32(ids.data_ptr(), out.data_ptr(), cb.data_ptr(),
                                             e.data_ptr(), len(c["ids"]), K, C, st),
                  "huff_i32_embedding_f32")
        assert np.array_equal(e.cpu().numpy(), c["emb"]), name


def test_embedding_rows_config5_like(cuda, oracle):
    """Huffman embedding: only requested rows decoded; bit-exact gather."""
    from gpu_huffman_functions import HuffmanCodebookEmbedding
    vocab, H = 3000, 4096
    w = cbb.bf16_round(np.random.default_rng(12).standard_normal((vocab, H)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    enc = hc.huffman_encode_indices(idx, shape=(vocab, H))
    emb = HuffmanCodebookEmbedding("emb", enc["huff_stream"], enc["huff_lengths"],
                                   int(enc["huff_n"][0]), torch.from_numpy(cb), (vocab, H), 13,
                                   huff_chunk_offsets=enc["huff_chunk_offsets"],
                                   huff_sub_lens=enc["huff_sub_lens"])
    ids = np.array([0, 1, 2999, 1500, 1500, 77, 4095 % vocab], np.int32)
    out = emb(torch.from_numpy(ids).to(cuda)).cpu().numpy()
    assert np.array_equal(out, w[ids])
    # H not a multiple of 4096 and row starts mid-chunk
    vocab2, H2 = 700, 320
    w2 = cbb.bf16_round(np.random.default_rng(13).standard_normal((vocab2, H2)) * 0.02)
    cb2, idx2 = cbb.frequency_sorted_codebook(w2)
    enc2 = hc.huffman_encode_indices(idx2, shape=(vocab2, H2))
    emb2 = HuffmanCodebookEmbedding("emb2", enc2["huff_stream"], enc2["huff_lengths"],
                                    int(enc2["huff_n"][0]), torch.from_numpy(cb2), (vocab2, H2), 13)
    ids2 = np.arange(0, vocab2, 7, dtype=np.int32)
    assert np.array_equal(emb2(torch.from_numpy(ids2).to(cuda)).cpu().numpy(), w2[ids2])


@pytest.mark.parametrize("M,K,payload", [(300, 4096, "value"), (70, 12288, "value"),
                                         (130, 8192, "symbol")])
def test_k_tiled_path(cuda, oracle, M, K, payload):
    """K % 4096 == 0 and T == 1 run the k-tiled kernel: phases over 4096-wide
    x tiles, two chunks per lane.  Also run with a tiny staging cap, which
    sends every chunk down the global-window path of the same kernel."""
    rng = np.random.default_rng(M + K)
    if payload == "value":
        w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
        cb, idx = cbb.frequency_sorted_codebook(w)
    else:
        C = 2500
        f = np.ones(C)
        f[:50] = rng.uniform(100, 5000, 50)
        idx = rng.choice(C, size=M * K, p=f / f.sum())
        cb = rng.standard_normal(C).astype(np.float32)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    x = rng.standard_normal((1, K)).astype(np.float32)
    ref = oracle.huff_gemv(x, enc, cb, M, K, chunk_rows=None)
    auto = _lin(enc, cb, M, K)                 # split format for the value payloads
    assert (auto.split is not None) == (payload == "value")
    assert rel_l2(auto(torch.from_numpy(x).to(cuda)).cpu().numpy(), ref) <= TOL
    lin = _lin(enc, cb, M, K, layout="columns" if payload == "value" else "stream")
    assert lin.dev.value_payload == (payload == "value")
    y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert rel_l2(y, ref) <= TOL
    lin.cols = lin.split = None           # packed-stream kernel (value payloads use columns)
    y1 = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert rel_l2(y1, ref) <= TOL
    lin.dev.desc.stage_words = 8
    y2 = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert rel_l2(y2, ref) <= TOL


def test_k_tiled_long_codes(cuda, oracle):
    """Codes up to 30 bits through the k-tiled kernel's second table level and
    canonical stage."""
    rng = np.random.default_rng(11)
    lengths = np.array(list(range(1, 31)) + [30], np.uint8)
    M, K = 24, 4096
    p = 0.5 ** np.minimum(lengths, 12).astype(np.float64)
    idx = rng.choice(31, size=M * K, p=p / p.sum())
    enc = oracle.huffman_encode(idx, shape=(M, K), lengths=lengths)
    cb = (rng.standard_normal(31) * 0.02).astype(np.float32)
    lin = _lin(enc, cb, M, K)
    lin.cols = lin.split = None           # packed-stream kernel
    x = rng.standard_normal((1, K)).astype(np.float32)
    y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
    assert rel_l2(y, oracle.huff_gemv(x, enc, cb, M, K)) <= TOL
