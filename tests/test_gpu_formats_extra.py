"""Format producers and decoders on the GPU against the reference's own
encoder and the oracle:

- synthetic.huffman_encode_torch (the GPU encoder of the bench and decoder
  models) writes the same stream bytes and chunk index as
  huffman_codebook.huffman_encode_indices for the same code lengths, and the
  oracle decodes its stream back to the input indices;
- a stream with prefixes that match no code (incomplete codes, random bits)
  decodes on the GPU exactly as the reference's guard does: symbol 0 and one
  bit (src/compressed_matmul.c:183-185);
- cbq_split_to_packed writes the LSB-first stream bit for bit at every
  transient width (8, 10 for 9, 11, 12, 13 bits)."""
import ctypes

import numpy as np
import pytest
import torch

import cbq_native as nat
import codebook_builder as cbb
import huffman_codebook as hc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K,seed", [(64, 4096, 1), (37, 1000, 2), (1, 4096 * 3 + 64, 3)])
def test_gpu_encoder_matches_reference_encoder(cuda, oracle, M, K, seed):
    import synthetic
    rng = np.random.default_rng(seed)
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    _, idx = cbb.frequency_sorted_codebook(w)
    idx = idx.reshape(-1).astype(np.int64)
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lengths = enc["huff_lengths"]
    words, chunk_off, sub_len, total = synthetic.huffman_encode_torch(
        torch.from_numpy(idx).to(cuda), lengths)
    nbytes = (total + 7) // 8
    dev_bytes = words.cpu().numpy().view(np.uint8)[:nbytes]
    stream = hc.REV8[dev_bytes]                        # LSB-first words -> MSB-first bytes
    assert np.array_equal(stream, enc["huff_stream"][:nbytes])
    assert np.array_equal(chunk_off.cpu().numpy().view(np.uint64), enc["huff_chunk_offsets"])
    assert np.array_equal(sub_len.cpu().numpy().view(np.uint16), enc["huff_sub_lens"])
    dec = oracle.huff_decode_indices(dict(enc, huff_stream=np.concatenate(
        [stream, np.zeros(4, np.uint8)])), M, K).reshape(-1)
    assert np.array_equal(dec, idx)


@pytest.mark.parametrize("lengths", [[1, 3, 3, 5], [1], [2, 2, 3],
                                     [3, 3, 3, 3, 5, 5, 9, 14, 20, 26]])
def test_corrupt_prefix_decode(cuda, oracle, lengths):
    """Incomplete codes (Kraft sum < 1) over random bits: every prefix that
    matches no code gives symbol 0 and advances one bit.  The stream is
    indexed by the host indexer with the same rule, so every chunk start
    lies inside the stream."""
    from gpu_huffman_functions import SymbolDecoder
    rng = np.random.default_rng(len(lengths))
    lengths = np.array(lengths, np.uint8)
    n = 4 * 4096 + 640
    stream = np.concatenate([rng.integers(0, 256, size=n * int(lengths.max()) // 8 + 8)
                             .astype(np.uint8), np.zeros(4, np.uint8)])
    enc = {"huff_lengths": lengths, "huff_stream": stream, "huff_n": np.array([n], np.int64),
           "huff_row_bit_starts": np.zeros(1, np.int64)}
    enc["huff_lut_sym"], enc["huff_lut_len"] = hc.build_gpu_lut(lengths)
    (enc["huff_sl_first_code"], enc["huff_sl_base_offset"],
     enc["huff_sl_sym"]) = hc.build_slow_tables(lengths)
    want = oracle.huff_decode_indices(enc, 1, n).reshape(-1)
    assert (want == 0).any() and n * int(lengths.max()) > 0
    ch, sub = hc.index_stream(stream, lengths, 1, n, None)
    assert int(ch[-1]) <= 8 * stream.size
    words = torch.from_numpy(hc.device_words_from_stream(stream).view(np.int32)).to(cuda)
    dec = SymbolDecoder(words, torch.from_numpy(ch.view(np.int64)).to(cuda),
                        torch.from_numpy(sub.view(np.int16)).to(cuda), lengths, cuda).indices(n)
    assert np.array_equal(dec.cpu().numpy().astype(np.int64), want)


@pytest.mark.parametrize("C,bits", [(200, 8), (300, 10), (1500, 11), (3000, 12), (6000, 13)])
def test_split_to_packed_widths(cuda, oracle, C, bits):
    """A bf16 codebook of exactly C distinct values (spread evenly over the
    bf16 patterns of the synthetic normal table), split format built from the
    module, then decoded to the transient stream at the width prefill_bits(C)
    gives."""
    import synthetic
    from gpu_huffman_functions import prefill_bits, split_inverse
    from test_gpu_huffman import _lin
    assert prefill_bits(C) == bits
    rng = np.random.default_rng(C)
    pats, _ = synthetic.normal_bf16_table(0.02)
    sel = np.linspace(0, len(pats) - 1, C).round().astype(np.int64)
    assert np.unique(sel).size == C
    vals = (pats[sel].astype(np.uint32) << 16).view(np.float32)
    M, K = 48, 4096
    pick = rng.integers(0, C, size=M * K)
    pick[:C] = np.arange(C)                                     # every value occurs
    w = vals[pick].reshape(M, K)
    cb, idx = cbb.frequency_sorted_codebook(w)
    assert len(cb) == C
    enc = hc.huffman_encode_indices(idx, shape=(M, K))
    lin = _lin(enc, cb, M, K)
    assert lin.split is not None
    inv = split_inverse(cb, cuda)
    out = torch.zeros(M * K * bits // 8 + 16, dtype=torch.uint8, device=cuda)
    nat.check(nat.load().cbq_split_to_packed(ctypes.byref(lin.split[1]), inv.data_ptr(), bits,
                                             out.data_ptr(), nat.stream_ptr(cuda)), "s2p")
    want = oracle.pack_lsb(idx.reshape(-1).astype(np.int64), bits)
    assert np.array_equal(out.cpu().numpy()[:want.size], want)
