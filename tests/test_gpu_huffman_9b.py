"""Config 3 at the 9B model's own shapes: canonical-Huffman streams of full
12288 x 4096 (gate/up), 4096 x 12288 (down) and 1024 x 4096 (k/v) matrices,
encoded on the CPU exactly as the reference encoder does, run through
HuffmanCodebookLinear with each device format (split, the reference-format
stream, stream + column layout) and checked against the oracle's C
huffman_matmul (src/compressed_matmul_cpu.py:446-506 restated) on the same
stream: rel-L2 <= 1e-5.  The split format also runs 4 and 16 tokens (the
fused few-token kernel) and 40 tokens (decoded to a transient fixed-width
stream, then the fp32 matrix-core GEMM); every format decodes back to the
encoder's indices bit for bit.  Weights: bf16-rounded N(0, 0.02), the
frequency-sorted lossless codebook (~5 100 entries, 13-bit indices)."""
import numpy as np
import pytest
import torch

import codebook_builder as cbb
import huffman_codebook as hc
from conftest import rel_l2
from test_gpu_huffman import _lin

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(scope="module")
def mats():
    return {}


def _case(mats, M, K):
    if (M, K) not in mats:
        w = cbb.bf16_round(np.random.default_rng(M * 7 + K).standard_normal((M, K))
                           .astype(np.float32) * 0.02)
        cb, idx = cbb.frequency_sorted_codebook(w)
        del w
        mats[(M, K)] = (cb, idx, hc.huffman_encode_indices(idx, shape=(M, K)))
    return mats[(M, K)]


@pytest.mark.parametrize("M,K", [(12288, 4096), (4096, 12288), (1024, 4096)])
@pytest.mark.parametrize("layout", ["split", "stream", "columns"])
def test_full_shape_layouts(cuda, oracle, mats, M, K, layout):
    cb, idx, enc = _case(mats, M, K)
    print("case", M, K, layout, flush=True)
    lin = _lin(enc, cb, M, K, layout=layout)
    assert (lin.split is not None) == (layout == "split")
    dec = lin.decode_indices().cpu().numpy().reshape(-1)
    assert np.array_equal(dec, idx.astype(np.int32).reshape(-1))
    rng = np.random.default_rng(M + K)
    for T in ((1, 4, 16, 40) if layout == "split" else (1,)):
        x = rng.standard_normal((T, K)).astype(np.float32)
        y = lin(torch.from_numpy(x).to(cuda)).cpu().numpy()
        ref = oracle.huff_gemv(x, enc, cb, M, K, chunk_rows=None)
        assert rel_l2(y, ref) <= TOL, (M, K, layout, T)
