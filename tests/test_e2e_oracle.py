"""CPU oracle decoder vs transformers' Qwen3 on the same compressed weights.

tests/golden/e2e_golden.npz holds greedy tokens and first-step logits that
transformers' Qwen3ForCausalLM (float32, eager attention) produced from the
exact dense decode of synthetic.compress_model_cpu's tensors.  The oracle
decoder (oracle/cpu_decoder.py) runs the same model through the C restatement
of the reference kernels, with the weights in fixed-width and in Huffman form.
It must give the same tokens, and logits within fp32 reordering noise.
"""
import os

import numpy as np
import pytest

import decoder
import synthetic
from conftest import rel_l2

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "e2e_golden.npz")


def cases():
    g = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in g.files})
    return g, names


def _cfg(c):
    layers, hidden, inter, n_q, n_kv, hd, vocab, seed = [int(v) for v in c]
    return decoder.DecoderConfig(layers=layers, hidden=hidden, inter=inter, n_q=n_q, n_kv=n_kv,
                                 head_dim=hd, vocab=vocab), seed


@pytest.mark.parametrize("encoding", ["fixed", "huffman"])
def test_oracle_decoder_matches_transformers(oracle, encoding):
    import cpu_decoder
    g, names = cases()
    for name in names:
        cfg, seed = _cfg(g[f"{name}/config"])
        comp = synthetic.compress_model_cpu(cfg, seed, encoding)
        model = cpu_decoder.CpuQwen3(cfg, comp, max_len=64)
        prompt = g[f"{name}/prompt"]
        want = g[f"{name}/tokens"]
        toks, logits = model.generate(prompt, len(want), return_logits=True)
        assert rel_l2(logits, g[f"{name}/logits0"]) <= 1e-5, name
        assert toks == [int(t) for t in want], (name, toks, list(want))


def test_compressed_weights_are_the_golden_weights():
    """Fixed-width and Huffman forms of the same tensor decode to the same
    dense bf16 weights (the fixture was built from these)."""
    import bitpack
    cfg = decoder.DecoderConfig(layers=1, hidden=128, inter=256, n_q=2, n_kv=1, head_dim=64,
                                vocab=256)
    f = synthetic.compress_model_cpu(cfg, 3, "fixed")
    n = "model.layers.0.mlp.up_proj"
    M, K = f[n]["shape"]
    idx = bitpack.unpack_any_bits(f[n]["indices"], f[n]["bits"], M * K)
    assert np.array_equal(f[n]["codebook"][idx].reshape(M, K), f[n]["_dense"])
