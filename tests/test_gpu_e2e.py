"""GPU always-compressed decoder vs transformers' Qwen3 golden tokens.

decoder.from_compressed builds the model from reference-format data dicts,
as AdaptiveCodebookLinear.from_compressed would.  Every linear, the lm_head
and the embedding run through libcbq_hip.so, and so does the fp32 glue
(include/cbq_decode.h; multi-token attention is torch matmuls).  Greedy
tokens must equal the golden ones (tests/golden/e2e_golden.npz, from
transformers' Qwen3ForCausalLM on the same dense weights), for fixed-width
and Huffman weights alike.
"""
import os

import numpy as np
import pytest
import torch

import decoder
import synthetic
from conftest import rel_l2

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "e2e_golden.npz")


@pytest.mark.parametrize("encoding", ["fixed", "huffman"])
def test_gpu_decoder_matches_transformers(cuda, encoding):
    g = np.load(GOLDEN)
    for name in sorted({k.split("/")[0] for k in g.files}):
        layers, hidden, inter, n_q, n_kv, hd, vocab, seed = [int(v) for v in g[f"{name}/config"]]
        cfg = decoder.DecoderConfig(layers=layers, hidden=hidden, inter=inter, n_q=n_q,
                                    n_kv=n_kv, head_dim=hd, vocab=vocab)
        comp = synthetic.compress_model_cpu(cfg, seed, encoding)
        model = decoder.from_compressed(cfg, comp, device=cuda, max_len=64)
        want = [int(t) for t in g[f"{name}/tokens"]]
        toks, logits = model.generate([int(t) for t in g[f"{name}/prompt"]], len(want),
                                      return_logits=True)
        print(name, encoding, rel_l2(logits.cpu().numpy(), g[f"{name}/logits0"]), flush=True)
        assert rel_l2(logits.cpu().numpy(), g[f"{name}/logits0"]) <= 1e-4, name
        assert toks == want, (name, toks, want)


def test_prefill_equals_incremental(cuda):
    """Logits after a 12-token prompt equal those after feeding the same
    tokens one at a time (KV cache and positions)."""
    cfg = decoder.DecoderConfig(layers=2, hidden=256, inter=512, n_q=4, n_kv=2, head_dim=64,
                                vocab=512)
    comp = synthetic.compress_model_cpu(cfg, 5, "fixed")
    m = decoder.from_compressed(cfg, comp, device=cuda, max_len=32)
    ids = list(np.random.default_rng(0).integers(0, cfg.vocab, 12))
    m.reset()
    a = m.forward(torch.tensor(ids)).cpu().numpy()
    m.reset()
    for t in ids:
        b = m.forward(torch.tensor([t]))
    assert rel_l2(b.cpu().numpy(), a) <= 1e-5


@pytest.mark.parametrize("encoding", ["fixed", "huffman"])
def test_graph_decode_matches_eager(cuda, encoding):
    """Decode steps captured once as a HIP graph and replayed give the same
    tokens as the eager loop, on a fresh model, and again on a second run
    (the graph replays several times, with eager work in between)."""
    cfg = decoder.DecoderConfig(layers=2, hidden=256, inter=512, n_q=4, n_kv=2, head_dim=64,
                                vocab=1024)
    comp = synthetic.compress_model_cpu(cfg, 7, encoding)
    m = decoder.from_compressed(cfg, comp, device=cuda, max_len=48)
    prompt = [int(t) for t in np.random.default_rng(1).integers(0, cfg.vocab, 9)]
    eager = m.generate(prompt, 20)
    g1 = m.generate_graph(prompt, 20)
    g2 = m.generate_graph(prompt[:5], 20)
    eager2 = m.generate(prompt[:5], 20)
    assert g1 == eager
    assert g2 == eager2
