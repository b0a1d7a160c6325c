"""benchmark config 5 at full size: the random-init 36-layer Qwen3-8B-shape
decoder on the GPU against the CPU oracle's golden run
(tests/golden/gen_e2e_full_golden.py: the reference's own C kernel for every
GEMV, numpy fp32 glue pinned to transformers' Qwen3).

The GPU rebuilds exactly the oracle's model: synthetic.make_bf16 gives the
same weight bits on both sides (checked here through the per-category
codebooks' CRCs and the first packed bytes of two tensors).  Both encodings
run: fixed-width 13-bit indices and canonical Huffman (split format); the
oracle's Huffman GEMV equals its fixed-width GEMV bit for bit (recorded in
the fixture), so one golden serves both.  Greedy tokens must equal the
golden's; the first step's logits (after the 128-token prompt, which runs on
the fp32 matrix cores) within rel-L2 1e-4."""
import os
import zlib

import numpy as np
import pytest
import torch

import decoder
import synthetic

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "e2e_qwen3_8b_golden.npz")
LOGITS_TOL = 1e-4


@pytest.fixture(scope="module")
def golden():
    g = np.load(GOLDEN, allow_pickle=False)
    assert bool(g["huffman_equals_fixed"][0])
    return {k: g[k] for k in g.files}


@pytest.fixture(scope="module")
def dec(cuda):
    return synthetic.SyntheticDecoder("qwen3-8b", log=lambda *a: None)


def _cfg(dec):
    c = dec.cfg
    return decoder.DecoderConfig(layers=c["layers"], hidden=c["hidden"], inter=c["inter"],
                                 n_q=c["n_q"], n_kv=c["n_kv"], head_dim=c["head_dim"],
                                 vocab=c["vocab"])


@pytest.mark.parametrize("encoding", ["fixed", "huffman"])
def test_full_decoder_matches_oracle(cuda, golden, dec, encoding):
    names = dec.all_linears() + [dec.embed]
    print(f"e2e full: building {encoding}", flush=True)
    tensors = dec.build_huffman(names) if encoding == "huffman" else dec.build_fixed(names)
    if encoding == "fixed":
        cats = {"attention": "model.layers.0.self_attn.q_proj",
                "mlp_ffn": "model.layers.0.mlp.gate_proj", "embedding": "lm_head"}
        for i, cat in enumerate(("attention", "mlp_ffn", "embedding")):
            cb = tensors[cats[cat]].codebook.cpu().numpy()
            assert cb.size == int(golden["codebook_sizes"][i]), cat
            assert zlib.crc32(cb.tobytes()) == int(golden["codebook_crc32"][i]), cat
        for n, key in (("model.layers.0.self_attn.q_proj", "q_proj0_packed_head"),
                       ("lm_head", "lm_head_packed_head")):
            head = golden[key]
            assert np.array_equal(tensors[n].packed[:head.size].cpu().numpy(), head), n
    prompt = [int(t) for t in golden["prompt"]]
    want = [int(t) for t in golden["tokens"]]
    model = decoder.from_synthetic(_cfg(dec), tensors, max_len=len(prompt) + len(want))
    del tensors
    model.reset()
    logits0 = model.forward(torch.tensor(prompt)).cpu().numpy()
    ref = golden["logits0"]
    rel = float(np.linalg.norm(logits0.astype(np.float64) - ref) / np.linalg.norm(ref))
    print(f"e2e full {encoding}: step-0 logits rel-L2 {rel:.3e}", flush=True)
    assert rel <= LOGITS_TOL, rel
    toks = model.generate_graph(prompt, len(want))
    print(f"e2e full {encoding}: tokens {toks[:8]}... golden {want[:8]}...", flush=True)
    first_diff = next((i for i, (a, b) in enumerate(zip(toks, want)) if a != b), None)
    assert first_diff is None, (first_diff, float(golden["margins"][first_diff]))
    del model
    torch.cuda.empty_cache()
