"""Golden greedy tokens for the compressed decoder from transformers' Qwen3.

Builds small random-init Qwen3-style decoders whose every matrix is the exact
dense decode of the compressed tensors that synthetic.compress_model_cpu
produces (bf16 N(0, 0.02) values, per-tensor PCG64 seeds).  It loads them into
transformers' Qwen3ForCausalLM (float32, eager attention, norm weights 1) and
records:
  - the prompt;
  - the first-step logits;
  - the greedy tokens, from a plain full-recompute loop.

The reference's compressed modules run inside this modelling code
(src/model_loader.py:213-277), so these fixtures pin the decoder glue, both
codebook-quantization_amd/decoder.py and oracle/cpu_decoder.py.

Run from the repository root:  python tests/golden/gen_e2e_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "codebook-quantization_amd"))

import decoder  # noqa: E402
import synthetic  # noqa: E402

CASES = {
    # name: (config, base_seed, prompt_len, new_tokens)
    "tiny": (decoder.DecoderConfig(layers=2, hidden=256, inter=512, n_q=4, n_kv=2, head_dim=64,
                                   vocab=1024), 0, 16, 16),
    "deep": (decoder.DecoderConfig(layers=4, hidden=512, inter=1024, n_q=4, n_kv=1,
                                   head_dim=128, vocab=2048), 1, 24, 12),
}


def hf_tokens(cfg, dense, prompt, n_new):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    hc = Qwen3Config(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.inter,
                     num_hidden_layers=cfg.layers, num_attention_heads=cfg.n_q,
                     num_key_value_heads=cfg.n_kv, head_dim=cfg.head_dim,
                     max_position_embeddings=512, rms_norm_eps=cfg.eps,
                     rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta},
                     tie_word_embeddings=False, attention_bias=False,
                     attn_implementation="eager")
    m = Qwen3ForCausalLM(hc).float().eval()
    sd = m.state_dict()
    for k in sd:
        if k.endswith("norm.weight"):
            sd[k] = torch.ones_like(sd[k])
        else:
            name = k[:-len(".weight")]
            sd[k] = torch.from_numpy(dense[name])
    m.load_state_dict(sd)
    ids = torch.tensor([prompt], dtype=torch.int64)
    out, first = [], None
    with torch.no_grad():
        for _ in range(n_new):
            logits = m(ids).logits[0, -1].float()
            if first is None:
                first = logits.numpy().copy()
            tok = int(torch.argmax(logits))
            out.append(tok)
            ids = torch.cat([ids, torch.tensor([[tok]])], dim=1)
    return out, first


def main():
    arrays = {}
    for name, (cfg, seed, plen, n_new) in CASES.items():
        comp = synthetic.compress_model_cpu(cfg, seed, "fixed")
        dense = {n: d["_dense"] for n, d in comp.items()}
        prompt = np.random.default_rng(2 + seed).integers(0, cfg.vocab, plen)
        toks, first = hf_tokens(cfg, dense, [int(t) for t in prompt], n_new)
        print(name, "tokens", toks)
        arrays[f"{name}/prompt"] = prompt.astype(np.int64)
        arrays[f"{name}/tokens"] = np.array(toks, np.int64)
        arrays[f"{name}/logits0"] = first.astype(np.float32)
        arrays[f"{name}/config"] = np.array([cfg.layers, cfg.hidden, cfg.inter, cfg.n_q, cfg.n_kv,
                                             cfg.head_dim, cfg.vocab, seed], np.int64)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "e2e_golden.npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path)


if __name__ == "__main__":
    main()
