"""Golden greedy tokens of the full benchmark config-5 decoder, written by the
CPU oracle (test fixture generator; run in this container, not on the GPU box).

The model is the random-init 36-layer Qwen3-8B-shape decoder the bench and
the GPU decoder run: every linear, the lm_head and the embedding stored as
lossless codebook indices (one frequency-sorted codebook per category:
attention, mlp_ffn, embedding; 13 bits each).  Weights come from
synthetic.make_bf16, the counter-based generator that gives the same bits on
the CPU and on the GPU, so tests/test_gpu_e2e_full.py rebuilds exactly this
model on the GPU, fixed-width and Huffman, and compares its tokens and
first-step logits with the ones written here.

The oracle is oracle/cpu_decoder.py (Qwen3 glue in numpy fp32, pinned to
transformers' Qwen3ForCausalLM by tests/golden/gen_e2e_golden.py) with every
fixed-width GEMV run by the reference's own compiled C kernel
(oracle/_ref, src/compressed_matmul.c compressed_matmul_f32_chunk) when it is
built here, else by its restatement (bitwise equal to it on the committed
golden vectors).

Huffman: the C GEMV over a canonical-Huffman stream adds the same codebook
values in the same order as over the fixed-width stream
(src/compressed_matmul.c:208-239 against :416-450), so the Huffman model's
logits are the fixed-width ones bit for bit.  Rather than decode the whole
model twice on the CPU, this script checks that equality on layer 0's
q_proj and gate_proj and records it.

    python tests/golden/gen_e2e_full_golden.py [--tokens 256] [--prompt 128]

About 35 minutes on 8 cores (12 for the prompt, ~5 s per generated token) and ~30 GB of RAM.
"""
import argparse
import os
import sys
import time
import zlib

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "codebook-quantization_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import torch  # noqa: E402

import cbq_oracle as O  # noqa: E402
import codebook_builder as cbb  # noqa: E402
import decoder as D  # noqa: E402
import huffman_codebook as hc  # noqa: E402
import synthetic  # noqa: E402
from cpu_decoder import CpuQwen3  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "e2e_qwen3_8b_golden.npz")
PACK_CHUNK = 1 << 24                     # indices per packing call (multiple of 8)


def log(*a):
    print("[golden]", *a, flush=True)


def pack_chunked(idx: torch.Tensor, bits: int) -> np.ndarray:
    """LSB-first packing (cbb.pack_torch) in chunks of 2^24 indices, whose
    packed lengths are whole bytes, plus 4 zero pad bytes."""
    n = idx.numel()
    nb = (n * bits + 7) // 8
    out = np.zeros(nb + 4, np.uint8)
    o = 0
    for s0 in range(0, n, PACK_CHUNK):
        pk = cbb.pack_torch(idx[s0:s0 + PACK_CHUNK], bits).numpy()
        out[o:o + pk.size] = pk
        o += pk.size
    assert o == nb
    return out


def build_model(cfg: D.DecoderConfig, threads: int):
    torch.set_num_threads(threads)
    names = cfg.linear_shapes() + [("model.embed_tokens", cfg.vocab, cfg.hidden)]
    cats = {}
    for n, M, K in names:
        cats.setdefault(cbb.classify_tensor(n), []).append((n, M, K))
    comp, books = {}, {}
    for cat, ts in cats.items():
        t0 = time.time()
        pats = {}
        counts = torch.zeros(65536, dtype=torch.int64)
        for n, M, K in ts:
            p = cbb.patterns_torch(synthetic.make_bf16((M, K), n, device="cpu")).reshape(-1)
            counts += torch.bincount(p, minlength=65536)
            pats[n] = p.to(torch.int16)
        cb, lut = cbb.codebook_from_counts_torch(counts)
        bits = cbb.bits_for(cb.numel())
        books[cat] = cb.numpy().copy()
        for n, M, K in ts:
            idx = lut[pats.pop(n).to(torch.int64) & 0xFFFF]
            comp[n] = {"mode": "direct_codebook", "shape": (M, K), "bits": bits,
                       "codebook": books[cat], "indices": pack_chunked(idx, bits)}
            del idx
        log(f"{cat}: {len(ts)} tensors, C={cb.numel()}, {bits} bits, {time.time() - t0:.0f}s")
    return comp, books


def huffman_check(comp, x_q: np.ndarray, x_gate: np.ndarray, kind: str) -> bool:
    """The oracle's Huffman GEMV equals its fixed-width GEMV bit for bit on
    layer 0's q_proj and gate_proj (same values, same summation order; any
    x shows it, here seeded N(0, 1) rows)."""
    ok = True
    for n, x in (("model.layers.0.self_attn.q_proj", x_q), ("model.layers.0.mlp.gate_proj", x_gate)):
        d = comp[n]
        M, K = d["shape"]
        idx = O.unpack_indices_c(d["indices"], d["bits"], M * K)
        enc = hc.huffman_encode_indices(idx, shape=(M, K))
        yh = O.huff_gemv(x, enc, d["codebook"], M, K, chunk_rows=None)
        yf = O.fixed_gemv(x, d["indices"], d["codebook"], M, K, d["bits"], chunk_rows=None,
                          kind=kind)
        same = bool(np.array_equal(yh.view(np.uint32), yf.view(np.uint32)))
        log(f"huffman vs fixed oracle GEMV on {n}: bitwise equal {same}")
        ok &= same
    return ok


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--tokens", type=int, default=256)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 8)
    ap.add_argument("--out", default=OUT)
    ap.add_argument("--layers", type=int, default=0)
    ap.add_argument("--vocab", type=int, default=151936)
    args = ap.parse_args()

    cfg = D.QWEN3_8B
    if args.layers:                          # reduced dry run of the script itself
        cfg = D.DecoderConfig(**{**cfg.__dict__, "layers": args.layers, "vocab": args.vocab})
    kind = "ref" if O.ref_available() else "oracle"
    t0 = time.time()
    comp, books = build_model(cfg, args.threads)
    log(f"model built in {time.time() - t0:.0f}s; GEMV kernel: {kind}")

    prompt = np.random.default_rng(2).integers(0, cfg.vocab, args.prompt).astype(np.int64)
    oracle = CpuQwen3(cfg, comp, max_len=args.prompt + args.tokens, threads=args.threads,
                      kind=kind)

    t0 = time.time()
    logits = oracle.forward(prompt)
    log(f"prompt of {args.prompt} tokens in {time.time() - t0:.0f}s")
    logits0 = logits.copy()
    toks, margins, top1 = [], [], []
    for s in range(args.tokens):
        order = np.argsort(logits)[::-1]
        tok = int(np.argmax(logits))
        toks.append(tok)
        margins.append(float(logits[order[0]] - logits[order[1]]))
        top1.append(float(logits[tok]))
        if len(toks) == args.tokens:
            break
        t1 = time.time()
        logits = oracle.forward([tok])
        log(f"token {s + 1}: {tok} (margin {margins[-1]:.4g}) {time.time() - t1:.1f}s")

    xr = np.random.default_rng(3).standard_normal((2, cfg.hidden)).astype(np.float32)
    huff_ok = huffman_check(comp, xr[:1], xr[1:], kind)

    cb_crc = {cat: zlib.crc32(cb.tobytes()) for cat, cb in books.items()}
    sample = {n: comp[n]["indices"][:4096].copy()
              for n in ("model.layers.0.self_attn.q_proj", "lm_head")}
    np.savez_compressed(
        args.out,
        prompt=prompt.astype(np.int32), tokens=np.asarray(toks, np.int32),
        logits0=logits0.astype(np.float32), margins=np.asarray(margins, np.float32),
        top1=np.asarray(top1, np.float32),
        codebook_sizes=np.asarray([books[c].size for c in ("attention", "mlp_ffn", "embedding")],
                                  np.int32),
        codebook_crc32=np.asarray([cb_crc[c] for c in ("attention", "mlp_ffn", "embedding")],
                                  np.uint32),
        q_proj0_packed_head=sample["model.layers.0.self_attn.q_proj"],
        lm_head_packed_head=sample["lm_head"],
        huffman_equals_fixed=np.asarray([huff_ok]),
        gemv_kernel=np.asarray([kind]))
    log(f"wrote {args.out}: tokens {toks[:8]}..., min margin {min(margins):.4g}")


if __name__ == "__main__":
    main()
