"""Always-compressed Qwen3-style greedy decoder (batch 1) on the gfx950 library.

This is the end-to-end caller of the compressed path: every linear of every
layer, the lm_head and the token embedding stay compressed in HBM, as
fixed-width indices or canonical Huffman, and run through libcbq_hip.so.
The glue around them runs as fused fp32 HIP kernels of the same library
(include/cbq_decode.h: residual add + RMSNorm, head norm + rope + KV-cache
write, single-token attention, SiLU product); multi-token attention uses
torch matmuls.  It follows the HF Qwen3 modelling that the reference's
compressed modules plug into (src/model_loader.py:213-277):

- RMSNorm: x * rsqrt(mean(x^2) + eps) * weight;
- q/k head RMSNorm;
- rotary embedding ("default" rope, rotate-half form);
- grouped-query causal attention with an fp32 softmax;
- SiLU-gated MLP;
- final norm, then argmax over the logits.

For a random-init model the norm weights are ones, as at HF initialisation.

Activations are fp32 throughout, so the compressed GEMVs run their fp32
kernels (rel-L2 <= 1e-5 against the reference's C kernel).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, List, Optional

import numpy as np
import torch

LAYER_LINEARS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                 "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


@dataclass(frozen=True)
class DecoderConfig:
    layers: int
    hidden: int
    inter: int
    n_q: int
    n_kv: int
    head_dim: int
    vocab: int
    rope_theta: float = 1.0e6          # Qwen3-8B's published config
    eps: float = 1.0e-6

    def linear_shapes(self):
        """(name, out_features, in_features) of every compressed matrix."""
        h, hd = self.hidden, self.head_dim
        per = {"self_attn.q_proj": (self.n_q * hd, h), "self_attn.k_proj": (self.n_kv * hd, h),
               "self_attn.v_proj": (self.n_kv * hd, h), "self_attn.o_proj": (h, self.n_q * hd),
               "mlp.gate_proj": (self.inter, h), "mlp.up_proj": (self.inter, h),
               "mlp.down_proj": (h, self.inter)}
        out = [(f"model.layers.{i}.{n}", *per[n]) for i in range(self.layers) for n in LAYER_LINEARS]
        return out + [("lm_head", self.vocab, h)]


QWEN3_8B = DecoderConfig(layers=36, hidden=4096, inter=12288, n_q=32, n_kv=8, head_dim=128,
                         vocab=151936)


def rope_tables(cfg: DecoderConfig, max_len: int):
    """cos, sin [max_len, head_dim] float32, computed as HF's default rotary
    embedding does: fp32 inverse frequencies, fp32 angles, duplicated halves."""
    d = cfg.head_dim
    inv = (1.0 / (np.float32(cfg.rope_theta) ** (np.arange(0, d, 2, dtype=np.int64)
                                                  .astype(np.float32) / np.float32(d))))
    inv = inv.astype(np.float32)
    pos = np.arange(max_len, dtype=np.float32)
    freqs = (pos[:, None] * inv[None, :]).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    t = torch.from_numpy(emb)
    return t.cos().numpy(), t.sin().numpy()


Linear = Callable[[torch.Tensor], torch.Tensor]        # [T, K] fp32 -> [T, M] fp32


class _Glue:
    """The fused decoder kernels of libcbq_hip.so (include/cbq_decode.h) on
    torch's current stream; outputs are fresh tensors (graph-pool memory
    under capture)."""

    def __init__(self, cfg: DecoderConfig):
        import cbq_native as nat
        self.nat = nat
        self.lib = nat.load()
        self.cfg = cfg

    def add_rms(self, h: torch.Tensor, delta: Optional[torch.Tensor]) -> torch.Tensor:
        """h += delta (in place, when given); returns rmsnorm(h)."""
        T, H = h.shape
        out = torch.empty_like(h)
        self.nat.check(self.lib.cbq_add_rmsnorm_f32(
            h.data_ptr(), None if delta is None else delta.data_ptr(), None, out.data_ptr(),
            T, H, self.cfg.eps, self.nat.stream_ptr(h.device)), "cbq_add_rmsnorm_f32")
        return out

    def head_norm_rope(self, q, k, v, cos, sin, pos_dev, k_cache, v_cache) -> torch.Tensor:
        c = self.cfg
        T = q.shape[0]
        q_out = torch.empty(T, c.n_q * c.head_dim, dtype=torch.float32, device=q.device)
        self.nat.check(self.lib.cbq_head_norm_rope_f32(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None, cos.data_ptr(), sin.data_ptr(),
            pos_dev.data_ptr(), q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
            T, c.n_q, c.n_kv, c.head_dim, k_cache.shape[1], c.eps,
            self.nat.stream_ptr(q.device)), "cbq_head_norm_rope_f32")
        return q_out

    def attn_workspace(self, device, max_len: int) -> torch.Tensor:
        """Scratch of the split one-token attention, allocated once per device
        and cache length (before any graph capture)."""
        key = (torch.device(device), int(max_len))
        if getattr(self, "_aws", None) is None or self._aws[0] != key:
            n = self.lib.cbq_attn_rope_decode_workspace(self.cfg.n_q, self.cfg.head_dim,
                                                        int(max_len))
            self._aws = (key, torch.empty(n, dtype=torch.uint8, device=key[0]))
        return self._aws[1]

    # Caches at least this long take the split-over-blocks attention: one
    # block per head is held to one CU's load bandwidth, which the longer
    # contexts exceed; below it the single launch is cheaper than the split
    # launch plus its merge launch.
    SPLIT_ATTN_MIN_LEN = 2048

    def attend_rope1(self, q, k, v, cos, sin, pos_dev, k_cache, v_cache) -> torch.Tensor:
        """One token: head norm + rope of q and k, cache write, attention."""
        c = self.cfg
        out = torch.empty(1, c.n_q * c.head_dim, dtype=torch.float32, device=q.device)
        max_len = k_cache.shape[1]
        args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None, cos.data_ptr(),
                sin.data_ptr(), pos_dev.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                out.data_ptr(), c.n_q, c.n_kv, c.head_dim, max_len, float(c.head_dim ** -0.5),
                c.eps)
        if max_len >= self.SPLIT_ATTN_MIN_LEN:
            ws = self.attn_workspace(q.device, max_len)
            self.nat.check(self.lib.cbq_attn_rope_decode_ws_f32(
                *args, ws.data_ptr(), ws.numel(), self.nat.stream_ptr(q.device)),
                "cbq_attn_rope_decode_ws_f32")
        else:
            self.nat.check(self.lib.cbq_attn_rope_decode_f32(
                *args, self.nat.stream_ptr(q.device)), "cbq_attn_rope_decode_f32")
        return out

    def argmax_step(self, logits, ids32, toks, pos_dev, first: int) -> None:
        """ids32[0] = argmax(logits); toks[pos - first] = it; pos += 1."""
        if getattr(self, "_ws", None) is None or self._ws.device != logits.device:
            self._ws = torch.empty(256, dtype=torch.int32, device=logits.device)
        self.nat.check(self.lib.cbq_argmax_step(
            logits.data_ptr(), logits.numel(), self._ws.data_ptr(), ids32.data_ptr(), toks.data_ptr(),
            pos_dev.data_ptr(), first, toks.numel(), self.nat.stream_ptr(logits.device)),
            "cbq_argmax_step")

    def silu_mul(self, g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(g)
        self.nat.check(self.lib.cbq_silu_mul_f32(g.data_ptr(), u.data_ptr(), out.data_ptr(),
                                                 g.numel(), self.nat.stream_ptr(g.device)),
                       "cbq_silu_mul_f32")
        return out


class Qwen3Decoder:
    """Greedy decoder over compressed linears / embedding (callables)."""

    def __init__(self, cfg: DecoderConfig, linears: Dict[str, Linear], embed: Callable,
                 device: torch.device, max_len: int = 512, fuse_glue: bool = True):
        self.cfg = cfg
        self.linears = linears
        self.embed = embed
        self.device = torch.device(device)
        self.max_len = max_len
        cos, sin = rope_tables(cfg, max_len)
        self.cos = torch.from_numpy(cos).to(self.device)
        self.sin = torch.from_numpy(sin).to(self.device)
        kv = (cfg.layers, 2, cfg.n_kv, max_len, cfg.head_dim)
        self.cache = torch.zeros(kv, dtype=torch.float32, device=self.device)
        self.pos = 0
        self.glue = _Glue(cfg)
        if max_len >= _Glue.SPLIT_ATTN_MIN_LEN:
            self.glue.attn_workspace(self.device, max_len)
        # One-token steps fold RMSNorm / SiLU into the GEMVs' x staging when
        # every linear that consumes them offers `xform` (stacked q/k/v and
        # gate/up, down, lm_head): 5 launches per layer instead of 8, with
        # values identical to the separate glue kernels.  The GEMVs stage a
        # transformed x of at most 16384 values.
        need = ["lm_head"] + [f"model.layers.{i}.{n}" for i in range(cfg.layers)
                              for n in ("self_attn.qkv_proj", "mlp.gate_up_proj", "mlp.down_proj")]
        self.fused = (fuse_glue and max(cfg.hidden, cfg.inter) <= 16384 and
                      all(callable(getattr(linears.get(n), "xform", None)) for n in need))

    # ---- building blocks (HF Qwen3 semantics, fp32) -------------------------
    def _attend(self, i: int, q: torch.Tensor, L: int, pos: torch.Tensor) -> torch.Tensor:
        """Causal GQA over cache positions [0, L): q [T, n_q, hd] -> [T, n_q*hd].
        Query head h reads kv head h // (n_q / n_kv), as HF's repeat_kv; the
        grouping is a reshape, so no kv copy is made."""
        c = self.cfg
        T = q.shape[0]
        rep = c.n_q // c.n_kv
        kk = self.cache[i, 0, :, :L]                                    # [n_kv, L, hd]
        vv = self.cache[i, 1, :, :L]
        qg = q.reshape(T, c.n_kv, rep, c.head_dim).permute(1, 0, 2, 3).reshape(c.n_kv, T * rep,
                                                                            c.head_dim)
        scores = torch.matmul(qg, kk.transpose(1, 2).contiguous()) * (c.head_dim ** -0.5)
        # query row r of group g is token r // rep
        tpos = pos.repeat_interleave(rep)                               # [T * rep]
        causal = torch.arange(L, device=self.device)[None, :] > tpos[:, None]
        scores = scores.masked_fill(causal[None], float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        att = torch.matmul(probs, vv)                                   # [n_kv, T*rep, hd]
        return att.reshape(c.n_kv, T, rep, c.head_dim).permute(1, 0, 2, 3).reshape(
            T, c.n_q * c.head_dim)

    def _layer(self, i: int, h: torch.Tensor, x: torch.Tensor, pos: torch.Tensor,
               pos_dev: torch.Tensor, L: int) -> torch.Tensor:
        """One layer over T tokens at positions pos (pos_dev: device int64
        holding pos[0]; L = pos[-1] + 1, or max_len for the captured step).
        x = rmsnorm(h) on entry; h is updated in place; returns the next
        rmsnorm(h)."""
        c = self.cfg
        T = h.shape[0]
        p = f"model.layers.{i}."
        g = self.glue
        qkv = self.linears.get(p + "self_attn.qkv_proj")
        if qkv is not None:                          # row-stacked q/k/v: one launch
            y = qkv(x)
            nq, nk = c.n_q * c.head_dim, c.n_kv * c.head_dim
            q, k, v = (y[:, :nq].contiguous(), y[:, nq:nq + nk].contiguous(),
                       y[:, nq + nk:].contiguous())
        else:
            q = self.linears[p + "self_attn.q_proj"](x)
            k = self.linears[p + "self_attn.k_proj"](x)
            v = self.linears[p + "self_attn.v_proj"](x)
        if T == 1:
            att = g.attend_rope1(q, k, v, self.cos, self.sin, pos_dev, self.cache[i, 0],
                                 self.cache[i, 1])
        else:
            q = g.head_norm_rope(q, k, v, self.cos, self.sin, pos_dev, self.cache[i, 0],
                                 self.cache[i, 1])
            att = self._attend(i, q.view(T, c.n_q, c.head_dim), L, pos)
        x = g.add_rms(h, self.linears[p + "self_attn.o_proj"](att))
        gu = self.linears.get(p + "mlp.gate_up_proj")
        if gu is not None:                           # row-stacked gate/up: one launch
            y = gu(x)
            a = g.silu_mul(y[:, :c.inter].contiguous(), y[:, c.inter:].contiguous())
        else:
            a = g.silu_mul(self.linears[p + "mlp.gate_proj"](x), self.linears[p + "mlp.up_proj"](x))
        return g.add_rms(h, self.linears[p + "mlp.down_proj"](a))

    # ---- captured decode step (static shapes) -------------------------------
    def _graph_step(self, ids_buf: torch.Tensor, pos_buf: torch.Tensor, toks: torch.Tensor,
                    first_pos: int):
        """One token at device position pos_buf[0] (kernels read the position
        from device memory, so launch shapes never change).  Writes the argmax
        into ids_buf (int32, next input) and toks[pos - first_pos], and
        advances pos_buf."""
        c = self.cfg
        h = self.embed(ids_buf).reshape(1, c.hidden).to(torch.float32)
        if self.fused:
            logits = self._forward1_fused(h, pos_buf, pick=(ids_buf, toks, pos_buf, first_pos))
            if logits is None:                      # the lm_head GEMV picked the token itself
                return
        else:
            x = self.glue.add_rms(h, None)
            for i in range(c.layers):
                x = self._layer(i, h, x, pos_buf, pos_buf, self.max_len)
            logits = self.linears["lm_head"](x).reshape(-1)
        self.glue.argmax_step(logits, ids_buf, toks, pos_buf, first_pos)

    def _forward1_fused(self, h: torch.Tensor, pos_dev: torch.Tensor, pick=None):
        """One token through every layer with the norms and the SiLU product
        applied by the GEMVs that consume them; h [1, hidden] is the
        embedding.  Returns the logits [vocab]; with pick = (ids32, toks,
        pos, first) and an lm_head that fuses the greedy pick
        (`xform_argmax`), the pick is made in the lm_head GEMV instead
        (cbq_argmax_step's bookkeeping) and None is returned."""
        import cbq_native as nat
        c = self.cfg
        L = self.linears
        nq, nk = c.n_q * c.head_dim, c.n_kv * c.head_dim
        delta = None                                # residual not yet added to h
        for i in range(c.layers):
            p = f"model.layers.{i}."
            if delta is None:
                y = L[p + "self_attn.qkv_proj"].xform(h, None, None, nat.XF_RMS)
            else:
                h2 = torch.empty_like(h)
                y = L[p + "self_attn.qkv_proj"].xform(h, delta, h2, nat.XF_ADD_RMS)
                h = h2
            att = self.glue.attend_rope1(y[:, :nq], y[:, nq:nq + nk], y[:, nq + nk:], self.cos,
                                         self.sin, pos_dev, self.cache[i, 0], self.cache[i, 1])
            o = L[p + "self_attn.o_proj"](att)
            h2 = torch.empty_like(h)
            glu = getattr(L[p + "mlp.gate_up_proj"], "xform_glu", None)
            if glu is not None:                     # SiLU product in the gate/up epilogue
                a = glu(h, o, h2, nat.XF_ADD_RMS)
                h = h2
                delta = L[p + "mlp.down_proj"](a)
                continue
            gu = L[p + "mlp.gate_up_proj"].xform(h, o, h2, nat.XF_ADD_RMS)
            h = h2
            delta = L[p + "mlp.down_proj"].xform(gu[:, :c.inter], gu[:, c.inter:], None,
                                                 nat.XF_SILU)
        head = L["lm_head"]
        mode = nat.XF_RMS if delta is None else nat.XF_ADD_RMS
        if pick is not None and callable(getattr(head, "xform_argmax", None)):
            head.xform_argmax(h, delta, mode, *pick)
            return None
        return head.xform(h, delta, None, mode).reshape(-1)

    @torch.no_grad()
    def generate_graph(self, prompt: List[int], n_new: int, timing: Optional[dict] = None):
        """generate() with the decode steps captured once as a HIP graph and
        replayed (no host round trip per token).  timing, if given, receives
        decode_s (wall time of the n_new - 1 replayed steps, synchronised)."""
        self.reset()
        logits = self.forward(torch.tensor(prompt, dtype=torch.int64))
        plen = len(prompt)
        ids_buf = torch.argmax(logits).reshape(1).to(torch.int32)
        toks = torch.zeros(n_new, dtype=torch.int64, device=self.device)
        toks[0] = ids_buf[0]
        pos_buf = torch.tensor([plen], dtype=torch.int64, device=self.device)
        first = plen - 1                      # toks[k] holds the token sampled at pos plen-1+k
        if n_new > 1:
            snap = (self.cache.clone(), ids_buf.clone(), pos_buf.clone())
            s = torch.cuda.Stream(self.device)
            s.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(s):
                self._graph_step(ids_buf, pos_buf, toks, first)   # warm-up (eager, then undone)
            torch.cuda.current_stream(self.device).wait_stream(s)
            self.cache.copy_(snap[0]); ids_buf.copy_(snap[1]); pos_buf.copy_(snap[2])
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._graph_step(ids_buf, pos_buf, toks, first)
            torch.cuda.synchronize(self.device)
            import time
            t0 = time.perf_counter()
            for _ in range(n_new - 1):
                graph.replay()
            torch.cuda.synchronize(self.device)
            if timing is not None:
                timing["decode_s"] = time.perf_counter() - t0
                timing["decode_steps"] = n_new - 1
        self.pos = plen + n_new - 1
        return [int(t) for t in toks.cpu()]

    # ---- public API ----------------------------------------------------------
    def reset(self):
        self.pos = 0

    @torch.no_grad()
    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        """Run ids [T] at the next positions; return the last position's
        logits [vocab] (fp32)."""
        T = int(ids.numel())
        if self.pos + T > self.max_len:
            raise ValueError(f"sequence of {self.pos + T} exceeds max_len {self.max_len}")
        pos = torch.arange(self.pos, self.pos + T, device=self.device)
        pos_dev = pos[:1].contiguous()
        h = self.embed(ids.to(self.device)).reshape(T, self.cfg.hidden).to(torch.float32)
        if T == 1 and self.fused:
            logits = self._forward1_fused(h, pos_dev)
            self.pos += 1
            return logits
        x = self.glue.add_rms(h, None)
        for i in range(self.cfg.layers):
            x = self._layer(i, h, x, pos, pos_dev, self.pos + T)
        self.pos += T
        return self.linears["lm_head"](x[-1:]).reshape(-1)

    @torch.no_grad()
    def generate(self, prompt: List[int], n_new: int, return_logits: bool = False):
        """Greedy: prompt prefill, then n_new tokens (EOS ignored)."""
        self.reset()
        logits = self.forward(torch.tensor(prompt, dtype=torch.int64))
        out, first = [], logits.clone() if return_logits else None
        for _ in range(n_new):
            tok = int(torch.argmax(logits))
            out.append(tok)
            if len(out) == n_new:
                break
            logits = self.forward(torch.tensor([tok], dtype=torch.int64))
        return (out, first) if return_logits else out


# ---- builders ------------------------------------------------------------------

def from_compressed(cfg: DecoderConfig, comp: Dict[str, dict], device="cuda",
                    max_len: int = 512) -> Qwen3Decoder:
    """Decoder over reference-format data dicts (as produced by the
    compressor; see synthetic.compress_model_cpu).  Fixed-width tensors use
    GPUAcceleratedLinear/Embedding, Huffman ones HuffmanCodebookLinear/
    Embedding, exactly as AdaptiveCodebookLinear.from_compressed would."""
    from gpu_accelerated_functions import GPUAcceleratedEmbedding, GPUAcceleratedLinear
    from gpu_huffman_functions import HuffmanCodebookEmbedding, HuffmanCodebookLinear
    dev = torch.device(device)

    def make(name, d, emb=False):
        cb = torch.from_numpy(np.asarray(d["codebook"], np.float32)).to(dev)
        shape, bits = tuple(d["shape"]), int(d["bits"])
        if d.get("encoding") == "huffman":
            cls = HuffmanCodebookEmbedding if emb else HuffmanCodebookLinear
            kw = {k: d[k] for k in ("huff_row_bit_starts", "huff_chunk_offsets", "huff_sub_lens")
                  if k in d}
            return cls(name, d["huff_stream"], d["huff_lengths"], int(np.asarray(d["huff_n"])[0]),
                       cb, shape, bits, **kw)
        cls = GPUAcceleratedEmbedding if emb else GPUAcceleratedLinear
        return cls(name, d["indices"], cb, shape, bits)

    linears = {n: make(n, comp[n]) for n, _, _ in cfg.linear_shapes()}
    embed = make("model.embed_tokens", comp["model.embed_tokens"], emb=True)
    return Qwen3Decoder(cfg, linears, embed, dev, max_len)


def from_synthetic(cfg: DecoderConfig, tensors: Dict[str, object], device="cuda",
                   max_len: int = 512, stack: bool = True, fuse_glue: bool = True,
                   split: bool = True) -> Qwen3Decoder:
    """Decoder over device-resident tensors (device_formats.FixedTensor /
    HuffTensor / SplitTensor: built on the GPU for the 9B-shape bench, or
    loaded from a device image by cbq_image.load_image); calls the C ABI
    directly on torch's current stream.  With stack, each layer's q/k/v and
    gate/up run as one GEMV launch each instead of three / two: fixed-width
    rows are stacked into one matrix, Huffman matrices (one code each) share
    a grouped launch.  With split, every Huffman linear whose shape and
    codebook allow it is re-encoded into the split format (built from its
    decoded stream) and keeps only that format: closures hold the split
    format alone, so the caller may drop the HuffTensors' streams.  Others
    keep their stream.  SplitTensors run in the split format whatever
    `split` says.  model.linear_bytes maps each launched matrix to its
    device bytes."""
    import ctypes
    import cbq_native as nat
    import synthetic
    from gpu_huffman_functions import (SymbolDecoder, build_split, huffman_prefill,
                                       split_bytes, split_eligible, split_inverse,
                                       split_prefill, stack_split)
    lib = nat.load()
    dev = torch.device(device)
    resident: Dict[str, int] = {}               # device bytes of each matrix's format
    # (max, index) pairs of the lm_head's fused greedy pick, allocated before
    # any graph capture
    argmax_ws = torch.empty(nat.ARGMAX_WORKSPACE, dtype=torch.uint8, device=dev)

    def sym_of(t):
        """Symbol-payload decode tables of a stream (for the split build and
        the stream path's batched tokens)."""
        return SymbolDecoder(t.words, t.chunk_off, t.sub_len, t.lengths, dev)

    def cb_of(t):
        return t.codebook if isinstance(t, synthetic.SplitTensor) else t.tables["codebook"]

    def huff_split(t):
        """The split format of a Huffman tensor, or None when it does not
        apply (then the stream stays the matrix's format).  A SplitTensor
        (loaded already in that format) is used as it is."""
        if isinstance(t, synthetic.SplitTensor):
            resident[t.name] = t.nbytes
            return t.split
        M, K = t.shape
        if not split or not split_eligible(M, K):
            return None
        idx = sym_of(t).indices(M * K)
        sp = build_split(idx, t.tables["codebook"].cpu().numpy(), dev)
        del idx
        if sp is not None:
            resident[t.name] = split_bytes(sp[0])
        return sp

    def split_fns(sps, Ms, K):
        """(one-token GEMV, xform) over split-format matrices sharing x."""
        n = len(sps)
        mats = (ctypes.POINTER(nat.SplitMatrix) * n)(*[ctypes.pointer(sp[1]) for sp in sps])
        m_arr = (ctypes.c_int * n)(*Ms)
        # output pointers: one array, refilled per call (the entry point reads
        # it on the host before it returns)
        o_arr = (ctypes.c_void_p * n)()
        o_off = [4 * sum(Ms[:i]) for i in range(n)]

        def xform(x0, x1, h_out, mode, keep=(sps, mats, m_arr)):
            out = torch.empty(1, sum(Ms), device=dev)
            base = out.data_ptr()
            for i in range(n):
                o_arr[i] = base + o_off[i]
            nat.check(lib.cbq_split_linear_f32(
                x0.data_ptr(), None if x1 is None else x1.data_ptr(),
                None if h_out is None else h_out.data_ptr(), mode, cfg.eps, n, mats,
                o_arr, m_arr, K, nat.stream_ptr(dev)),
                "cbq_split_linear_f32")
            return out

        def one(x):
            return xform(x.reshape(1, K).contiguous(), None, None, 0)
        return one, xform

    def fixed_linear(t):
        M, K = t.shape

        def f(x):
            x = x.reshape(-1, K).contiguous()
            T = x.shape[0]
            out = torch.empty(T, M, device=dev)
            # a prompt (T >= 64) may split K: fp32 partials in a torch workspace
            nws = int(lib.cbq_linear_f32_workspace(T, M, K)) if T >= 64 else 0
            ws = torch.empty(max(1, nws // 4), device=dev) if nws else None
            nat.check(lib.cbq_linear_f32_ws(x.data_ptr(), t.packed.data_ptr(),
                                            t.codebook.data_ptr(), out.data_ptr(), T, M, K,
                                            t.codebook.numel(), t.bits,
                                            None if ws is None else ws.data_ptr(), nws,
                                            nat.stream_ptr(dev)), "cbq_linear_f32_ws")
            return out

        def xform(x0, x1, h_out, mode):
            """One token, x = transform(x0, x1) staged by the GEMV."""
            out = torch.empty(1, M, device=dev)
            nat.check(lib.cbq_linear_xform_f32(
                x0.data_ptr(), None if x1 is None else x1.data_ptr(),
                None if h_out is None else h_out.data_ptr(), mode, cfg.eps, t.packed.data_ptr(),
                t.codebook.data_ptr(), out.data_ptr(), M, K, t.codebook.numel(), t.bits,
                nat.stream_ptr(dev)), "cbq_linear_xform_f32")
            return out

        def xform_argmax(x0, x1, mode, ids32, toks, pos, first, out=None):
            """One token, then the greedy pick in the GEMV's epilogue."""
            nat.check(lib.cbq_linear_xform_argmax_f32(
                x0.data_ptr(), None if x1 is None else x1.data_ptr(), None, mode, cfg.eps,
                t.packed.data_ptr(), t.codebook.data_ptr(), nat.ptr(out), M, K,
                t.codebook.numel(), t.bits, argmax_ws.data_ptr(), argmax_ws.numel(),
                ids32.data_ptr(), toks.data_ptr(), pos.data_ptr(), first, toks.numel(),
                nat.stream_ptr(dev)), "cbq_linear_xform_argmax_f32")
        def xform_glu(x0, x1, h_out, mode):
            """One token over a row-stacked [gate; up] matrix: silu(gate . x) *
            (up . x), x = transform(x0, x1), in one launch."""
            out = torch.empty(1, M // 2, device=dev)
            nat.check(lib.cbq_linear_xform_glu_f32(
                x0.data_ptr(), None if x1 is None else x1.data_ptr(),
                None if h_out is None else h_out.data_ptr(), mode, cfg.eps, t.packed.data_ptr(),
                t.codebook.data_ptr(), out.data_ptr(), M // 2, K, t.codebook.numel(), t.bits,
                nat.stream_ptr(dev)), "cbq_linear_xform_glu_f32")
            return out
        f.xform = xform
        f.xform_argmax = xform_argmax
        if M % 2 == 0:
            f.xform_glu = xform_glu
        return f

    def huff_desc(t):
        tb = t.tables
        return nat.HuffStream(words=t.words.data_ptr(), n_words=t.words.numel(),
                              chunk_off=t.chunk_off.data_ptr(), sub_len=t.sub_len.data_ptr(),
                              lut1=tb["lut1"].data_ptr(), lut2=tb["lut2"].data_ptr(),
                              n_lut2=tb["lut2"].numel(), canon=tb["canon"].data_ptr(),
                              canon_pay=tb["pay"].data_ptr(), value_cb=None,
                              C=tb["codebook"].numel(), stage_words=tb["stage_words"])

    inv_tables: Dict[bytes, torch.Tensor] = {}

    def inv_of(cbt):
        """bf16 value -> index table of a codebook (128 KiB), one per
        distinct codebook: the tensors of a category share it."""
        cb_np = cbt.cpu().numpy()
        key = cb_np.tobytes()
        if key not in inv_tables:
            inv_tables[key] = split_inverse(cb_np, dev)
        return inv_tables[key]

    def split_linear(sp, M, K, cbt):
        """A split-format matrix: one token on the split GEMV, batched tokens
        through its transient fixed-width stream.  Captures only the split
        format, so the tensor's stream can be freed."""
        inv = inv_of(cbt)
        one, sxform = split_fns([sp], [M], K)

        def f(x):
            x = x.reshape(-1, K).contiguous()
            if x.shape[0] == 1:
                return one(x)
            return split_prefill(sp, inv, x, M, K, cbt)

        def xform_argmax(x0, x1, mode, ids32, toks, pos, first, out=None, keep=sp):
            """One token, then the greedy pick in the GEMV's epilogue."""
            nat.check(lib.cbq_split_linear_argmax_f32(
                x0.data_ptr(), None if x1 is None else x1.data_ptr(), None, mode, cfg.eps,
                ctypes.byref(sp[1]), nat.ptr(out), M, K, argmax_ws.data_ptr(), argmax_ws.numel(),
                ids32.data_ptr(), toks.data_ptr(), pos.data_ptr(), first, toks.numel(),
                nat.stream_ptr(dev)), "cbq_split_linear_argmax_f32")
        f.xform = sxform
        f.xform_argmax = xform_argmax
        f.split = sp
        return f

    def huff_linear(t):
        """One Huffman matrix: the split format where it applies, else the
        stream (every token count on the fused stream kernels; batched
        tokens >= 64 through a transient fixed-width stream)."""
        M, K = t.shape
        cbt = cb_of(t)
        sp = huff_split(t)
        if sp is not None:
            return split_linear(sp, M, K, cbt)
        resident[t.name] = t.nbytes
        desc = huff_desc(t)

        def f(x, desc=desc, keep=(t.words, t.chunk_off, t.sub_len, t.tables, t.lengths)):
            x = x.reshape(-1, K).contiguous()
            T = x.shape[0]
            if T >= 64:
                return huffman_prefill(SymbolDecoder(keep[0], keep[1], keep[2], keep[4], dev),
                                       x, M, K, cbt)
            out = torch.empty(T, M, device=dev)
            for t0 in range(0, T, 16):
                tt = min(16, T - t0)
                nat.check(lib.cbq_huff_linear_f32(x.data_ptr() + t0 * K * 4, ctypes.byref(desc),
                                                  out.data_ptr() + t0 * M * 4, tt, M, K,
                                                  nat.stream_ptr(dev)), "cbq_huff_linear_f32")
            return out
        f.desc = desc
        return f

    def huff_group(ts, name):
        """One grouped split-GEMV launch for matrices sharing x (q/k/v,
        gate/up), each with its own code; None when a part has no split
        format (the parts then run one by one).  gate/up of one codebook with
        K % 4096 == 0 are re-coded as one stacked matrix under a shared table
        (the only resident copy; the parts point into it), which adds the
        one-launch gate/up with the SiLU product in its epilogue
        (`xform_glu`)."""
        K = ts[0].shape[1]
        presplit = all(isinstance(t, synthetic.SplitTensor) for t in ts)
        if any(t.shape[1] != K for t in ts) or not (split or presplit):
            return None
        sps = [huff_split(t) for t in ts]
        if not all(sp is not None for sp in sps):
            return None
        Ms = [t.shape[0] for t in ts]
        glu = None
        cbs = [cb_of(t).cpu().numpy() for t in ts]
        if (name.endswith("gate_up_proj") and len(ts) == 2 and Ms[0] == Ms[1]
                and K % 4096 == 0 and np.array_equal(cbs[0], cbs[1])):
            st = stack_split(sps, cbs[0], Ms, K, dev)
            if st is not None:
                keep, sdesc, parts = st
                sps = [(keep, parts[0]), (keep, parts[1])]
                for t in ts:
                    resident.pop(t.name, None)
                resident[name] = split_bytes(keep)
                M = Ms[0]

                def glu(x0, x1, h_out, mode, keep=(keep, sdesc)):
                    """silu(gate . x) * (up . x), x = transform(x0, x1), one launch."""
                    out = torch.empty(1, M, device=dev)
                    nat.check(lib.cbq_split_linear_glu_f32(
                        x0.data_ptr(), None if x1 is None else x1.data_ptr(),
                        None if h_out is None else h_out.data_ptr(), mode, cfg.eps,
                        ctypes.byref(sdesc), out.data_ptr(), M, K, nat.stream_ptr(dev)),
                        "cbq_split_linear_glu_f32")
                    return out
        one, sxform = split_fns(sps, Ms, K)
        singles = [split_linear(sp, t.shape[0], K, cb_of(t))   # batched tokens
                   for t, sp in zip(ts, sps)]

        def g(x):
            x = x.reshape(-1, K).contiguous()
            if x.shape[0] > 1:
                return torch.cat([h(x) for h in singles], dim=1)
            return one(x)
        g.xform = sxform
        g.name = name
        if glu is not None:
            g.xform_glu = glu
        return g

    def embed_fn(t):
        V, H = t.shape
        if isinstance(t, synthetic.HuffTensor):
            desc = huff_desc(t)

            # desc holds raw device pointers: keep the tensors they point at
            def e(ids, desc=desc, keep=(t.words, t.chunk_off, t.sub_len, t.tables)):
                ids = ids.reshape(-1).to(torch.int32)
                out = torch.empty(ids.numel(), H, device=dev)
                nat.check(lib.cbq_huff_embedding_f32(ids.data_ptr(), ctypes.byref(desc),
                                                     out.data_ptr(), ids.numel(), V, H,
                                                     nat.stream_ptr(dev)), "cbq_huff_embedding_f32")
                return out
            return e

        def e2(ids):
            ids = ids.reshape(-1).to(torch.int32)
            out = torch.empty(ids.numel(), H, device=dev)
            nat.check(lib.cbq_embedding_f32(ids.data_ptr(), t.packed.data_ptr(),
                                            t.codebook.data_ptr(), out.data_ptr(), ids.numel(),
                                            V, H, t.codebook.numel(), t.bits, nat.stream_ptr(dev)),
                      "cbq_embedding_f32")
            return out
        return e2

    linears = {}
    for i in range(cfg.layers):
        p = f"model.layers.{i}."
        for fused, parts in (("self_attn.qkv_proj", ("self_attn.q_proj", "self_attn.k_proj",
                                                     "self_attn.v_proj")),
                             ("mlp.gate_up_proj", ("mlp.gate_proj", "mlp.up_proj"))):
            ts = [tensors[p + n] for n in parts]
            if not stack:
                continue
            if all(isinstance(t, synthetic.FixedTensor) for t in ts):
                st = synthetic.stack_fixed(ts, p + fused)
                if st is not None:
                    linears[p + fused] = fixed_linear(st)
                    resident[p + fused] = st.nbytes
            elif all(isinstance(t, (synthetic.HuffTensor, synthetic.SplitTensor)) for t in ts):
                g = huff_group(ts, p + fused)
                if g is not None:
                    linears[p + fused] = g
    for n, _, _ in cfg.linear_shapes():
        t = tensors[n]
        stem, _, leaf = n.rpartition(".")
        fused = {"q_proj": "qkv_proj", "k_proj": "qkv_proj", "v_proj": "qkv_proj",
                 "gate_proj": "gate_up_proj", "up_proj": "gate_up_proj"}.get(leaf)
        if fused is not None and f"{stem}.{fused}" in linears:
            continue
        if isinstance(t, (synthetic.HuffTensor, synthetic.SplitTensor)):
            linears[n] = huff_linear(t)
        else:
            linears[n] = fixed_linear(t)
            resident[n] = t.nbytes
    emb = tensors["model.embed_tokens"]
    model = Qwen3Decoder(cfg, linears, embed_fn(emb), dev, max_len, fuse_glue=fuse_glue)
    # device bytes of every linear's format (what a decode step streams) and
    # of the embedding (read one row per token)
    model.linear_bytes = dict(resident)
    model.embed_bytes = int(emb.nbytes)
    return model
