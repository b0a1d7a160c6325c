"""The reference's on-disk compression cache: read, write, and swap modules.

Layout of a cache directory (src/compressor.py:199-243, 330-361;
src/adaptive_compressor.py:1225-1315; src/name_resolver.py:114-118):

    <cache>/codebooks/<type>_codebook[_<suffix>].npy   global codebooks
    <cache>/tensors/<safe name>.npz                   one tensor per file
    <cache>/tensors/<safe name>.idx                   optional flat packed
                                                      indices (mmap)

where <safe name> is the parameter name with '.' and '/' replaced by '_'.
Each .npz holds 'name', 'mode', 'shape' and the mode's keys; one-element
metadata (bits, codebook_type, encoding, scale, ...) is stored as a length-1
array, as the reference writes it.  Everything is read with
allow_pickle=False: string fields are numpy unicode arrays, never objects.

This package's Huffman encoder adds 'huff_chunk_offsets' and
'huff_sub_lens' (the chunk and sub-block bit index).  They are written
beside the reference's keys and read back when present; a reader that does
not know them ignores them, and a reference-written file without them is
indexed again at load (huffman_codebook.index_stream).
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path
from typing import Dict, Iterable, Optional, Tuple

import numpy as np
import torch
import torch.nn as nn

HUFF_TABLE_KEYS = ("huff_row_bit_starts", "huff_lut_sym", "huff_lut_len",
                   "huff_sl_first_code", "huff_sl_base_offset", "huff_sl_sym")
HUFF_INDEX_KEYS = ("huff_chunk_offsets", "huff_sub_lens")


def safe_name(name: str) -> str:
    """File stem of a tensor (src/name_resolver.py:117, src/compressor.py:376)."""
    return name.replace(".", "_").replace("/", "_")


def _one(v):
    return np.array([v])


def _scalar(arr, cast):
    return cast(np.asarray(arr).reshape(-1)[0])


def save_cached_tensor(npz_file, name: str, data: dict) -> None:
    """Write one compressed tensor in the reference's .npz schema
    (src/compressor.py:199-243)."""
    mode = data["mode"]
    out = {"name": np.array(name), "mode": np.array(mode),
           "shape": np.asarray(tuple(int(s) for s in data["shape"]), np.int64)}
    if mode == "exact":
        out["data"] = np.asarray(data["data"])
    elif mode == "codebook":
        out["type"] = _one(data["type"])
        out["indices"] = np.asarray(data["indices"])
    elif mode == "direct_codebook":
        out["codebook_type"] = _one(data.get("codebook_type", "mlp_ffn"))
        out["bits"] = _one(int(data.get("bits", 8)))
        if data.get("codebook") is not None:
            out["codebook"] = np.asarray(data["codebook"])
        if data.get("encoding") == "huffman":
            out["encoding"] = _one("huffman")
            for k in ("huff_lengths", "huff_stream", "huff_n"):
                out[k] = np.asarray(data[k])
            for k in HUFF_TABLE_KEYS + HUFF_INDEX_KEYS:
                if data.get(k) is not None:
                    out[k] = np.asarray(data[k])
        else:
            out["indices"] = np.asarray(data["indices"])
    elif mode == "linear_quant":
        out["indices"] = np.asarray(data["indices"])
        out["scale"] = _one(float(data["scale"]))
        out["v_min"] = _one(float(data["v_min"]))
        out["bits"] = _one(int(data.get("bits", 8)))
    elif mode == "q8_packed_7bit":
        out["packed"] = np.asarray(data["packed"])
        out["original_len"] = _one(int(data["original_len"]))
        out["scale"] = _one(float(data["scale"]))
        out["offset"] = _one(float(data["offset"]))
        out["unique_q8"] = np.asarray(data["unique_q8"])
        out["codebook_values"] = np.asarray(data["codebook_values"])
    else:
        raise ValueError(f"{name}: unknown mode {mode!r}")
    np.savez_compressed(npz_file, **out)


def load_cached_tensor(npz_file) -> Tuple[str, dict]:
    """Read one compressed tensor (src/compressor.py:144-196).  Returns
    (name, data) with the reference's keys and scalar types."""
    with np.load(npz_file, allow_pickle=False) as f:
        keys = set(f.files)
        mode = str(f["mode"])
        name = str(f["name"])
        d = {"mode": mode, "name": name, "shape": f["shape"]}
        if mode == "exact":
            d["data"] = f["data"]
        elif mode == "codebook":
            d["type"] = _scalar(f["type"], str)
            d["indices"] = f["indices"]
        elif mode == "direct_codebook":
            d["codebook_type"] = _scalar(f["codebook_type"], str)
            d["bits"] = _scalar(f["bits"], int) if "bits" in keys else 8
            if "codebook" in keys:
                d["codebook"] = f["codebook"]
            if "encoding" in keys and _scalar(f["encoding"], str) == "huffman":
                d["encoding"] = "huffman"
                for k in ("huff_lengths", "huff_stream", "huff_n"):
                    d[k] = f[k]
                for k in HUFF_TABLE_KEYS + HUFF_INDEX_KEYS:
                    if k in keys:
                        d[k] = f[k]
            else:
                d["indices"] = f["indices"]
        elif mode == "q8_packed_7bit":
            d["packed"] = f["packed"]
            d["original_len"] = _scalar(f["original_len"], int)
            d["scale"] = _scalar(f["scale"], float)
            d["offset"] = _scalar(f["offset"], float)
            d["unique_q8"] = f["unique_q8"]
            d["codebook_values"] = f["codebook_values"]
        elif mode == "linear_quant":
            d["indices"] = f["indices"]
            d["scale"] = _scalar(f["scale"], float)
            d["v_min"] = _scalar(f["v_min"], float)
            d["bits"] = _scalar(f["bits"], int) if "bits" in keys else 8
        elif mode == "q8_codebook":
            d["indices"] = f["indices"]
            d["scale"] = _scalar(f["scale"], float)
            d["offset"] = _scalar(f["offset"], float)
            if "codebook" in keys:
                d["codebook"] = f["codebook"]
        else:
            raise ValueError(f"{npz_file}: unknown mode {mode!r}")
    return name, d


def codebook_type_of(npy_name: str) -> str:
    """Codebook type from a codebooks/ file name: 'mlp_ffn_codebook.npy' and
    'attention_codebook_e8m7.npy' give 'mlp_ffn' and 'attention'
    (src/compressor.py:335-343)."""
    if "_codebook_" in npy_name:
        return npy_name.split("_codebook_")[0]
    if npy_name.endswith("_codebook.npy"):
        return npy_name[:-len("_codebook.npy")]
    return npy_name[:-4] if npy_name.endswith(".npy") else npy_name


def save_global_codebook(cache_dir, ttype: str, codebook) -> Path:
    d = Path(cache_dir) / "codebooks"
    d.mkdir(parents=True, exist_ok=True)
    p = d / f"{ttype}_codebook.npy"
    np.save(p, np.asarray(codebook), allow_pickle=False)
    return p


def load_global_codebooks(cache_dir) -> Dict[str, torch.Tensor]:
    """Every codebooks/*.npy as a bf16 tensor keyed by codebook type
    (src/adaptive_compressor.py:1225-1249)."""
    out = {}
    d = Path(cache_dir) / "codebooks"
    if not d.is_dir():
        return out
    for p in sorted(d.glob("*.npy")):
        cb = np.load(p, allow_pickle=False)
        out[codebook_type_of(p.name)] = torch.from_numpy(
            np.ascontiguousarray(cb, np.float32)).to(torch.bfloat16)
    return out


def save_cache(cache_dir, tensors: Dict[str, dict],
               global_codebooks: Optional[Dict[str, np.ndarray]] = None) -> None:
    t = Path(cache_dir) / "tensors"
    t.mkdir(parents=True, exist_ok=True)
    for name, data in tensors.items():
        save_cached_tensor(t / f"{safe_name(name)}.npz", name, data)
    for ttype, cb in (global_codebooks or {}).items():
        save_global_codebook(cache_dir, ttype, cb)


def load_cache(cache_dir, threads: int = 8) -> Dict[str, dict]:
    """Every tensors/*.npz, read on a thread pool as the reference preloads
    them (src/compressor.py:347-361); keyed by the stored parameter name."""
    files = sorted((Path(cache_dir) / "tensors").glob("*.npz"))
    if not files:
        return {}
    with ThreadPoolExecutor(max_workers=max(1, min(threads, len(files)))) as ex:
        return dict(ex.map(load_cached_tensor, files))


def export_flat_idx(model_dir, tensors_subdir: str = "codebook/tensors",
                    verbose: bool = False) -> int:
    """Write <stem>.idx (the raw packed index bytes) beside every .npz that has
    an 'indices' key and no .idx yet; returns the number written
    (src/adaptive_compressor.py:1255-1315)."""
    tdir = Path(model_dir) / tensors_subdir
    if not tdir.is_dir():
        raise FileNotFoundError(f"tensors directory not found: {tdir}")
    files = sorted(tdir.glob("*.npz"))
    if not files:
        raise FileNotFoundError(f"no .npz files in {tdir}")
    written = 0
    for p in files:
        q = p.with_suffix(".idx")
        if q.exists():
            continue
        with np.load(p, allow_pickle=False) as f:
            if "indices" not in f.files:
                continue
            packed = f["indices"]
        np.asarray(packed).astype(np.uint8, copy=False).tofile(q)
        written += 1
        if verbose:
            print(f"{p.stem}: {q.stat().st_size} bytes -> {q.name}")
    return written


def idx_file_for(tensor_name: str, model_path, use_mmap: bool) -> Optional[Path]:
    """.idx path of a tensor under <model>/codebook/tensors, or None without
    mmap (src/name_resolver.py:114-118)."""
    if not use_mmap:
        return None
    return Path(model_path) / "codebook" / "tensors" / f"{safe_name(tensor_name)}.idx"


def replace_modules(model: nn.Module, cache: Dict[str, dict], global_codebooks: dict,
                    use_gpu: bool = True, use_mmap: bool = False, model_path=None,
                    resolve=lambda n: n) -> int:
    """Swap every nn.Linear / nn.Embedding whose cached tensor is
    'direct_codebook' for AdaptiveCodebookLinear / AdaptiveCodebookEmbedding
    built by from_compressed (src/model_loader.py:205-277).  An lm_head with
    no tensor of its own uses model.embed_tokens' (tied weights); a Linear's
    bias is kept; an embedding class named '*Scaled*' gets
    embed_scale = sqrt(embedding_dim).  `resolve` maps a parameter name to
    its cache name.  Returns the number of modules replaced."""
    from compressed_modules import AdaptiveCodebookEmbedding, AdaptiveCodebookLinear

    replaced = 0

    def walk(mod: nn.Module, prefix: str):
        nonlocal replaced
        for attr, child in list(mod.named_children()):
            full = f"{prefix}.{attr}" if prefix else attr
            wname = f"{full}.weight"
            if isinstance(child, (nn.Linear, nn.Embedding)):
                key = resolve(wname)
                data = cache.get(key)
                if data is None and isinstance(child, nn.Linear) and "lm_head" in full:
                    key = resolve("model.embed_tokens.weight")
                    data = cache.get(key)
                if data is not None and data.get("mode") == "direct_codebook":
                    idx = idx_file_for(key, model_path, use_mmap) if model_path else None
                    if isinstance(child, nn.Linear):
                        new = AdaptiveCodebookLinear.from_compressed(
                            wname, data, global_codebooks, use_gpu=use_gpu,
                            use_mmap=use_mmap, idx_file=idx)
                        if child.bias is not None:
                            new.bias = child.bias.data.clone().detach()
                    else:
                        new = AdaptiveCodebookEmbedding.from_compressed(
                            wname, data, global_codebooks, use_gpu=use_gpu,
                            use_mmap=use_mmap, idx_file=idx)
                        if "scaled" in type(child).__name__.lower():
                            dim = getattr(child, "embedding_dim", None)
                            if dim and dim > 1:
                                new.embed_scale = float(dim ** 0.5)
                    setattr(mod, attr, new)
                    replaced += 1
                    continue
            walk(child, full)

    walk(model, "")
    return replaced


def replace_modules_from_image(model: nn.Module, image_path, device="cuda", threads: int = 8,
                               resolve=lambda n: n, load_dense: bool = True):
    """replace_modules over a device image (cbq_image): every nn.Linear /
    nn.Embedding whose weight the image holds becomes an
    AdaptiveCodebookLinear / AdaptiveCodebookEmbedding bound to the loaded
    device tensors (no host decode, no re-encoding); an lm_head without its
    own tensor uses model.embed_tokens' (tied weights); a Linear's bias is
    kept.  With load_dense, every other image tensor whose name is a
    parameter of the model (norm weights and the like) replaces that
    parameter's data.  Returns (modules replaced, load statistics)."""
    import cbq_image
    from compressed_modules import AdaptiveCodebookEmbedding, AdaptiveCodebookLinear

    tensors, _, stats = cbq_image.load_image(image_path, device, threads=threads)
    replaced = 0

    def walk(mod: nn.Module, prefix: str):
        nonlocal replaced
        for attr, child in list(mod.named_children()):
            full = f"{prefix}.{attr}" if prefix else attr
            wname = f"{full}.weight"
            if isinstance(child, (nn.Linear, nn.Embedding)):
                t = tensors.get(resolve(wname))
                if t is None and isinstance(child, nn.Linear) and "lm_head" in full:
                    t = tensors.get(resolve("model.embed_tokens.weight"))
                if t is not None and not isinstance(t, torch.Tensor):
                    if isinstance(child, nn.Linear):
                        new = AdaptiveCodebookLinear.from_device(wname, t)
                        if child.bias is not None:
                            new.bias = child.bias.data.clone().detach()
                    else:
                        new = AdaptiveCodebookEmbedding.from_device(wname, t)
                        if "scaled" in type(child).__name__.lower():
                            dim = getattr(child, "embedding_dim", None)
                            if dim and dim > 1:
                                new.embed_scale = float(dim ** 0.5)
                    setattr(mod, attr, new)
                    replaced += 1
                    continue
            walk(child, full)

    walk(model, "")
    if load_dense:
        params = dict(model.named_parameters())
        for name, t in tensors.items():
            p = params.get(resolve(name)) if isinstance(t, torch.Tensor) else None
            if p is not None and tuple(p.shape) == tuple(t.shape):
                p.data = t
    return replaced, stats
