"""A cache directory written in the reference's on-disk schema, read back and
swapped into a small model (fixed-width, Huffman, global codebook, tied
lm_head, flat .idx files): the swapped modules equal modules built from the
in-memory data bit for bit, and dense fp32 products to rel-L2 <= 1e-5."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import bitpack
import cache_io
import codebook_builder as cbb
import huffman_codebook as hc
from compressed_modules import AdaptiveCodebookEmbedding, AdaptiveCodebookLinear

pytestmark = pytest.mark.gpu


class _Model(nn.Module):
    def __init__(self, V=512, H=256, M=384):
        super().__init__()
        self.model = nn.Module()
        self.model.embed_tokens = nn.Embedding(V, H)
        self.model.proj = nn.Linear(H, M)
        self.model.hproj = nn.Linear(H, H, bias=False)
        self.lm_head = nn.Linear(H, V, bias=False)


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def _data(tmp_path):
    rng = np.random.default_rng(7)
    V, H, M = 512, 256, 384
    we = cbb.bf16_round(rng.standard_normal((V, H)) * 0.02)
    wp = cbb.bf16_round(rng.standard_normal((M, H)) * 0.02)
    wh = cbb.bf16_round(rng.standard_normal((H, H)) * 0.02)
    cb_e, idx_e = cbb.frequency_sorted_codebook(we)
    emb = {"mode": "direct_codebook", "shape": (V, H), "bits": cbb.bits_for(len(cb_e)),
           "codebook_type": "embedding",
           "indices": bitpack.pack_any_bits(idx_e, cbb.bits_for(len(cb_e)))}
    proj = cbb.compress_fixed(wp)
    proj.pop("_raw_indices")
    proj["codebook_type"] = "attention"
    cb_h, idx_h = cbb.frequency_sorted_codebook(wh)
    hp = {"mode": "direct_codebook", "shape": (H, H), "bits": cbb.bits_for(len(cb_h)),
          "codebook": cb_h.astype(np.float32), "codebook_type": "attention", "encoding": "huffman"}
    hp.update(hc.huffman_encode_indices(idx_h, shape=(H, H)))
    tensors = {"model.embed_tokens.weight": emb, "model.proj.weight": proj,
               "model.hproj.weight": hp}
    root = tmp_path / "model"
    cache_io.save_cache(root / "codebook", tensors, {"embedding": cb_e.astype(np.float32)})
    return root, tensors, (we, wp, wh)


def test_cache_dir_to_modules(cuda, tmp_path):
    root, tensors, (we, wp, wh) = _data(tmp_path)
    cache = cache_io.load_cache(root / "codebook")
    gcb = cache_io.load_global_codebooks(root / "codebook")
    m = _Model()
    bias = m.model.proj.bias.detach().clone()
    assert cache_io.replace_modules(m, cache, gcb, use_gpu=True) == 4
    assert isinstance(m.lm_head, AdaptiveCodebookLinear)          # tied to embed_tokens
    assert isinstance(m.model.embed_tokens, AdaptiveCodebookEmbedding)

    x = torch.randn(3, 256, device=cuda)
    ids = torch.tensor([0, 5, 511, 77], device=cuda)
    xd = x.double().cpu()
    for mod, w, b in ((m.model.proj, wp, bias), (m.model.hproj, wh, None), (m.lm_head, we, None)):
        y = mod(x)
        ref = xd @ torch.from_numpy(w).double().t()
        if b is not None:
            ref = ref + b.double()
        assert _rel(y.cpu(), ref) <= 1e-5
    # bit-equal to modules built straight from the in-memory data
    direct = AdaptiveCodebookLinear.from_compressed("model.proj.weight", tensors["model.proj.weight"], {})
    direct.bias = bias
    assert torch.equal(direct(x), m.model.proj(x))
    dh = AdaptiveCodebookLinear.from_compressed("model.hproj.weight", tensors["model.hproj.weight"], {})
    assert torch.equal(dh(x), m.model.hproj(x))
    e = m.model.embed_tokens(ids)
    assert torch.equal(e.float().cpu(), torch.from_numpy(we)[ids.cpu()])


def test_flat_idx_mmap(cuda, tmp_path):
    root, tensors, (we, wp, wh) = _data(tmp_path)
    assert cache_io.export_flat_idx(root) == 2
    cache = cache_io.load_cache(root / "codebook")
    for d in cache.values():
        d.pop("indices", None)          # the packed bytes now come from the .idx file only
    gcb = cache_io.load_global_codebooks(root / "codebook")
    m = _Model()
    m.model.proj.bias = None
    assert cache_io.replace_modules(m, cache, gcb, use_mmap=True, model_path=root) == 4
    x = torch.randn(2, 256, device=cuda)
    direct = AdaptiveCodebookLinear.from_compressed("model.proj.weight", tensors["model.proj.weight"], {})
    assert torch.equal(direct(x), m.model.proj(x))
    ids = torch.tensor([3, 400], device=cuda)
    assert torch.equal(m.model.embed_tokens(ids).float().cpu(), torch.from_numpy(we)[ids.cpu()])
