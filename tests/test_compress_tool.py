"""The checkpoint encoder (cbq_compress) and the device image writer on the
CPU: a small safetensors checkpoint is compressed, the reference-schema
.npz files it writes are read back with cache_io and decoded by the oracle
to the original weights bit for bit, the codebook orders follow the
reference's definitions, the Huffman stream equals the reference-format
encoder's bytes and its chunk index equals the host indexer's, and the
device image's header and sections hold the encoder's arrays."""
import os

import numpy as np
import pytest
import torch

import bitpack
import cache_io
import cbq_compress
import cbq_image
import codebook_builder as cbb
import huffman_codebook as hc
import synthetic

SHAPES = {"model.layers.0.self_attn.q_proj.weight": (64, 128),
          "model.layers.0.mlp.down_proj.weight": (96, 64),
          "model.embed_tokens.weight": (200, 64),
          "model.layers.0.input_layernorm.weight": (64,),
          "tiny.weight": (4, 4)}


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    from safetensors.torch import save_file
    d = tmp_path_factory.mktemp("model")
    ts = {}
    for n, shp in SHAPES.items():
        std = 0.02 if len(shp) == 2 else 0.5
        ts[n] = synthetic.make_bf16(shp, n, std=std, device="cpu")
    # two shards, as checkpoints come
    names = sorted(ts)
    save_file({k: ts[k] for k in names[:2]}, str(d / "model-00001-of-00002.safetensors"))
    save_file({k: ts[k] for k in names[2:]}, str(d / "model-00002-of-00002.safetensors"))
    return d, ts


def _weights(data) -> np.ndarray:
    M, K = (int(s) for s in data["shape"])
    bits = int(data["bits"])
    cb = np.asarray(data["codebook"], np.float32)
    if data.get("encoding") == "huffman":
        return None
    raw = data["indices"]
    if raw.dtype == np.uint16:
        idx = raw.astype(np.int64)
    else:
        idx = bitpack.unpack_any_bits(raw, bits, M * K).astype(np.int64)
    return cb[np.minimum(idx, cb.size - 1)].reshape(M, K)


def _ref_codebook(w_bf16: torch.Tensor, order: str) -> np.ndarray:
    pats = w_bf16.view(torch.int16).numpy().astype(np.int64) & 0xFFFF
    counts = np.bincount(pats.reshape(-1), minlength=65536)
    present = np.nonzero(counts)[0]
    if order == "pattern":
        keep = present                                    # ascending bit pattern
    else:
        keep = present[np.lexsort((present, -counts[present]))]
    return (keep.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("order", ["frequency", "pattern"])
def test_fixed_cache_roundtrip(ckpt, tmp_path, order):
    d, ts = ckpt
    s = cbq_compress.compress_checkpoint(d, tmp_path / "out", order=order, device="cpu",
                                         export_idx=True, log=lambda *a: None)
    assert s["compressed"] == 3 and s["exact"] == 2
    cache = cache_io.load_cache(tmp_path / "out")
    assert set(cache) == set(SHAPES)
    for n, w in ts.items():
        data = cache[n]
        if w.dim() != 2 or w.numel() < 1000:
            assert data["mode"] == "exact"
            raw = np.asarray(data["data"])
            assert raw.dtype == np.uint16
            # the reference's decode of 'exact' (src/adaptive_compressor.py:599-602)
            ref = (raw.astype(np.uint32) << 16).view(np.float32).reshape(tuple(data["shape"]))
            assert np.array_equal(ref, w.float().numpy())
            continue
        assert data["mode"] == "direct_codebook"
        assert data["codebook_type"] == cbb.classify_tensor(n)
        assert np.array_equal(data["codebook"], _ref_codebook(w, order))
        assert int(data["bits"]) == cbb.bits_for(len(data["codebook"]))
        assert np.array_equal(_weights(data), w.float().numpy())
        idx_file = tmp_path / "out" / "tensors" / f"{cache_io.safe_name(n)}.idx"
        assert np.array_equal(np.fromfile(idx_file, np.uint8), data["indices"])


def test_category_codebooks(ckpt, tmp_path):
    d, ts = ckpt
    cbq_compress.compress_checkpoint(d, tmp_path / "out", codebooks="category", device="cpu",
                                     write_image=False, log=lambda *a: None)
    books = cache_io.load_global_codebooks(tmp_path / "out")
    assert set(books) == {"attention", "mlp_ffn", "embedding"}
    cache = cache_io.load_cache(tmp_path / "out")
    for n, w in ts.items():
        if cache[n]["mode"] == "exact":
            continue
        cb = cache[n]["codebook"]
        assert np.array_equal(cb, books[cbb.classify_tensor(n)].float().numpy())
        assert np.array_equal(_weights(cache[n]), w.float().numpy())


def test_huffman_cache_matches_reference_encoder(ckpt, tmp_path, oracle):
    d, ts = ckpt
    s = cbq_compress.compress_checkpoint(d, tmp_path / "out", entropy_code=True, device="cpu",
                                         log=lambda *a: None)
    assert s["huffman"] == 3 and s["split"] == 0           # no split format without a GPU
    cache = cache_io.load_cache(tmp_path / "out")
    for n, w in ts.items():
        data = cache[n]
        if data["mode"] == "exact":
            continue
        M, K = w.shape
        assert data["encoding"] == "huffman"
        cb = data["codebook"]
        lut = np.zeros(65536, np.int64)
        lut[(cb.view(np.uint32) >> 16).astype(np.int64)] = np.arange(cb.size)
        idx = lut[w.view(torch.int16).numpy().astype(np.int64) & 0xFFFF].reshape(-1)
        want = hc.huffman_encode_indices(idx, shape=(M, K), lengths=data["huff_lengths"])
        for k in ("huff_stream", "huff_row_bit_starts", "huff_lut_sym", "huff_lut_len",
                  "huff_sl_first_code", "huff_sl_base_offset", "huff_sl_sym",
                  "huff_chunk_offsets", "huff_sub_lens"):
            assert np.array_equal(np.asarray(data[k]), np.asarray(want[k])), (n, k)
        ch, sub = hc.index_stream(data["huff_stream"], data["huff_lengths"], M, K,
                                  data["huff_row_bit_starts"])
        assert np.array_equal(ch, data["huff_chunk_offsets"])
        assert np.array_equal(sub, data["huff_sub_lens"])
        dec = oracle.huff_decode_indices(data, M, K).reshape(-1)
        assert np.array_equal(dec, idx)
        assert np.array_equal(cb[dec].reshape(M, K), w.float().numpy())


def test_image_header_and_sections(ckpt, tmp_path):
    d, ts = ckpt
    for enc in (False, True):
        out = tmp_path / f"out{int(enc)}"
        cbq_compress.compress_checkpoint(d, out, entropy_code=enc, device="cpu",
                                         write_npz=False, log=lambda *a: None)
        path = out / "device.cbq"
        h = cbq_image.read_header(path)
        size = os.path.getsize(path)
        assert h["data_offset"] % cbq_image.ALIGN == 0
        assert h["data_offset"] + h["payload_bytes"] == size
        kinds = {n: e["kind"] for n, e in h["tensors"].items()}
        for n, w in ts.items():
            if w.dim() != 2 or w.numel() < 1000:
                assert kinds[n] == "dense"
                off, nb, dt = h["tensors"][n]["sections"]["data"]
                raw = np.fromfile(path, np.uint8, nb, offset=h["data_offset"] + off)
                assert dt == "bfloat16"
                assert np.array_equal(raw.view(np.int16), w.view(torch.int16).numpy().reshape(-1))
                continue
            e = h["tensors"][n]
            assert kinds[n] == ("stream" if enc else "fixed")
            cbs = h["codebooks"][e["codebook"]]
            cb = np.fromfile(path, np.float32, cbs["nbytes"] // 4,
                             offset=h["data_offset"] + cbs["offset"])
            assert np.array_equal(cb, _ref_codebook(w, "frequency"))
            for key, (off, nb, dt) in e["sections"].items():
                assert off % cbq_image.ALIGN == 0 and off + nb <= h["payload_bytes"]
            if not enc:
                off, nb, _ = e["sections"]["packed"]
                raw = np.fromfile(path, np.uint8, nb, offset=h["data_offset"] + off)
                M, K = w.shape
                idx = bitpack.unpack_any_bits(raw, e["bits"], M * K).astype(np.int64)
                assert np.array_equal(cb[idx].reshape(M, K), w.float().numpy())


def test_image_rejects_foreign_files(tmp_path):
    p = tmp_path / "x.cbq"
    p.write_bytes(b"NOTANIMG" + bytes(32))
    with pytest.raises(ValueError):
        cbq_image.read_header(p)


def test_cli(ckpt, tmp_path, capsys):
    d, _ = ckpt
    out = tmp_path / "cli"
    assert cbq_compress.main([str(d), "--device", "cpu", "--out", str(out), "--no-image"]) == 0
    assert "3 tensors compressed" in capsys.readouterr().out
    assert cbq_compress.main([str(d), "--device", "cpu", "--out", str(out)]) == 0
    assert "already holds" in capsys.readouterr().out
    assert cbq_compress.main([str(tmp_path / "missing")]) == 1


def test_image_validation_rejects_corrupt_headers(ckpt, tmp_path):
    """The header checks that guard the kernels' descriptors: truncated
    payload, sections out of range or of the wrong size, unknown kinds."""
    import copy
    d, _ = ckpt
    for enc in (False, True):
        out = tmp_path / f"v{int(enc)}"
        cbq_compress.compress_checkpoint(d, out, entropy_code=enc, device="cpu",
                                         write_npz=False, log=lambda *a: None)
        path = out / "device.cbq"
        h = cbq_image.read_header(path)
        size = os.path.getsize(path)
        cbq_image.validate_header(h, size)                       # the writer's own image passes
        with pytest.raises(ValueError):
            cbq_image.validate_header(h, size - 1)                # truncated file
        name = "model.layers.0.self_attn.q_proj.weight"
        key = "packed" if not enc else "chunk_off"
        bad = copy.deepcopy(h)
        off, nb, dt = bad["tensors"][name]["sections"][key]
        M, K = SHAPES[name]
        e = h["tensors"][name]
        short = (M * K * e.get("bits", 0) + 7) // 8 if not enc else nb - 8   # no pad / one fewer
        bad["tensors"][name]["sections"][key] = [off, short, dt]
        with pytest.raises(ValueError):
            cbq_image.validate_header(bad, size)
        if not enc:
            # the reference's 4-byte pad is short of the 16-byte pieces the
            # streaming kernels read past the last word
            bad["tensors"][name]["sections"][key] = [off, short + 4, dt]
            with pytest.raises(ValueError):
                cbq_image.validate_header(bad, size)
        bad = copy.deepcopy(h)
        bad["payload_bytes"] = h["payload_bytes"] - 16            # payload not whole pages
        bad["data_offset"] = h["data_offset"] + 16
        with pytest.raises(ValueError):
            cbq_image.validate_header(bad, size)
        bad = copy.deepcopy(h)
        bad["tensors"][name]["sections"][key] = [h["payload_bytes"], nb, dt]   # past the end
        with pytest.raises(ValueError):
            cbq_image.validate_header(bad, size)
        bad = copy.deepcopy(h)
        bad["tensors"][name]["shape"] = [64, 256]                 # more weights than stored
        with pytest.raises(ValueError):
            cbq_image.validate_header(bad, size)
        bad = copy.deepcopy(h)
        bad["tensors"][name]["kind"] = "columns"
        with pytest.raises(ValueError):
            cbq_image.validate_header(bad, size)
