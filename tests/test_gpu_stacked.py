"""Row-stacked fixed-width linears (q/k/v, gate/up in one matrix) give the
same outputs as the separate matrices, and the decoder built on them emits
the same greedy tokens."""
import ctypes

import pytest
import torch

import cbq_native as nat
import decoder
import synthetic

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def built(cuda):
    dec = synthetic.SyntheticDecoder("qwen3-8b", layers=2, log=lambda *a: None)
    names = dec.all_linears() + [dec.embed]
    return dec, dec.build_fixed(names)


def test_stacked_outputs_equal_separate(cuda, built):
    dec, tensors = built
    lib = nat.load()
    p = "model.layers.1."
    parts = [tensors[p + n] for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")]
    st = synthetic.stack_fixed(parts, p + "qkv")
    assert st is not None and st.shape == (4096 + 1024 + 1024, 4096)
    for T in (1, 3):
        x = torch.randn(T, 4096, device=cuda)
        y = torch.empty(T, st.shape[0], device=cuda)
        nat.check(lib.ck_linear_f32(x.data_ptr(), st.packed.data_ptr(), st.codebook.data_ptr(),
                                    y.data_ptr(), T, st.shape[0], 4096, st.codebook.numel(), st.bits,
                                    nat.stream_ptr(cuda)), "stacked")
        o = 0
        for t in parts:
            M = t.shape[0]
            ys = torch.empty(T, M, device=cuda)
            nat.check(lib.ck_linear_f32(x.data_ptr(), t.packed.data_ptr(), t.codebook.data_ptr(),
                                        ys.data_ptr(), T, M, 4096, t.codebook.numel(), t.bits,
                                        nat.stream_ptr(cuda)), "part")
            assert torch.equal(y[:, o:o + M], ys), (t.name, T)
            o += M


def test_stack_refuses_mismatched_codebooks(cuda, built):
    dec, tensors = built
    q = tensors["model.layers.0.self_attn.q_proj"]
    g = tensors["model.layers.0.mlp.gate_proj"]             # MLP codebook, not attention's
    assert synthetic.stack_fixed([q, g], "bad") is None


def test_stacked_decoder_tokens(cuda, built):
    dec, tensors = built
    c = dec.cfg
    cfg = decoder.DecoderConfig(layers=c["layers"], hidden=c["hidden"], inter=c["inter"],
                                n_q=c["n_q"], n_kv=c["n_kv"], head_dim=c["head_dim"],
                                vocab=c["vocab"])
    prompt = list(range(100, 116))
    a = decoder.from_synthetic(cfg, tensors, max_len=40, stack=True)
    assert "model.layers.0.self_attn.qkv_proj" in a.linears
    ta = a.generate_graph(prompt, 12)
    del a
    b = decoder.from_synthetic(cfg, tensors, max_len=40, stack=False)
    assert "model.layers.0.self_attn.qkv_proj" not in b.linears
    tb = b.generate_graph(prompt, 12)
    assert ta == tb
    assert b.generate(prompt, 12) == tb                     # eager loop agrees too


@pytest.fixture(scope="module")
def built_huff(cuda):
    dec = synthetic.SyntheticDecoder("qwen3-8b", layers=2, log=lambda *a: None)
    names = dec.all_linears() + [dec.embed]
    return dec, dec.build_huffman(names)


def test_grouped_huffman_launch_equals_single(cuda, built_huff):
    """cbq_huff_linear_col_multi_f32 over a layer's q/k/v (three codes)
    equals three single column GEMVs bit for bit."""
    from gpu_huffman_functions import build_columns
    dec, tensors = built_huff
    lib = nat.load()
    p = "model.layers.1."
    ts = [tensors[p + n] for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj")]
    K = 4096
    descs, cols = [], []
    for t in ts:
        tb = t.tables
        d = nat.HuffStream(words=t.words.data_ptr(), n_words=t.words.numel(),
                           chunk_off=t.chunk_off.data_ptr(), sub_len=t.sub_len.data_ptr(),
                           lut1=tb["lut1"].data_ptr(), lut2=tb["lut2"].data_ptr(),
                           n_lut2=tb["lut2"].numel(), canon=tb["canon"].data_ptr(),
                           canon_pay=tb["pay"].data_ptr(), value_cb=None,
                           C=tb["codebook"].numel(), stage_words=tb["stage_words"])
        descs.append(d)
        cols.append(build_columns(d, t.shape[0] * K, cuda, t.lengths,
                                  tb["codebook"].cpu().numpy()))
    x = torch.randn(1, K, device=cuda)
    Ms = [t.shape[0] for t in ts]
    y = torch.empty(1, sum(Ms), device=cuda)
    st = nat.stream_ptr(cuda)
    offs = [y.data_ptr() + 4 * sum(Ms[:i]) for i in range(3)]
    nat.check(lib.cbq_huff_linear_col_multi_f32(
        x.data_ptr(), 3, (ctypes.POINTER(nat.HuffStream) * 3)(*[ctypes.pointer(d) for d in descs]),
        (ctypes.POINTER(nat.HuffColumns) * 3)(*[ctypes.pointer(c[1]) for c in cols]),
        (ctypes.c_void_p * 3)(*offs), (ctypes.c_int * 3)(*Ms), K, st), "multi")
    o = 0
    for d, c, M in zip(descs, cols, Ms):
        ys = torch.empty(1, M, device=cuda)
        nat.check(lib.cbq_huff_linear_col_f32(x.data_ptr(), ctypes.byref(d), ctypes.byref(c[1]),
                                              ys.data_ptr(), M, K, st), "single")
        assert torch.equal(y[:, o:o + M], ys)
        o += M


def test_grouped_huffman_decoder_tokens(cuda, built_huff):
    dec, tensors = built_huff
    c = dec.cfg
    cfg = decoder.DecoderConfig(layers=c["layers"], hidden=c["hidden"], inter=c["inter"],
                                n_q=c["n_q"], n_kv=c["n_kv"], head_dim=c["head_dim"],
                                vocab=c["vocab"])
    prompt = list(range(300, 316))
    a = decoder.from_synthetic(cfg, tensors, max_len=40, stack=True)
    assert "model.layers.0.self_attn.qkv_proj" in a.linears
    ta = a.generate_graph(prompt, 10)
    del a
    b = decoder.from_synthetic(cfg, tensors, max_len=40, stack=False)
    assert ta == b.generate_graph(prompt, 10)

