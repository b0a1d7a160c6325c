"""RMSNorm and the SiLU product staged by the GEMVs that consume them
(cbq_linear_xform_f32, cbq_huff_linear_col_xform_f32) equal the separate
decoder glue kernels followed by the plain GEMV, bit for bit, and the
decoder built on them emits the same logits and tokens."""
import pytest
import torch

import cbq_native as nat
import decoder
import synthetic

pytestmark = pytest.mark.gpu


def _cfg(dec):
    c = dec.cfg
    return decoder.DecoderConfig(layers=c["layers"], hidden=c["hidden"], inter=c["inter"],
                                 n_q=c["n_q"], n_kv=c["n_kv"], head_dim=c["head_dim"],
                                 vocab=c["vocab"])


@pytest.fixture(scope="module", params=["fixed", "huffman"])
def model(request, cuda):
    dec = synthetic.SyntheticDecoder("qwen3-8b", layers=2, log=lambda *a: None)
    names = dec.all_linears() + [dec.embed]
    tensors = dec.build_fixed(names) if request.param == "fixed" else dec.build_huffman(names)
    return request.param, dec, tensors


@pytest.mark.parametrize("name", ["model.layers.1.self_attn.qkv_proj",
                                  "model.layers.1.mlp.gate_up_proj", "model.layers.1.mlp.down_proj",
                                  "lm_head"])
def test_xform_equals_glue_then_gemv(cuda, model, name):
    kind, dec, tensors = model
    cfg = _cfg(dec)
    m = decoder.from_synthetic(cfg, tensors, max_len=8)
    lin = m.linears[name]
    assert callable(getattr(lin, "xform", None)), (kind, name)
    g = decoder._Glue(cfg)
    gen = torch.Generator(device=cuda).manual_seed(5)
    for rep in range(3):
        if name.endswith("down_proj"):
            a = torch.randn(1, cfg.inter, device=cuda, generator=gen) * 3
            b = torch.randn(1, cfg.inter, device=cuda, generator=gen)
            want = lin(g.silu_mul(a, b))
            got = lin.xform(a, b, None, nat.XF_SILU)
            assert torch.equal(got, want), (kind, name, rep, "silu")
            continue
        h = torch.randn(1, cfg.hidden, device=cuda, generator=gen) * 2
        d = torch.randn(1, cfg.hidden, device=cuda, generator=gen)
        want = lin(g.add_rms(h.clone(), None))
        got = lin.xform(h, None, None, nat.XF_RMS)
        assert torch.equal(got, want), (kind, name, rep, "rms")
        hc = h.clone()
        want = lin(g.add_rms(hc, d))
        h2 = torch.full_like(h, float("nan"))
        got = lin.xform(h, d, h2, nat.XF_ADD_RMS)
        assert torch.equal(h2, hc), (kind, name, rep, "h_out")
        assert torch.equal(got, want), (kind, name, rep, "add_rms")


def test_fused_decoder_identical(cuda, model):
    """One-token steps with the glue folded into the GEMVs give the same
    logits as the separate glue kernels, and the same tokens."""
    kind, dec, tensors = model
    cfg = _cfg(dec)
    prompt = torch.tensor(list(range(500, 520)))
    models = [decoder.from_synthetic(cfg, tensors, max_len=48, fuse_glue=f) for f in (True, False)]
    assert models[0].fused and not models[1].fused
    logits = []
    for m in models:
        m.reset()
        m.forward(prompt)                                   # multi-token prefill (unfused)
        steps = [m.forward(torch.tensor([7]))]
        for _ in range(3):
            steps.append(m.forward(torch.tensor([int(torch.argmax(steps[-1]))])))
        logits.append(steps)
    for s, (a, b) in enumerate(zip(*logits)):
        assert torch.equal(a, b), (kind, s, float((a - b).abs().max()))
    toks = [m.generate_graph(list(range(40, 52)), 8) for m in models]
    assert toks[0] == toks[1]


def test_long_cache_split_attention_decoder(cuda, model, monkeypatch):
    """A decoder whose cache is long enough for the split-over-blocks
    attention gives the same tokens as the single-launch attention and
    logits equal to rounding (graph replays and eager steps), and repeats
    its own logits bit for bit."""
    kind, dec, tensors = model
    cfg = _cfg(dec)
    prompt = list(range(40, 52))

    def run(split):
        monkeypatch.setattr(decoder._Glue, "SPLIT_ATTN_MIN_LEN", 2048 if split else 1 << 30)
        m = decoder.from_synthetic(cfg, tensors, max_len=2048)
        toks = m.generate_graph(prompt, 6)
        m.reset()
        m.forward(torch.tensor(prompt))
        return toks, m.forward(torch.tensor([7]))

    ta, la = run(True)
    tb, lb = run(False)
    assert ta == tb, (kind, ta, tb)
    rel = float((la - lb).norm() / lb.norm())
    assert rel <= 1e-5, (kind, rel)
    tc, lc = run(True)
    assert tc == ta and torch.equal(lc, la), kind


@pytest.mark.parametrize("M,K,bits,C", [(12288, 4096, 13, 5000),     # 8B gate/up shape
                                        (137733, 32, 13, 8192),     # > 64 pairs per wave
                                        (1003, 4096, 11, 2048),     # ragged pair count
                                        (77, 96, 8, 300),           # fewer pairs than waves
                                        (300, 6144, 13, 4000)])     # K > 4096: 16 glue terms
def test_glu_epilogue_equals_gemv_then_silu(cuda, M, K, bits, C):
    """cbq_linear_xform_glu_f32 over a row-stacked [gate; up] matrix equals
    the stacked GEMV (same x transform) followed by cbq_silu_mul_f32, bit for
    bit; plain x (mode 0) is checked against ck_linear_f32 + silu within the
    GEMV tolerance, since ck_linear_f32 may pick another kernel at small K."""
    lib = nat.load()
    gen = torch.Generator(device=cuda).manual_seed(M + K)
    nbytes = 2 * M * K * bits // 8
    packed = torch.randint(0, 256, (nbytes + 256,), dtype=torch.uint8, device=cuda,
                           generator=gen)
    cb = torch.randn(C, device=cuda, generator=gen)
    st = nat.stream_ptr(cuda)

    def silu_mul(y):
        out = torch.empty(1, M, device=cuda)
        nat.check(lib.cbq_silu_mul_f32(y[:, :M].contiguous().data_ptr(),
                                       y[:, M:].contiguous().data_ptr(), out.data_ptr(), M, st),
                  "cbq_silu_mul_f32")
        return out

    def glu(h, d, h_out, mode):
        out = torch.full((1, M), float("nan"), device=cuda)
        nat.check(lib.cbq_linear_xform_glu_f32(
            h.data_ptr(), None if d is None else d.data_ptr(),
            None if h_out is None else h_out.data_ptr(), mode, 1e-6, packed.data_ptr(),
            cb.data_ptr(), out.data_ptr(), M, K, C, bits, st), "cbq_linear_xform_glu_f32")
        return out

    for rep in range(2):
        h = torch.randn(1, K, device=cuda, generator=gen) * 2
        d = torch.randn(1, K, device=cuda, generator=gen)
        for mode in (nat.XF_RMS, nat.XF_ADD_RMS):
            y = torch.empty(1, 2 * M, device=cuda)
            h_ref = torch.full_like(h, float("nan"))
            nat.check(lib.cbq_linear_xform_f32(
                h.data_ptr(), d.data_ptr() if mode == nat.XF_ADD_RMS else None,
                h_ref.data_ptr(), mode, 1e-6, packed.data_ptr(), cb.data_ptr(), y.data_ptr(),
                2 * M, K, C, bits, st), "cbq_linear_xform_f32")
            want = silu_mul(y)
            h_out = torch.full_like(h, float("nan"))
            got = glu(h, d if mode == nat.XF_ADD_RMS else None, h_out, mode)
            assert torch.equal(got, want), (M, K, rep, mode)
            if mode == nat.XF_ADD_RMS:
                assert torch.equal(h_out, h_ref), (M, K, rep)
        y = torch.empty(1, 2 * M, device=cuda)
        nat.check(lib.ck_linear_f32(h.data_ptr(), packed.data_ptr(), cb.data_ptr(), y.data_ptr(),
                                    1, 2 * M, K, C, bits, st), "ck_linear_f32")
        want = silu_mul(y).double()
        got = glu(h, None, None, 0).double()
        rel = float((got - want).norm() / want.norm())
        assert rel <= 1e-5, (M, K, rep, rel)
