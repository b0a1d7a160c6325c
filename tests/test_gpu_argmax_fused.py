"""lm_head GEMV with the greedy pick fused (cbq_linear_xform_argmax_f32,
cbq_split_linear_argmax_f32): the logits equal the plain GEMV's bit for bit,
and the picked token equals torch.argmax of the oracle's logits (the
reference C kernel's, src/compressed_matmul.c:416-450) - first maximum on
ties, the first NaN when a row is NaN - with cbq_argmax_step's bookkeeping
(ids32, toks[pos - first], pos + 1)."""
import ctypes

import numpy as np
import pytest
import torch

import cbq_native as nat
import codebook_builder as cbb

pytestmark = pytest.mark.gpu


def _case(rng, M, K, special):
    """Weights [M, K] as indices into a codebook; `special` plants exact ties
    (two identical rows at the top) or NaN rows (a NaN codebook entry)."""
    w = cbb.bf16_round(rng.standard_normal((M, K)) * 0.02)
    cb, idx = cbb.frequency_sorted_codebook(w)
    idx = idx.reshape(M, K).astype(np.int64)
    x = np.abs(rng.standard_normal((1, K))).astype(np.float32)
    if special == "tie":
        top = int(np.argmax(cb))                        # the largest value, x > 0: rows win
        r1, r2 = M // 3, M // 3 + 17
        idx[r1] = top
        idx[r2] = top
        want = r1
    elif special == "nan":
        cb = np.concatenate([cb, np.float32([np.nan])])
        r1, r2 = M - 40, M // 2 + 3
        idx[r1, 5] = len(cb) - 1
        idx[r2, K - 1] = len(cb) - 1
        want = min(r1, r2)
    else:
        want = None
    return cb.astype(np.float32), idx, x, want


def _bookkeeping(cuda, pos0=9, first=4):
    ids = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    toks = torch.full((8,), -7, dtype=torch.int64, device=cuda)
    pos = torch.tensor([pos0], dtype=torch.int64, device=cuda)
    return ids, toks, pos, first


def _check_pick(ids, toks, pos, first, tok, pos0=9):
    assert int(ids[0]) == tok
    t = toks.cpu().numpy()
    assert t[pos0 - first] == tok and (np.delete(t, pos0 - first) == -7).all()
    assert int(pos[0]) == pos0 + 1


@pytest.mark.parametrize("M,K,special", [(5003, 4096, None), (4096, 2048, "tie"),
                                         (3000, 1024, "nan"), (151936, 1024, None)])
@pytest.mark.parametrize("mode", [0, 3])                 # x0 itself; RMSNorm(x0)
def test_fixed_xform_argmax(cuda, oracle, M, K, special, mode):
    lib = nat.load()
    rng = np.random.default_rng(M + K + mode)
    cb, idx, x, want = _case(rng, M, K, special)
    bits = cbb.bits_for(len(cb))
    packed = oracle.pack_lsb(idx.reshape(-1), bits)
    pk = torch.zeros(packed.size + 32, dtype=torch.uint8, device=cuda)
    pk[:packed.size] = torch.from_numpy(packed).to(cuda)
    cbd = torch.from_numpy(cb).to(cuda)
    xd = torch.from_numpy(x).to(cuda)
    st = nat.stream_ptr(cuda)
    plain = torch.empty(1, M, device=cuda)
    if mode == 0:
        nat.check(lib.ck_linear_f32(xd.data_ptr(), pk.data_ptr(), cbd.data_ptr(),
                                    plain.data_ptr(), 1, M, K, len(cb), bits, st), "plain")
        x_eff = x
    else:
        nat.check(lib.cbq_linear_xform_f32(xd.data_ptr(), None, None, mode, 1e-6, pk.data_ptr(),
                                           cbd.data_ptr(), plain.data_ptr(), M, K, len(cb), bits,
                                           st), "plain xform")
        x64 = x.astype(np.float64)
        x_eff = (x64 / np.sqrt((x64 ** 2).mean() + 1e-6)).astype(np.float32)
    logits = torch.full((1, M), 7.0, device=cuda)
    ws = torch.empty(nat.ARGMAX_WORKSPACE, dtype=torch.uint8, device=cuda)
    ids, toks, pos, first = _bookkeeping(cuda)
    nat.check(lib.cbq_linear_xform_argmax_f32(
        xd.data_ptr(), None, None, mode, 1e-6, pk.data_ptr(), cbd.data_ptr(), logits.data_ptr(),
        M, K, len(cb), bits, ws.data_ptr(), ws.numel(), ids.data_ptr(), toks.data_ptr(),
        pos.data_ptr(), first, toks.numel(), st), "argmax")
    torch.cuda.synchronize()
    assert torch.equal(logits.isnan(), plain.isnan())
    assert torch.equal(logits.nan_to_num(0.0), plain.nan_to_num(0.0))
    tok = int(torch.argmax(plain))
    if want is not None:
        assert tok == want
    else:
        ref = oracle.fixed_gemv(x_eff, packed, cb, M, K, bits, chunk_rows=None)
        assert tok == int(torch.argmax(torch.from_numpy(ref)))
    _check_pick(ids, toks, pos, first, tok)
    # without the logits: the same pick
    ids2, toks2, pos2, _ = _bookkeeping(cuda)
    nat.check(lib.cbq_linear_xform_argmax_f32(
        xd.data_ptr(), None, None, mode, 1e-6, pk.data_ptr(), cbd.data_ptr(), None,
        M, K, len(cb), bits, ws.data_ptr(), ws.numel(), ids2.data_ptr(), toks2.data_ptr(),
        pos2.data_ptr(), first, toks2.numel(), st), "argmax, no logits")
    _check_pick(ids2, toks2, pos2, first, tok)


@pytest.mark.parametrize("M,K,special", [(4096, 4096, "tie"), (6000, 2048, None),
                                         (2048, 6144, None), (8192, 4096, "nan")])
def test_split_argmax(cuda, oracle, M, K, special):
    from gpu_huffman_functions import build_split
    lib = nat.load()
    rng = np.random.default_rng(M * 3 + K)
    cb, idx, x, want = _case(rng, M, K, special)      # a NaN entry is a bf16 value too
    sp = build_split(torch.from_numpy(idx.reshape(-1).astype(np.int32)).to(cuda), cb, cuda)
    assert sp is not None
    xd = torch.from_numpy(x).to(cuda)
    st = nat.stream_ptr(cuda)
    plain = torch.empty(1, M, device=cuda)
    nat.check(lib.cbq_split_linear_f32(
        xd.data_ptr(), None, None, 0, 1e-6, 1,
        (ctypes.POINTER(nat.SplitMatrix) * 1)(ctypes.pointer(sp[1])),
        (ctypes.c_void_p * 1)(plain.data_ptr()), (ctypes.c_int * 1)(M), K, st), "plain")
    logits = torch.full((1, M), 7.0, device=cuda)
    ws = torch.empty(nat.ARGMAX_WORKSPACE, dtype=torch.uint8, device=cuda)
    ids, toks, pos, first = _bookkeeping(cuda)
    nat.check(lib.cbq_split_linear_argmax_f32(
        xd.data_ptr(), None, None, 0, 1e-6, ctypes.byref(sp[1]), logits.data_ptr(), M, K,
        ws.data_ptr(), ws.numel(), ids.data_ptr(), toks.data_ptr(), pos.data_ptr(), first,
        toks.numel(), st), "split argmax")
    torch.cuda.synchronize()
    assert torch.equal(logits.isnan(), plain.isnan())
    assert torch.equal(logits.nan_to_num(0.0), plain.nan_to_num(0.0))
    tok = int(torch.argmax(plain))
    if want is not None:
        assert tok == want
    else:
        bits = cbb.bits_for(len(cb))
        ref = oracle.fixed_gemv(x, oracle.pack_lsb(idx.reshape(-1), bits), cb, M, K, bits,
                                chunk_rows=None)
        assert tok == int(torch.argmax(torch.from_numpy(ref)))
    _check_pick(ids, toks, pos, first, tok)


def test_decoder_graph_tokens_with_fused_pick(cuda):
    """The graph-captured decode step (lm_head GEMV + fused pick) gives the
    same tokens as eager steps with torch.argmax over the logits."""
    import decoder
    import synthetic
    dec = synthetic.SyntheticDecoder("qwen3-8b", layers=2, log=lambda *a: None)
    names = dec.all_linears() + [dec.embed]
    c = dec.cfg
    cfg = decoder.DecoderConfig(layers=c["layers"], hidden=c["hidden"], inter=c["inter"],
                                n_q=c["n_q"], n_kv=c["n_kv"], head_dim=c["head_dim"],
                                vocab=c["vocab"])
    for enc in ("fixed", "huffman"):
        tensors = dec.build_huffman(names) if enc == "huffman" else dec.build_fixed(names)
        m = decoder.from_synthetic(cfg, tensors, max_len=40)
        assert callable(getattr(m.linears["lm_head"], "xform_argmax", None)), enc
        prompt = list(range(1000, 1012))
        assert m.generate_graph(prompt, 12) == m.generate(prompt, 12), enc
        del m, tensors
        torch.cuda.empty_cache()
