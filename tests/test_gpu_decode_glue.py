"""Fused decoder glue kernels (include/cbq_decode.h) against plain PyTorch
fp32 restatements of the HF Qwen3 ops they replace: RMSNorm with residual
add, q/k head norm + rotary embedding + KV-cache write, single-token GQA
attention, SiLU product.  Elementwise steps are rounded as torch rounds them,
so those outputs are compared exactly; reductions differ in order only."""
import numpy as np
import pytest
import torch

import cbq_native as nat
import decoder

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = a.double().cpu(); b = b.double().cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


@pytest.fixture(scope="module")
def lib():
    return nat.load()


@pytest.mark.parametrize("T,H,with_delta,with_weight", [(1, 4096, True, False), (3, 2048, False, True),
                                                         (2, 100, True, True)])
def test_add_rmsnorm(cuda, lib, T, H, with_delta, with_weight):
    g = torch.Generator().manual_seed(T * 7 + H)
    h = torch.randn(T, H, generator=g).to(cuda)
    d = torch.randn(T, H, generator=g).to(cuda) if with_delta else None
    w = (torch.rand(H, generator=g) + 0.5).to(cuda) if with_weight else None
    h0 = h.clone()
    out = torch.empty_like(h)
    nat.check(lib.cbq_add_rmsnorm_f32(h.data_ptr(), nat.ptr(d), nat.ptr(w), out.data_ptr(), T, H,
                                      1e-6, nat.stream_ptr(cuda)), "add_rmsnorm")
    hr = h0 + d if with_delta else h0
    ref = hr * torch.rsqrt(hr.pow(2).mean(-1, keepdim=True) + 1e-6)
    if with_weight:
        ref = w * ref
    assert torch.equal(h, hr)                       # residual add is exact
    assert _rel(out, ref) <= 1e-6


@pytest.mark.parametrize("T,hd,pos0", [(1, 128, 37), (5, 64, 0), (2, 256, 10), (3, 128, 62)])
def test_head_norm_rope_cache(cuda, lib, T, hd, pos0):
    n_q, n_kv, max_len, eps = 8, 2, 64, 1e-6
    g = torch.Generator().manual_seed(hd + T)
    q = torch.randn(T, n_q * hd, generator=g).to(cuda)
    k = torch.randn(T, n_kv * hd, generator=g).to(cuda)
    v = torch.randn(T, n_kv * hd, generator=g).to(cuda)
    cfg = decoder.DecoderConfig(layers=1, hidden=n_q * hd, inter=64, n_q=n_q, n_kv=n_kv,
                                head_dim=hd, vocab=16)
    cos, sin = (torch.from_numpy(a).to(cuda) for a in decoder.rope_tables(cfg, max_len))
    kc = torch.full((n_kv, max_len, hd), 7.0, device=cuda)
    vc = torch.full((n_kv, max_len, hd), 7.0, device=cuda)
    q_out = torch.empty_like(q)
    pos = torch.tensor([pos0], dtype=torch.int64, device=cuda)
    nat.check(lib.cbq_head_norm_rope_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None,
                                         cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
                                         q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), T, n_q,
                                         n_kv, hd, max_len, eps, nat.stream_ptr(cuda)), "rope")

    def ref(x, heads):
        x = x.view(T, heads, hd)
        x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
        ps = torch.arange(pos0, pos0 + T, device=cuda)
        ps = torch.where(ps < max_len, ps, torch.zeros_like(ps))   # table row 0 past the cache
        c, s = cos[ps][:, None, :], sin[ps][:, None, :]
        rot = torch.cat([-x[..., hd // 2:], x[..., :hd // 2]], dim=-1)
        return x * c + rot * s

    assert _rel(q_out.view(T, n_q, hd), ref(q, n_q)) <= 1e-6
    kr = ref(k, n_kv)
    n_in = max(0, min(T, max_len - pos0))
    for t in range(T):
        p = pos0 + t
        if t < n_in:
            assert _rel(kc[:, p], kr[t]) <= 1e-6
            assert torch.equal(vc[:, p], v.view(T, n_kv, hd)[t])
    untouched = torch.ones(max_len, dtype=torch.bool)
    untouched[pos0:pos0 + n_in] = False
    assert bool((kc[:, untouched.to(cuda)] == 7.0).all()) and bool((vc[:, untouched.to(cuda)] == 7.0).all())


def test_head_norm_rope_skips_positions_past_cache(cuda, lib):
    """Tokens at positions >= max_len write nothing (no out-of-bounds store)."""
    T, n_q, n_kv, hd, max_len = 4, 2, 1, 64, 8
    q = torch.randn(T, n_q * hd, device=cuda)
    k = torch.randn(T, n_kv * hd, device=cuda)
    v = torch.randn(T, n_kv * hd, device=cuda)
    cos = torch.ones(max_len, hd, device=cuda); sin = torch.zeros(max_len, hd, device=cuda)
    kc = torch.zeros(n_kv, max_len + 4, hd, device=cuda)      # guard rows after the cache
    vc = torch.zeros(n_kv, max_len + 4, hd, device=cuda)
    q_out = torch.empty_like(q)
    pos = torch.tensor([6], dtype=torch.int64, device=cuda)   # tokens at 6, 7, 8, 9
    # view the first max_len rows as the cache: stride per kv head is max_len+4 rows,
    # so use n_kv = 1 and pass max_len = 8
    nat.check(lib.cbq_head_norm_rope_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None,
                                         cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
                                         q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), T, n_q,
                                         n_kv, hd, max_len, 1e-6, nat.stream_ptr(cuda)), "rope")
    assert bool((kc[0, 6:8] != 0).any()) and bool((kc[0, max_len:] == 0).all())
    assert bool((vc[0, max_len:] == 0).all())


@pytest.mark.parametrize("hd,n_q,n_kv,pos0,max_len", [(128, 32, 8, 0, 512), (128, 32, 8, 130, 512),
                                                      (64, 4, 2, 63, 64), (256, 4, 4, 300, 1024),
                                                      (128, 8, 1, 511, 512)])
def test_attn_decode(cuda, lib, hd, n_q, n_kv, pos0, max_len):
    g = torch.Generator().manual_seed(pos0 + hd)
    q = torch.randn(n_q, hd, generator=g).to(cuda)
    kc = torch.randn(n_kv, max_len, hd, generator=g).to(cuda)
    vc = torch.randn(n_kv, max_len, hd, generator=g).to(cuda)
    out = torch.empty(n_q, hd, device=cuda)
    pos = torch.tensor([pos0], dtype=torch.int64, device=cuda)
    scale = hd ** -0.5
    nat.check(lib.cbq_attn_decode_f32(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(),
                                      out.data_ptr(), n_q, n_kv, hd, max_len, scale,
                                      nat.stream_ptr(cuda)), "attn")
    L = pos0 + 1
    rep = n_q // n_kv
    kk = kc[:, :L].repeat_interleave(rep, 0).cpu()           # [n_q, L, hd], CPU fp32
    vv = vc[:, :L].repeat_interleave(rep, 0).cpu()
    s = torch.einsum("hd,hld->hl", q.cpu(), kk) * scale
    ref = torch.einsum("hl,hld->hd", torch.softmax(s, -1), vv)
    assert _rel(out, ref) <= 1e-5


def test_silu_mul(cuda, lib):
    g = torch.randn(12288 * 3 + 5, device=cuda) * 4
    u = torch.randn_like(g)
    out = torch.empty_like(g)
    nat.check(lib.cbq_silu_mul_f32(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(),
                                   nat.stream_ptr(cuda)), "silu")
    ref = torch.nn.functional.silu(g) * u
    assert _rel(out, ref) <= 1e-6


@pytest.mark.parametrize("hd,n_q,n_kv,pos0,max_len", [(128, 32, 8, 0, 512), (128, 32, 8, 200, 512),
                                                      (64, 4, 2, 63, 64), (256, 8, 2, 17, 64)])
def test_attn_rope_decode_matches_two_step(cuda, lib, hd, n_q, n_kv, pos0, max_len):
    """The fused one-token kernel equals head_norm_rope followed by
    attn_decode, and writes the same cache row."""
    g = torch.Generator().manual_seed(pos0 * 3 + hd)
    q = torch.randn(n_q * hd, generator=g).to(cuda)
    k = torch.randn(n_kv * hd, generator=g).to(cuda)
    v = torch.randn(n_kv * hd, generator=g).to(cuda)
    cfg = decoder.DecoderConfig(layers=1, hidden=n_q * hd, inter=64, n_q=n_q, n_kv=n_kv,
                                head_dim=hd, vocab=16)
    cos, sin = (torch.from_numpy(a).to(cuda) for a in decoder.rope_tables(cfg, max_len))
    kc = torch.randn(n_kv, max_len, hd, generator=g).to(cuda)
    vc = torch.randn(n_kv, max_len, hd, generator=g).to(cuda)
    kc2, vc2 = kc.clone(), vc.clone()
    pos = torch.tensor([pos0], dtype=torch.int64, device=cuda)
    st = nat.stream_ptr(cuda)
    out = torch.empty(n_q * hd, device=cuda)
    nat.check(lib.cbq_attn_rope_decode_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None,
                                           cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
                                           kc.data_ptr(), vc.data_ptr(), out.data_ptr(), n_q, n_kv,
                                           hd, max_len, hd ** -0.5, 1e-6, st), "fused")
    qr = torch.empty_like(q)
    nat.check(lib.cbq_head_norm_rope_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None,
                                         cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
                                         qr.data_ptr(), kc2.data_ptr(), vc2.data_ptr(), 1, n_q,
                                         n_kv, hd, max_len, 1e-6, st), "rope")
    ref = torch.empty_like(out)
    nat.check(lib.cbq_attn_decode_f32(qr.data_ptr(), kc2.data_ptr(), vc2.data_ptr(),
                                      pos.data_ptr(), ref.data_ptr(), n_q, n_kv, hd, max_len,
                                      hd ** -0.5, st), "attn")
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    assert _rel(out, ref) <= 1e-6


@pytest.mark.parametrize("hd,n_q,n_kv,pos0,max_len", [(128, 32, 8, 0, 512), (128, 32, 8, 200, 512),
                                                      (128, 32, 8, 511, 512), (64, 4, 2, 63, 64),
                                                      (256, 8, 2, 17, 64), (128, 8, 2, 3000, 4096),
                                                      (128, 4, 4, 64, 64), (64, 8, 8, 700, 1000)])
def test_attn_rope_split_matches_fused(cuda, lib, hd, n_q, n_kv, pos0, max_len):
    """The split-over-blocks kernels (flash decoding, then a merge launch)
    write the same cache row as the one-block kernel, give its output to
    rounding and the float64 softmax attention to 1e-5, and repeat bit for
    bit on a workspace left dirty by the previous call."""
    g = torch.Generator().manual_seed(pos0 * 7 + hd + n_q)
    q = torch.randn(n_q * hd, generator=g).to(cuda)
    k = torch.randn(n_kv * hd, generator=g).to(cuda)
    v = torch.randn(n_kv * hd, generator=g).to(cuda)
    cfg = decoder.DecoderConfig(layers=1, hidden=n_q * hd, inter=64, n_q=n_q, n_kv=n_kv,
                                head_dim=hd, vocab=16)
    cos, sin = (torch.from_numpy(a).to(cuda) for a in decoder.rope_tables(cfg, max_len + 1))
    kc = torch.randn(n_kv, max_len, hd, generator=g).to(cuda)
    vc = torch.randn(n_kv, max_len, hd, generator=g).to(cuda)
    kc2, vc2 = kc.clone(), vc.clone()
    pos = torch.tensor([pos0], dtype=torch.int64, device=cuda)
    st = nat.stream_ptr(cuda)
    nbytes = lib.cbq_attn_rope_decode_workspace(n_q, hd, max_len)
    ws = torch.full((nbytes,), 0x7f, dtype=torch.uint8, device=cuda)
    outs = []
    for _ in range(2):
        kcs, vcs = kc.clone(), vc.clone()
        out = torch.empty(n_q * hd, device=cuda)
        nat.check(lib.cbq_attn_rope_decode_ws_f32(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None, cos.data_ptr(), sin.data_ptr(),
            pos.data_ptr(), kcs.data_ptr(), vcs.data_ptr(), out.data_ptr(), n_q, n_kv, hd, max_len,
            hd ** -0.5, 1e-6, ws.data_ptr(), nbytes, st), "split")
        outs.append((out, kcs, vcs))
    assert torch.equal(outs[0][0], outs[1][0])
    ref = torch.empty_like(outs[0][0])
    nat.check(lib.cbq_attn_rope_decode_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None,
                                           cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
                                           kc2.data_ptr(), vc2.data_ptr(), ref.data_ptr(), n_q,
                                           n_kv, hd, max_len, hd ** -0.5, 1e-6, st), "fused")
    out, kcs, vcs = outs[0]
    assert torch.equal(kcs, kc2) and torch.equal(vcs, vc2)
    assert _rel(out, ref) <= 2e-6
    # float64 reference over the rows the kernel attends: the cached rows
    # [0, min(pos, max_len)) and the new (normed, rotated) key/value
    qr = torch.empty_like(q)
    kc3, vc3 = kc.clone(), vc.clone()
    nat.check(lib.cbq_head_norm_rope_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None,
                                         cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
                                         qr.data_ptr(), kc3.data_ptr(), vc3.data_ptr(), 1, n_q,
                                         n_kv, hd, max_len, 1e-6, st), "rope")
    n_old = min(pos0, max_len)
    rep = n_q // n_kv
    kk = kc[:, :n_old].double().cpu()
    vv = vc[:, :n_old].double().cpu()
    if pos0 < max_len:
        knew, vnew = kc3[:, pos0].double().cpu(), vc3[:, pos0].double().cpu()
    else:
        knew, vnew = None, None
    if knew is not None:
        kk = torch.cat([kk, knew[:, None]], 1)
        vv = torch.cat([vv, vnew[:, None]], 1)
        kk, vv = kk.repeat_interleave(rep, 0), vv.repeat_interleave(rep, 0)
        s = torch.einsum("hd,hld->hl", qr.view(n_q, hd).double().cpu(), kk) * hd ** -0.5
        want = torch.einsum("hl,hld->hd", torch.softmax(s, -1), vv)
        assert _rel(out.view(n_q, hd), want) <= 1e-5


@pytest.mark.parametrize("n", [1, 7, 151936])
def test_argmax_step(cuda, lib, n):
    x = torch.randn(n, device=cuda)
    if n > 7:
        x[90000] = x[100000] = x.max() + 1        # tie across slices: the first index wins
    ids = torch.full((1,), -5, dtype=torch.int32, device=cuda)
    toks = torch.zeros(8, dtype=torch.int64, device=cuda)
    pos = torch.tensor([20], dtype=torch.int64, device=cuda)
    ws = torch.empty(256, dtype=torch.int32, device=cuda)
    nat.check(lib.cbq_argmax_step(x.data_ptr(), n, ws.data_ptr(), ids.data_ptr(), toks.data_ptr(),
                                  pos.data_ptr(), 17, 8, nat.stream_ptr(cuda)), "argmax")
    want = int(torch.argmax(x))
    assert int(ids[0]) == want and int(toks[3]) == want and int(pos[0]) == 21
    assert int(toks.sum()) == want                  # nothing else written
    pos.fill_(40)                                   # index outside toks: only ids and pos change
    nat.check(lib.cbq_argmax_step(x.data_ptr(), n, ws.data_ptr(), ids.data_ptr(), toks.data_ptr(),
                                  pos.data_ptr(), 17, 8, nat.stream_ptr(cuda)), "argmax")
    assert int(pos[0]) == 41 and int(toks.sum()) == want
