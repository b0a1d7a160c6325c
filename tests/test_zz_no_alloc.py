"""cbq_attn_rope_decode_noalloc_f32 (split one-token attention with its
partials in the library's static scratch) against the workspace entry point
cbq_attn_rope_decode_ws_f32 it varies: same kernels, so outputs and cache
rows must be equal bit for bit.  Two calls in a row, the second smaller, so
the scratch's leftover contents from the first call must not leak into the
second; and a shape whose partials exceed the scratch is refused on the
host."""
import pytest
import torch

import cbq_native as nat
import decoder

pytestmark = pytest.mark.gpu


def _inputs(cuda, n_q, n_kv, hd, max_len, pos0, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n_q * hd, generator=g).to(cuda)
    k = torch.randn(n_kv * hd, generator=g).to(cuda)
    v = torch.randn(n_kv * hd, generator=g).to(cuda)
    kc = torch.randn(n_kv, max_len, hd, generator=g).to(cuda)
    vc = torch.randn(n_kv, max_len, hd, generator=g).to(cuda)
    cfg = decoder.DecoderConfig(layers=1, hidden=n_q * hd, inter=64, n_q=n_q, n_kv=n_kv,
                                head_dim=hd, vocab=16)
    cos, sin = (torch.from_numpy(a).to(cuda) for a in decoder.rope_tables(cfg, max_len))
    pos = torch.tensor([pos0], dtype=torch.int64, device=cuda)
    return q, k, v, kc, vc, cos, sin, pos


def _call(lib, name, cuda, inp, n_q, n_kv, hd, max_len, ws=None):
    q, k, v, kc, vc, cos, sin, pos = inp
    kc, vc = kc.clone(), vc.clone()
    out = torch.full((n_q * hd,), float("nan"), device=cuda)
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None, cos.data_ptr(), sin.data_ptr(),
            pos.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), n_q, n_kv, hd, max_len,
            float(hd ** -0.5), 1e-6)
    if ws is not None:
        rc = lib.cbq_attn_rope_decode_ws_f32(*args, ws.data_ptr(), ws.numel(),
                                             nat.stream_ptr(cuda))
    else:
        rc = getattr(lib, name)(*args, nat.stream_ptr(cuda))
    torch.cuda.synchronize(cuda)
    return rc, out, kc, vc


@pytest.mark.parametrize("shapes", [
    # (n_q, n_kv, hd, max_len, pos): a long cache first, then a smaller call
    [(32, 8, 128, 2048, 1500), (8, 2, 64, 300, 123)],
    [(16, 4, 256, 1024, 1023), (4, 4, 128, 96, 5)],
])
def test_noalloc_equals_workspace(cuda, shapes):
    lib = nat.load()
    print(f"noalloc vs ws: {shapes}", flush=True)
    for i, (n_q, n_kv, hd, max_len, pos0) in enumerate(shapes):
        inp = _inputs(cuda, n_q, n_kv, hd, max_len, pos0, seed=11 + i)
        need = lib.cbq_attn_rope_decode_workspace(n_q, hd, max_len)
        ws = torch.empty(need, dtype=torch.uint8, device=cuda)
        rc0, ref, kc0, vc0 = _call(lib, None, cuda, inp, n_q, n_kv, hd, max_len, ws=ws)
        rc1, out, kc1, vc1 = _call(lib, "cbq_attn_rope_decode_noalloc_f32", cuda, inp, n_q,
                                   n_kv, hd, max_len)
        assert rc0 == 0 and rc1 == 0
        assert torch.isfinite(ref).all()
        assert torch.equal(out, ref)
        assert torch.equal(kc1, kc0) and torch.equal(vc1, vc0)


def test_noalloc_refuses_oversize(cuda):
    lib = nat.load()
    n_q, n_kv, hd, max_len = 128, 8, 128, 2048          # 128*16*130*4 bytes > 1 MiB
    assert lib.cbq_attn_rope_decode_workspace(n_q, hd, max_len) > (1 << 20)
    inp = _inputs(cuda, n_q, n_kv, hd, max_len, 700, seed=3)
    rc, out, _, _ = _call(lib, "cbq_attn_rope_decode_noalloc_f32", cuda, inp, n_q, n_kv, hd,
                          max_len)
    assert rc == nat.CK_ERR_ARG
    assert torch.isnan(out).all()                       # nothing was launched
