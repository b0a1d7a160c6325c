"""benchmark configs 2 and 4 at their own shapes.

Config 2: every Qwen3-1.7B layer shape (K -> M: 2048 -> 2048, 2048 -> 1024,
6144 -> 2048, 2048 -> 6144), fixed-width lossless indices, T = 1, 4, 16,
against the oracle's C GEMV (rel-L2 <= 1e-5).

Config 4: the 9B prefill GEMMs at T = 512 and 2048 over full-width matrices
(q, k, gate, down), bf16 activations, on the path the bench times
(cbq_linear_bf16_ws).  The reference for three 64-row slices of each output
is the dense product of x (bf16 values, float64) with the slices' weights,
decoded from the same packed stream by the oracle's C unpack: the C GEMV at
these T takes minutes per slice on the host.  Bar rel-L2 <= 2e-3 (bf16
outputs of an fp32-accumulated product)."""
import numpy as np
import pytest
import torch

import codebook_builder as cbb
import synthetic
from conftest import rel_l2
from test_gpu_fixed import _run_linear

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("K,M", [(2048, 2048), (2048, 1024), (6144, 2048), (2048, 6144)])
@pytest.mark.parametrize("T", [1, 4, 16])
def test_config2_shapes(cuda, oracle, K, M, T):
    w = synthetic.make_bf16((M, K), f"config2.{K}x{M}", device="cpu").float().numpy()
    d = cbb.compress_fixed(w)
    bits = d["bits"]
    x = np.random.default_rng(T + K).standard_normal((T, K)).astype(np.float32)
    y = _run_linear(cuda, x, d["indices"], d["codebook"], M, K, len(d["codebook"]), bits)
    ref = oracle.fixed_gemv(x, d["indices"], d["codebook"], M, K, bits, chunk_rows=None)
    assert rel_l2(y, ref) <= 1e-5, (K, M, T)


@pytest.mark.parametrize("name,K,M", [("q", 4096, 4096), ("k", 4096, 1024),
                                      ("gate", 4096, 12288), ("down", 12288, 4096)])
@pytest.mark.parametrize("T", [512, 2048])
def test_config4_full_width(cuda, oracle, name, K, M, T):
    """T = 512 runs the split-K launch plans (q: 32 tiles x 8 K splits, k:
    8 x 16, gate: 96 x 2), T = 2048 whole tiles."""
    import cbq_native as nat
    lib = nat.load()
    wb = synthetic.make_bf16((M, K), f"config4.{name}", device=cuda)
    cb, lut = cbb.codebook_from_counts_torch(cbb.counts_torch(wb))
    bits = cbb.bits_for(cb.numel())
    idx = lut[cbb.patterns_torch(wb).reshape(-1).to(torch.int64)]
    del wb
    pk = cbb.pack_torch(idx, bits)
    packed = torch.zeros(pk.numel() + 32, dtype=torch.uint8, device=cuda)
    packed[:pk.numel()] = pk
    del idx, pk
    xb = torch.randn(T, K, generator=torch.Generator().manual_seed(K + M + T)).bfloat16().to(cuda)
    out = torch.full((T, M), float("nan"), dtype=torch.bfloat16, device=cuda)
    nws = int(lib.cbq_linear_bf16_workspace(T, M, K))
    ws = torch.empty(max(1, nws // 4), dtype=torch.float32, device=cuda)
    nat.check(lib.cbq_linear_bf16_ws(xb.data_ptr(), packed.data_ptr(), cb.data_ptr(),
                                     out.data_ptr(), T, M, K, cb.numel(), bits, ws.data_ptr(), nws,
                                     nat.stream_ptr(cuda)), "cbq_linear_bf16_ws")
    torch.cuda.synchronize()
    x64 = xb.float().cpu().numpy().astype(np.float64)
    cbn = cb.cpu().numpy()
    row_bytes = K * bits // 8                               # K * bits is a multiple of 8
    for r0 in (0, M // 2 - 32, M - 64):
        raw = packed[r0 * row_bytes:(r0 + 64) * row_bytes].cpu().numpy()
        ridx = oracle.unpack_indices_c(raw, bits, 64 * K).reshape(64, K)
        wr = cbn[np.minimum(ridx, len(cbn) - 1)].astype(np.float64)
        ref = x64 @ wr.T
        y = out[:, r0:r0 + 64].float().cpu().numpy()
        assert np.isfinite(y).all()
        assert rel_l2(y, ref) <= 2e-3, (name, r0, rel_l2(y, ref))
