"""Shared pytest setup: import paths, markers, seeds, GPU gating."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "codebook-quantization_amd")
ORACLE = os.path.join(ROOT, "oracle")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libcbq_hip.so")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(autouse=True)
def _seeds():
    np.random.seed(42)
    try:
        import torch
        torch.manual_seed(42)
    except ImportError:
        pass


@pytest.fixture(scope="session")
def oracle():
    import cbq_oracle
    if not os.path.exists(cbq_oracle.ORACLE_SO):
        cbq_oracle.build(ref=False)
    return cbq_oracle


@pytest.fixture(scope="session")
def golden():
    def load(name):
        d = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
        cases = {}
        for k in d.files:
            case, field = k.split("/", 1)
            cases.setdefault(case, {})[field] = d[k]
        return cases
    return {"fixed": load("fixed_golden.npz"), "huffman": load("huffman_golden.npz")}


@pytest.fixture(scope="session")
def cuda():
    """Skip unless a GPU is visible; fail (not skip) if the library is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import cbq_native
    cbq_native.load()       # raises when libcbq_hip.so is not built
    return torch.device("cuda:0")


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
