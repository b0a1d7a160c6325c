"""The native C-ABI test (tests/native/cbq_abi_test.cpp, the analogue of the
reference's rocm/test_kernel.cpp run by rocm/Makefile:62): a C++ program that
uploads host arrays with ck_upload_codebook / ck_upload_packed, runs
ck_linear_f32 / ck_linear_bf16 / ck_embedding_f32 and compares with the
oracle's C library.  Built by __graft_entry__.build() (make -C tests/native)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "cbq_abi_test")


def test_native_abi_program(cuda):
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built (make -C tests/native)")
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stdout[-2000:]
    assert "all cases passed" in r.stdout
    assert r.stdout.count("PASS") >= 13
