"""The library's host-only C++ (csrc/cbq_huff_host.cpp, csrc/cbq_io.cpp) and
the oracle's C kernels under AddressSanitizer + UndefinedBehaviorSanitizer,
on the CPU: tests/native/cbq_host_sanitize.cpp runs the Huffman stream
indexer (offsets checked against its own encoder, then bit flips, truncated
streams, out-of-range and shuffled row starts, bad code lengths), the decode
table builders, cbq_file_upload's argument and file checks, and the oracle's
fixed-width and Huffman kernels on exactly padded inputs.  Any sanitizer
report aborts the program (non-zero exit)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
NATIVE = os.path.join(HERE, "native")


def test_host_code_under_sanitizers():
    r = subprocess.run(["make", "-s", "-C", NATIVE, "sanitize"], capture_output=True, text=True,
                       timeout=600)
    if r.returncode != 0:
        pytest.fail("sanitizer build failed:\n" + r.stderr[-3000:])
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:verify_asan_link_order=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([os.path.join(NATIVE, "cbq_host_sanitize")], capture_output=True,
                       text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "all cases passed" in r.stdout
    assert "runtime error" not in out and "AddressSanitizer" not in out
