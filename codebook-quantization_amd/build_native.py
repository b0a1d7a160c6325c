"""Build recipe for libcbq_hip.so (gfx950 only).

    python codebook-quantization_amd/build_native.py

Compiles csrc/*.hip with hipcc straight into a shared library next to this
file.  Packed-fp32 VALU ops are disabled (-packed-fp32-ops): the kernels are
written for scalar fp32 FMAs.
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
SO = os.path.join(HERE, "libcbq_hip.so")
ARCH = "gfx950"
SOURCES = ["cbq_fixed.hip", "cbq_huffman.hip", "cbq_prefill.hip", "cbq_prefill_f32.hip",
           "cbq_decode.hip", "cbq_split.hip", "cbq_tiny.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libcbq_hip.so)")


def command(out: str = SO):
    srcs = [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wno-unused-command-line-argument", "-pthread", "-o", out] + srcs


def build(verbose: bool = False) -> str:
    """Compile every time it is called; write atomically next to this file."""
    tmp = SO + ".tmp"
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + res.stderr[-4000:])
    os.replace(tmp, SO)
    return SO


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
