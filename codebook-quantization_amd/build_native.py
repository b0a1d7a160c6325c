"""Build recipe for libcbq_hip.so (gfx950 only).

    python codebook-quantization_amd/build_native.py

Compiles each csrc/*.hip with hipcc and the host-only csrc/*.cpp with g++
(in parallel) and links them into a shared library next to this file.  Packed-fp32 VALU ops are disabled (-packed-fp32-ops): the kernels are
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
# host-only C++ (no device code): compiled by the host compiler
HOST_SOURCES = ["cbq_huff_host.cpp", "cbq_io.cpp"]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-pthread", "-D__HIP_PLATFORM_AMD__=1",
              "-I/opt/rocm/include", "-Wall"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libcbq_hip.so)")


FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wno-unused-command-line-argument"]


def sources():
    return [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]


def host_sources():
    return [os.path.join(CSRC, s) for s in HOST_SOURCES]


TIMELINE_SO = os.path.join(HERE, "libcbq_hip_timeline.so")
TORCH_SO = os.path.join(HERE, "libcbq_torch.so")
TORCH_SRC = os.path.join(CSRC, "cbq_torch_ops.cpp")


def torch_ops_command(out: str = TORCH_SO):
    """g++ line of libcbq_torch.so: the torch.ops.cbq binding (host C++ only,
    no device code) over libcbq_hip.so, found next to it through $ORIGIN."""
    import torch
    tdir = os.path.dirname(torch.__file__)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return (["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__=1",
             "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
             "-I/opt/rocm/include", f"-I{tdir}/include",
             f"-I{tdir}/include/torch/csrc/api/include", TORCH_SRC, "-o", out,
             f"-L{tdir}/lib", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
             f"-L{HERE}", "-lcbq_hip", "-Wl,-rpath,$ORIGIN"])


def build_torch_ops(verbose: bool = False, out: str = TORCH_SO) -> str:
    """Compile the torch operator library (after libcbq_hip.so, which it links)."""
    cmd = torch_ops_command(out + ".tmp")
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("g++ failed on cbq_torch_ops.cpp:\n" + res.stderr[-4000:])
    os.replace(out + ".tmp", out)
    return out


def build(verbose: bool = False, jobs: int = 0, out: str = SO, defines=()) -> str:
    """Compile every time it is called (one hipcc per source, in parallel, in
    a temporary directory), link, and move the library to `out` (next to
    this file by default).  defines: extra -D macros (CBQ_TIMELINE builds the
    diagnostic variant)."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor
    srcs = sources() + host_sources()
    jobs = jobs or min(len(srcs), max(1, os.cpu_count() or 1))
    with tempfile.TemporaryDirectory(prefix="cbq_build_") as tmpd:
        objs = [os.path.join(tmpd, os.path.basename(s) + ".o") for s in srcs]

        def compile_one(so):
            src, obj = so
            if src.endswith(".cpp"):
                cmd = ["g++"] + HOST_FLAGS + [f"-D{d}" for d in defines] + ["-c", "-o", obj, src]
            else:
                cmd = [hipcc()] + FLAGS + [f"-D{d}" for d in defines] + ["-c", "-o", obj, src]
            if verbose:
                print(" ".join(cmd), flush=True)
            return subprocess.run(cmd, capture_output=True, text=True)

        with ThreadPoolExecutor(jobs) as ex:
            for src, res in zip(srcs, ex.map(compile_one, zip(srcs, objs))):
                if res.returncode != 0:
                    raise RuntimeError(f"hipcc failed on {src}:\n" + res.stderr[-4000:])
        tmp = os.path.join(tmpd, "libcbq_hip.so")
        cmd = [hipcc()] + FLAGS + ["-shared", "-pthread", "-o", tmp] + objs
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError("hipcc link failed:\n" + res.stderr[-4000:])
        shutil.copyfile(tmp, out + ".tmp")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    if "--timeline" in sys.argv:
        # the diagnostic library (per-wave timeline of the streaming GEMV)
        print(build(verbose="-v" in sys.argv, out=TIMELINE_SO, defines=("CBQ_TIMELINE",)))
    elif "--torch-ops" in sys.argv:
        print(build_torch_ops(verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
        print(build_torch_ops(verbose="-v" in sys.argv))
