"""Build libggq_hip.so (HIP kernels + C ABI) in-tree for gfx950.

    python -m ggnpu_amd.build

hipcc cross-compiles for gfx950 without a GPU.  Every device pass is built
with packed-FP32 instructions disabled and with FP contraction off: the
bit-exact dequant follows the reference's separately rounded multiply and
subtract, and the other kernels request fused multiply-adds explicitly.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libggq_hip.so")
# the benchmark's C++ driver of the synchronous entry point (no link to LIB:
# it calls the entry point through a pointer the caller passes)
HOST_BENCH = os.path.join(LIB_DIR, "libggq_host_bench.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
SOURCES = ["ggq_kernels.hip", "ggq_gemv_i8.hip", "ggq_api.cpp", "ggq_encode.cpp", "ggq_gguf.cpp"]
CXX = os.environ.get("CXX", "g++")
# Host-only sources go through the host compiler against the HIP runtime API.
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
              "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("GGQ_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
    # MFMA results in VGPRs rather than AGPRs: the GEMM epilogue reads every
    # int32 product once, and the AGPR form costs a v_accvgpr_read for each.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def build(verbose: bool = False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    objs, cmds = [], []
    for src in SOURCES:
        obj = os.path.join(LIB_DIR, os.path.splitext(src)[0] + ".o")
        if src.endswith(".hip"):
            cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
        else:
            cmd = [CXX, *HOST_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        cmds.append(cmd)
        objs.append(obj)
    # the translation units compile in parallel
    procs = [subprocess.Popen(cmd, stderr=None if verbose else subprocess.PIPE) for cmd in cmds]
    failed = []
    for cmd, p in zip(cmds, procs):
        _, err = p.communicate()
        if p.returncode != 0:
            failed.append((cmd, err))
    if failed:
        cmd, err = failed[0]
        raise subprocess.CalledProcessError(1, cmd, stderr=err)
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
                    "-lpthread"], check=True)
    os.replace(tmp, LIB)
    cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-Wall", "-shared", f"-I{INCLUDE}",
           os.path.join(CSRC, "ggq_host_bench.cpp"), "-o", HOST_BENCH + ".tmp"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(HOST_BENCH + ".tmp", HOST_BENCH)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
