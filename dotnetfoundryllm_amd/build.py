"""Build step for the native libraries (gfx950 HIP device library + C++ host library).

Compiles in-tree so the built .so files sit next to the sources:
  dotnetfoundryllm_amd/libfllm_hip.so   <- csrc/*.hip (hipcc, gfx950; one object per source, compiled
                                           in parallel under _build/, then linked)
  dotnetfoundryllm_amd/libfllm_host.so  <- host/fllm_host.cpp              (g++, links the above)
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("FLLM_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # a*b+c stays two roundings unless fmaf() is written: dequantized values and the RoPE
    # rotation must follow the reference's operation order bit for bit
    "-ffp-contract=off",
    "-Wno-unused-value",
    "-Wno-unused-result",
    # no packed-FP32 instructions in generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden", "-ffp-contract=off", "-Wall", "-Wextra"]


def _run(cmd, cwd):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed ({' '.join(cmd[:2])} ...):\n{out}")
    return out


DEVICE_SRCS = ["csrc/kernels.hip", "csrc/gemv.hip", "csrc/attention.hip", "csrc/prefill.hip", "csrc/api.hip"]


def build_device_lib(verbose=False):
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)

    def compile_one(src):
        obj = os.path.join("_build", os.path.splitext(os.path.basename(src))[0] + ".o")
        return obj, _run([HIPCC, *HIP_FLAGS, "-c", "-o", obj, src], PKG)

    with ThreadPoolExecutor(max_workers=min(len(DEVICE_SRCS), os.cpu_count() or 1)) as pool:
        results = list(pool.map(compile_one, DEVICE_SRCS))
    out = "libfllm_hip.so"
    tmp = out + ".tmp"
    log = "\n".join(r[1] for r in results)
    log += _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[r[0] for r in results]], PKG)
    os.replace(os.path.join(PKG, tmp), os.path.join(PKG, out))
    if verbose and log.strip():
        print(log)
    return os.path.join(PKG, out)


def build_host_lib(verbose=False):
    out = "libfllm_host.so"
    tmp = out + ".tmp"
    log = _run(["g++", *HOST_FLAGS, "-o", tmp, "host/fllm_host.cpp", "-L.", "-lfllm_hip",
                "-Wl,-rpath,$ORIGIN", "-lpthread"], PKG)
    os.replace(os.path.join(PKG, tmp), os.path.join(PKG, out))
    if verbose and log.strip():
        print(log)
    return os.path.join(PKG, out)


def build_all(verbose=False):
    build_device_lib(verbose)
    build_host_lib(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
    print("built", os.path.join(PKG, "libfllm_hip.so"), os.path.join(PKG, "libfllm_host.so"))
    sys.exit(0)
