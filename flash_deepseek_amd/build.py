"""Build libfdm.so (the HIP kernels + C ABI) in-tree for gfx950.

    python -m flash_deepseek_amd.build        # or build() from Python

Each .hip translation unit is compiled by hipcc in parallel, then linked
into flash_deepseek_amd/libfdm.so.  Packed-FP32 instructions are disabled
for all device code (-packed-fp32-ops).
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libfdm.so")
ARCH = "gfx950"

SOURCES = [
    "quant_kernels.hip",
    "matvec_kernels.hip",
    "router_kernels.hip",
    "moe_kernels.hip",
    "layer_kernel.hip",
    "expert_kernels.hip",
    "read_ceiling.hip",
    "batched_kernels.hip",
    "prefill_kernels.hip",
    "gemm_kernels.hip",
    "synth_kernels.hip",
    "dense_kernels.hip",
    "expert_stream.hip",
    "attn_kernels.hip",
    "gguf_host.hip",
    "capi.hip",
]

CXXFLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfdm.so)")


def _compile(hipcc, src, verbose):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc, *CXXFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = (res.stdout + res.stderr).strip()
    # hipcc's host pass does not know the device-only feature; that is harmless
    lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), file=sys.stderr)
    return obj


def build(verbose=False, jobs=None):
    """Compile every kernel source and link libfdm.so.  Returns the path."""
    hipcc = _hipcc()
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, verbose), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
