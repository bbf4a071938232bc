"""Build the gfx950 HIP library and the torch op shim in-tree.

* ``nibble_amd/libw4a16_hip.so``: kernels + C ABI (hipcc, --offload-arch=gfx950)
* ``nibble_amd/_C.so``: libtorch shim registering ``w4a16::linear`` /
  ``w4a16::dequantize`` (g++ against torch's headers, linked to the above)

Run ``python -m nibble_amd.build``. Both outputs are git-ignored and travel
with the source tree to the GPU box.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-shared",
    # packed fp32 VALU ops stay off (compiler emits scalar fp32 instead)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # kernel arguments preloaded into SGPRs (the code object keeps a 256-byte
    # prologue that loads them from memory on firmware without preloading):
    # 2-3% on the small decode-size GEMVs
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln and "--hip-link" not in ln]
    if proc.returncode != 0:
        sys.stderr.write("\n".join(lines) + "\n")
        raise RuntimeError(f"build step failed ({proc.returncode}): {cmd[0]} ... {cmd[-1]}")
    if verbose and lines:
        print("\n".join(lines), flush=True)


HIP_SOURCES = ["w4a16_hip.hip", "w4a16_decode.hip", "w4a16_pair.hip", "w4a16_stream.hip", "w4a16_gemm.hip",
               "w4a16_pair_ring.hip"]


def build_hip(verbose: bool = False) -> str:
    """Compile every HIP source to an object (in parallel), then link the library."""
    out = os.path.join(HERE, "libw4a16_hip.so")
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    objs, procs = [], []
    for name in HIP_SOURCES:
        obj = os.path.join(CSRC, os.path.splitext(name)[0] + ".o")
        cmd = [hipcc, *compile_flags, f"-I{INCLUDE}", "-c", "-o", obj, os.path.join(CSRC, name)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs.append(obj)
    failed = None
    for cmd, proc in procs:
        text = proc.communicate()[0]
        lines = [ln for ln in text.splitlines() if "packed-fp32-ops" not in ln]
        if proc.returncode != 0:
            sys.stderr.write("\n".join(lines) + "\n")
            failed = failed or f"build step failed ({proc.returncode}): {cmd[-1]}"
        elif verbose and lines:
            print("\n".join(lines), flush=True)
    if failed:
        raise RuntimeError(failed)
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out, *objs], verbose)
    for obj in objs:
        os.remove(obj)
    return out


def build_shim(verbose: bool = False) -> str:
    import torch

    torch_dir = os.path.dirname(torch.__file__)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = os.path.join(HERE, "_C.so")
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        f"-I{INCLUDE}",
        f"-I{os.path.join(torch_dir, 'include')}",
        f"-I{os.path.join(torch_dir, 'include', 'torch', 'csrc', 'api', 'include')}",
        f"-I{os.path.join(ROCM, 'include')}",
        f"-I{sysconfig.get_paths()['include']}",
        os.path.join(CSRC, "torch_op.cpp"),
        "-o", out,
        f"-L{HERE}", "-lw4a16_hip", "-Wl,-rpath,$ORIGIN",
        f"-L{os.path.join(torch_dir, 'lib')}", f"-Wl,-rpath,{os.path.join(torch_dir, 'lib')}",
        "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch",
    ]
    _run(cmd, verbose)
    return out


def build(verbose: bool = False) -> None:
    build_hip(verbose)
    build_shim(verbose)


if __name__ == "__main__":
    build(verbose=True)
