"""Build the gfx950 code objects and the C-ABI host library, in-tree.

Outputs (under llmpager_amd/lib/):
  lp_basic.hsaco, lp_moe.hsaco,
  lp_gemm.hsaco, lp_attn.hsaco,
  lp_step.hsaco                   kernels, hipcc --genco --offload-arch=gfx950
  libllmpager_hip.so              host runtime (g++), loads the code objects
                                  with hipModuleLoad at lp_init

Run as `python -m llmpager_amd.build`.  Always recompiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
KDIR = os.path.join(CSRC, "kernels")
OUT = os.path.join(HERE, "lib")
ROOT = os.path.dirname(HERE)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

KERNEL_SOURCES = ["lp_basic.hip", "lp_moe.hip", "lp_gemm.hip", "lp_attn.hip", "lp_step.hip"]
HOST_SOURCES = ["lp_runtime.cpp", "lp_synth.cpp", "lp_cache.cpp", "lp_pager.cpp", "lp_pack.cpp"]
HOST_HIP_SOURCES = ["lp_noalloc.hip"]

# Packed-FP32 instructions stay off (the code is written for scalar fp32).
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "--genco",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _hipcc() -> str:
    p = os.path.join(ROCM, "bin", "hipcc")
    return p if os.path.exists(p) else (shutil.which("hipcc") or "hipcc")


def build_kernels() -> list[str]:
    os.makedirs(OUT, exist_ok=True)
    jobs = []
    for src in KERNEL_SOURCES:
        dst = os.path.join(OUT, src.replace(".hip", ".hsaco"))
        jobs.append([_hipcc(), *HIPCC_FLAGS, "-I", CSRC, os.path.join(KDIR, src), "-o", dst])
    with cf.ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        list(ex.map(_run, jobs))
    return [j[-1] for j in jobs]


def build_host() -> str:
    os.makedirs(OUT, exist_ok=True)
    dst = os.path.join(OUT, "libllmpager_hip.so")
    srcs = [os.path.join(CSRC, s) for s in HOST_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    # host-library sources that carry device code (a file-scope device array):
    # compiled by hipcc into relocatable objects with an embedded gfx950 code
    # object, then linked into the library with the rest
    objs = []
    for src in HOST_HIP_SOURCES:
        obj = os.path.join(OUT, src.replace(".hip", ".o"))
        _run([_hipcc(), "--offload-arch=gfx950", "-O2", "-std=c++17", "-fPIC", "-c",
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
              "-Wno-unused-command-line-argument", "-I", CSRC, os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
        "-Wall", "-Wno-unused-function",
        "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"), "-I", CSRC,
        *srcs, *objs, "-o", dst,
        "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
    ]
    _run(cmd)
    for obj in objs:
        os.remove(obj)
    return dst


def build_oracle() -> str:
    """The CPU checker (oracle/), built by its own Makefile."""
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])
    return os.path.join(ROOT, "oracle", "liblp_oracle.so")


def build_all(with_oracle: bool = True) -> None:
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        fk = ex.submit(build_kernels)
        fh = ex.submit(build_host)
        fk.result()
        fh.result()
    if with_oracle:
        build_oracle()


if __name__ == "__main__":
    build_all()
    print("built", OUT)
