"""Build the native libraries in-tree.

* ``inferox_amd/lib/libinferox.so``  — HIP kernels for gfx950 + C++ host + C ABI
  (hipcc; every translation unit with -ffp-contract=off, packed-FP32 disabled).
* ``inferox_amd/lib/libifx_synth.so`` — host-only synthetic GGUF payload generator.
* ``oracle/liboracle.so``             — the CPU oracle (test infrastructure).

Usage: ``python -m inferox_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib")
ARCH = os.environ.get("IFX_OFFLOAD_ARCH", "gfx950")

HIP_SOURCES = ["kern_dequant.hip", "kern_gemv.hip", "kern_gemv_mfma.hip", "kern_ops.hip", "kern_attn.hip",
               "kern_gemm.hip", "kern_attn_prefill.hip", "kern_sample.hip", "noalloc.hip",
               "host_types.cpp", "host_gguf.cpp", "host_config.cpp", "host_model.cpp", "capi_ops.cpp", "capi_attn.cpp", "host_tokenizer.cpp"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off",  # the reference never fuses a*b+c; only explicit fmaf() fuse here
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}")
    return r.stdout


def build_product(jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIB, exist_ok=True)
    hipcc = _hipcc()
    objs = []

    def compile_one(src):
        obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        out = _run([hipcc, *HIPCC_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", obj])
        if verbose and out.strip():
            print(out)
        return obj

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, HIP_SOURCES))
    out_so = os.path.join(LIB, "libinferox.so")
    tmp = out_so + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"])
    os.replace(tmp, out_so)
    # the `inferox` command (src/main.rs), linked against the library beside it
    cli_obj = os.path.join(OBJ, "cli_main.o")
    _run([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, "cli_main.cpp"), "-o", cli_obj])
    cli = os.path.join(LIB, "inferox")
    _run([hipcc, f"--offload-arch={ARCH}", "-o", cli + ".tmp", cli_obj, "-L" + LIB, "-linferox",
          "-Wl,-rpath,$ORIGIN"])
    os.replace(cli + ".tmp", cli)
    return out_so


def build_synth() -> str:
    os.makedirs(LIB, exist_ok=True)
    out = os.path.join(LIB, "libifx_synth.so")
    _run(["g++", "-O2", "-fPIC", "-shared", "-fopenmp", "-std=c++17",
          os.path.join(CSRC, "synth_fill.cpp"), "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_oracle() -> str:
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])
    return os.path.join(ROOT, "oracle", "liboracle.so")


def build_all(verbose: bool = False) -> None:
    build_synth()
    build_oracle()
    build_product(verbose=verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built:", os.listdir(LIB))
