"""Build recipe for the gfx950 attention library (libzwgpu.so) and the C++ host test program.

    python -m zwhisper_amd.build          # compiles in-tree

Every HIP source is compiled with hipcc for gfx950 only, with packed-FP32 code generation
switched off (-Xclang -target-feature -Xclang -packed-fp32-ops).  Objects go to
zwhisper_amd/_build/, the library to zwhisper_amd/libzwgpu.so.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
BUILD = os.path.join(PKG, "_build")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(PKG, "libzwgpu.so")
CPP_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_attention.cpp")
CPP_TEST_BIN = os.path.join(BUILD, "test_attention")

SOURCES = ["zw_gpu.hip", "attn_flash.hip", "attn_flash_x3.hip", "attn_decode.hip", "attn_pad.hip", "attn_generic.hip", "kv_cache.hip", "linear.hip", "elementwise.hip",
           "encoder_layer.hip", "decoder.hip", "llm_step.hip"]
HOST_SOURCES = ["zw_ops.cpp"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: keeps the compiler from parking them in AGPRs and copying
    # them back and forth around every MFMA chain
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    f"-I{HOST}",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        err = (r.stdout + r.stderr).splitlines()
        sys.stderr.write(" ".join(cmd) + "\n" + "\n".join(err[:60]) + "\n")
        raise RuntimeError(f"build step failed: {cmd[-1]}")


def build(verbose: bool = False, defines: list[str] | None = None, out: str | None = None,
          build_dir: str | None = None) -> str:
    """Compile the library (and the C++ test program when building the default library).

    defines: extra -D options for the tunables of the kernels and planner; out/build_dir: where
    to put the library and objects (default: zwhisper_amd/libzwgpu.so, zwhisper_amd/_build/).
    """
    bdir = build_dir or BUILD
    lib = out or LIB
    os.makedirs(bdir, exist_ok=True)
    extra = [f"-D{d}" for d in (defines or [])]
    cc = hipcc()
    jobs = []
    objs = []
    for src in SOURCES:
        obj = os.path.join(bdir, src.replace(".hip", ".o"))
        objs.append(obj)
        jobs.append([cc, *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    for src in HOST_SOURCES:
        obj = os.path.join(bdir, src.replace(".cpp", ".o"))
        objs.append(obj)
        jobs.append([cc, *HIP_FLAGS, *extra, "-x", "c++", "-c", os.path.join(HOST, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=min(4, len(jobs))) as ex:
        list(ex.map(_run, jobs))
    tmp = lib + ".tmp"
    _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, lib)
    if lib == LIB and os.path.exists(CPP_TEST_SRC):
        _run([cc, "-O2", "-std=c++17", f"-I{INCLUDE}", f"-I{HOST}", CPP_TEST_SRC, "-o", CPP_TEST_BIN,
              f"-L{PKG}", "-lzwgpu", f"-Wl,-rpath,{PKG}", "-Wl,-rpath,$ORIGIN/.."])
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    build(verbose=True)
