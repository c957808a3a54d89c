"""Builds the gfx950 kernel library in-tree: mnemocuda_amd/libmnemo_hip.so.

HIP sources are compiled with hipcc for gfx950 only; the C host composition
(csrc/host/mnemo_host.c) with the system C compiler; both link into one shared library
whose exported symbols are exactly the declarations of include/mnemo_kernels.h and
include/mnemo_host.h.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
LIB = PKG / "libmnemo_hip.so"
CALLER = PKG / "engine_calls"  # tests/c_caller/engine_calls.c, linked against LIB
GRAPH_CALLER = PKG / "attn_graph"  # tests/c_caller/attn_graph.c, linked against LIB
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

HIP_SOURCES = ["abi.hip", "gemv_launch.hip", "router.hip", "gemm.hip", "moe.hip", "sample.hip", "attn.hip", "attn_decode.hip", "embed.hip"]
C_SOURCES = ["host/mnemo_host.c", "host/mnemo_model.c"]

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    # no packed-fp32 VALU code anywhere in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-flush-denormals-to-zero",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
]


# per-source flags: the router's count-in atomic is issued by one lane before the row's
# loads; LLVM's atomic optimizer would rewrite it into a wave-wide form that reads the
# result back at once, waiting for the round trip before the loads go out
SOURCE_FLAGS = {"router.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]}


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
    noise = "is not a recognized feature for this target"
    msg = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l and l.strip())
    if msg:
        print(msg, file=sys.stderr)


def build(jobs: int = 4) -> Path:
    hipcc = str(ROCM / "bin" / "hipcc")
    cc = shutil.which(os.environ.get("CC", "gcc")) or "gcc"
    BUILD.mkdir(exist_ok=True)
    objs: list[Path] = []
    cmds: list[list[str]] = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".hip.o")
        cmds.append([hipcc, *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    # the GEMV kernels, once per workgroup size (gemv_launch.hip picks per launch)
    for threads in (512, 256):
        obj = BUILD / f"gemv{threads}.hip.o"
        cmds.append([hipcc, *HIPCC_FLAGS, f"-DMNEMO_GEMV_THREADS={threads}", f"-DMNEMO_GEMV_NS=g{threads}", "-c",
                     str(CSRC / "gemv.hip"), "-o", str(obj)])
        objs.append(obj)
    for src in C_SOURCES:
        obj = BUILD / (Path(src).stem + ".c.o")
        cmds.append([cc, "-O2", "-std=c11", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
                     f"-I{ROCM / 'include'}", "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, "-shared", "-fPIC", "--offload-arch=gfx950", *map(str, objs), "-o", str(tmp),
          f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"])
    tmp.replace(LIB)
    # the C callers of the C-ABI that the GPU tests run (tests/c_caller/)
    for name, exe in (("engine_calls.c", CALLER), ("attn_graph.c", GRAPH_CALLER)):
        src = ROOT / "tests" / "c_caller" / name
        if src.exists():
            _run([cc, "-O2", "-std=c11", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}",
                  str(src), "-o", str(exe), f"-L{LIB.parent}", "-lmnemo_hip", f"-L{ROCM / 'lib'}", "-lamdhip64",
                  "-lm", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM / 'lib'}"])
    return LIB


if __name__ == "__main__":
    print(build())
