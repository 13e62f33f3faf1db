"""Builds the gfx950 C-ABI library physllm_amd/libphysllm_moe.so with hipcc.

Every HIP translation unit in physllm_amd/csrc is compiled for gfx950 only, with
packed-fp32 instruction selection disabled, then linked into one shared library
exporting the symbols declared in include/physllm_moe.h.

    python -m physllm_amd.build          # or physllm_amd.build.build()
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libphysllm_moe.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    p = os.path.join(rocm, "bin", "hipcc")
    return p if os.path.exists(p) else (shutil.which("hipcc") or "hipcc")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


COMMON_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc()] + COMMON_FLAGS + ["-DPHYSLLM_MOE_BUILD", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    # the host pass does not know the packed-fp32 feature; that warning is expected
    noise = [l for l in r.stderr.splitlines() if l.strip() and "packed-fp32-ops" not in l]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} HIP sources for {ARCH}")
    return LIB_PATH


def build_host_test(verbose: bool = True) -> str:
    """C++ host-layer test driver (tests/cpp/test_host_api), linked against the
    library and the CPU oracle (oracle/liboracle.so must be built first)."""
    root = os.path.dirname(HERE)
    src = os.path.join(root, "tests", "cpp", "test_host_api.cpp")
    out = os.path.join(root, "tests", "cpp", "test_host_api")
    cmd = [hipcc(), "-O2", "-std=c++17", src, "-o", out,
           "-L" + HERE, "-lphysllm_moe", "-L" + os.path.join(root, "oracle"), "-loracle",
           "-Wl,-rpath," + HERE, "-Wl,-rpath," + os.path.join(root, "oracle"),
           "-Wl,-rpath,$ORIGIN/../../physllm_amd", "-Wl,-rpath,$ORIGIN/../../oracle"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host test build failed:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {out}")
    return out


def build_checkpoint_tools(verbose: bool = True) -> list:
    """tests/cpp/checkpoint_tool (g++, the safetensors reader and GPT-OSS layer view on
    the CPU) and tests/cpp/gpt_oss_block (hipcc, loads a layer and runs the block)."""
    root = os.path.dirname(HERE)
    cpp = os.path.join(root, "tests", "cpp")
    tool = os.path.join(cpp, "checkpoint_tool")
    blk = os.path.join(cpp, "gpt_oss_block")
    cmds = [
        ["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", os.path.join(cpp, "checkpoint_tool.cpp"), "-o", tool],
        [hipcc(), "-O2", "-std=c++17", os.path.join(cpp, "gpt_oss_block.cpp"), "-o", blk,
         "-L" + HERE, "-lphysllm_moe", "-Wl,-rpath," + HERE, "-Wl,-rpath,$ORIGIN/../../physllm_amd"],
    ]
    for cmd in cmds:
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    if verbose:
        print(f"built {tool} and {blk}")
    return [tool, blk]


if __name__ == "__main__":
    build()
