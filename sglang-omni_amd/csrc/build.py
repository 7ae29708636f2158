"""Build the gfx950 codec kernels into the in-tree shared library ``libomni_codec.so``.

Each ``*.hip`` source compiles to an object in parallel, then one hipcc link produces
``sglang_omni_amd/libomni_codec.so`` next to the Python package that loads it. Runs without a
GPU (hipcc cross-compiles for gfx950).
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG_ROOT = CSRC.parent
REPO = PKG_ROOT.parent
INCLUDE = REPO / "include"
OUT_DIR = PKG_ROOT / "sglang_omni_amd"
LIB = OUT_DIR / "libomni_codec.so"
OBJ_DIR = PKG_ROOT / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["capi.hip", "rvq.hip", "conv.hip", "conv_k7_raw_wbf16.hip", "conv_k7_raw_wfp8.hip",
           "conv_k7_act_wbf16.hip", "conv_k7_act_wfp8.hip", "conv_k11.hip", "conv_ru_wbf16.hip",
           "conv_dma_t1.hip", "conv_dma_t2.hip", "conv_dma_t3.hip", "conv_dma_t7.hip",
           "conv_dma_t11.hip",
           "conv_ru_wfp8.hip", "residual_stack.hip", "residual_stack_wbf16.hip",
           "residual_stack_wfp8.hip", "single_output_conv.hip", "codec_state.hip", "snake.hip", "hift.hip",
           "egress.hip", "code2wav_front.hip", "channel_embedding.hip", "conv_general.hip",
           "gemm.hip", "resblock_pair.hip"]

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    # packed-FP32 VALU ops are kept off: the compiler may not form v_pk_{add,mul,fma}_f32.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _compile(src: str) -> Path:
    obj = OBJ_DIR / (Path(src).stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed on {src}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source for gfx950 and link the shared library; returns its path."""
    OBJ_DIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4, 16)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("hipcc link failed")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
