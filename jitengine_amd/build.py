"""Compile the gfx950 HIP sources into jitengine_amd/_lib/libjit_moe.so (hipcc, in-tree).

Every HIP translation unit is built with the packed-FP32 feature disabled (hipcc forms
v_pk_{add,mul,fma}_f32 from ordinary float code otherwise).  router.hip is built with
-ffp-contract=off: its softmax must reproduce the CPU restatement bit for bit.  qmm.hip is
built with MFMA results in ordinary VGPRs (-amdgpu-mfma-vgpr-form) instead of accumulation
registers, which removes a register copy per MFMA result from its inner loops, and so is
attention.hip (the prefill kernel's scores feed the softmax directly; the decode kernels compile to
the same code either way); qmm_seg.hip is not (its accumulators live in accumulation registers).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(HERE, "_lib")
LIB = os.path.join(OUT_DIR, "libjit_moe.so")
PROBE_LIB = os.path.join(OUT_DIR, "libjit_probe.so")  # bench.py's measurement kernels (csrc/probe.hip)
# the quantized projections and decode attention with per-workgroup phase stamps (JIT_QMM_STAMPS=1,
# JIT_ATTN_STAMPS=1), for bench.py --gemv-phases and --attn-phases
STAMPS_LIB = os.path.join(OUT_DIR, "libjit_stamps.so")
ARCH = "gfx950"

SOURCES = {
    "errors.cpp": [],
    "router.hip": ["-ffp-contract=off"],
    "qmm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "qmm_seg.hip": [],
    "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "block.hip": [],
    "head.hip": [],
    "sampler.hip": ["-ffp-contract=off"],
}

_COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", f"-I{INCLUDE}", f"-I{CSRC}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP extension cannot be built")
    return path


def _compile(src: str, extra: list, verbose: bool, tag: str = "") -> str:
    obj = os.path.join(OUT_DIR, src + tag + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [hipcc(), *lang, *_COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every source and link the shared library; returns its path."""
    os.makedirs(OUT_DIR, exist_ok=True)
    jobs = [(src, extra, "") for src, extra in SOURCES.items()]
    jobs += [(src, SOURCES[src] + ["-DJIT_QMM_STAMPS=1", "-DJIT_ATTN_STAMPS=1"], ".stamps")
             for src in ("errors.cpp", "qmm.hip", "attention.hip")]
    with ThreadPoolExecutor(max_workers=4) as ex:
        built = list(ex.map(lambda j: _compile(j[0], j[1], verbose, j[2]), jobs))
    objs, stamp_objs = built[:len(SOURCES)], built[len(SOURCES):]
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    _link(stamp_objs, STAMPS_LIB, verbose)
    for o in objs + stamp_objs:
        os.remove(o)
    _build_probe(verbose)
    return LIB


def _link(objs: list, out: str, verbose: bool) -> None:
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)


def _build_probe(verbose: bool) -> None:
    """The benchmark's measurement kernels, a library of their own (never loaded by the package)."""
    tmp = PROBE_LIB + ".tmp"
    cmd = [hipcc(), "-x", "hip", *_COMMON, "-shared", os.path.join(CSRC, "probe.hip"), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on probe.hip:\n{r.stderr}")
    os.replace(tmp, PROBE_LIB)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
