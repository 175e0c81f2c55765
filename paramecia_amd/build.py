"""Builds libpkv.so (the HIP kernels + C ABI) in-tree with hipcc for gfx950.

Each translation unit is compiled separately so that the quantizer keeps IEEE
two-rounding arithmetic (-ffp-contract=off) while the attention kernels may contract.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libpkv.so")
OBJ = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Packed FP32 VOP3P forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Leading scalar kernel arguments arrive in SGPRs at wave launch (gfx950 kernarg
    # preload); a kernel whose only argument is a struct is unaffected.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]
SOURCES = {
    "pkv_quant.hip": ["-ffp-contract=off"],
    "pkv_attn.hip": [],
    "pkv_attn_mfma.hip": [],
    "pkv_attn_mfma_prep.hip": [],
    "pkv_prefill_mfma.hip": [],
    "pkv_prefill_q8.hip": [],
    "pkv_q8_decode.hip": [],
    "pkv_util.hip": [],
    "pkv_deltanet.hip": [],
    "pkv_oproj.hip": [],
    "pkv_oproj_mfma.hip": [],
    "pkv_prep.hip": ["-ffp-contract=off"],
    "pkv_api.cpp": ["-x", "hip"],
    "pkv_paged.cpp": ["-x", "hip"],
}


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    warn = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if warn.strip():
        sys.stderr.write(warn + "\n")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        objs = list(ex.map(lambda kv: _compile(*kv), SOURCES.items()))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
