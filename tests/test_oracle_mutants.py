"""The Q4K fit's known answers catch plausible restatement mistakes: the oracle is built
once per mistake with it planted (ORC_MUTANT in oracle/pkv_oracle.c: one pass fewer, one
pass more, no early exit, ties to even, pairwise sums, GGML's make_qkx2_quants instead of
make_qkx1_quants, no min clamp inside the loop), and each build must fail at least one
known answer that the real oracle passes (tests/q4k_known_answers.py)."""
import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest

from q4k_known_answers import BLOCK_PQ_HEADER, BLOCK_PQ_QS, BLOCK_PQ_X, FITS

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "oracle", "pkv_oracle.c")
MUTANTS = {1: "one pass fewer", 2: "one pass more", 3: "no early exit", 4: "ties to even",
           5: "pairwise sums", 6: "make_qkx2_quants", 7: "no min clamp in the loop"}
FP = ctypes.POINTER(ctypes.c_float)


def _build(tmp, m):
    out = os.path.join(tmp, f"orc_mutant_{m}.so")
    subprocess.check_call([shutil.which("gcc") or "gcc", "-O2", "-std=c11", "-fPIC",
                           "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-w",
                           f"-DORC_MUTANT={m}", "-shared", "-o", out, SRC, "-lm"])
    return out


def _failures(path):
    """Names of the known answers this build gets wrong."""
    L = ctypes.CDLL(path)
    L.orc_make_qkx1_quants.argtypes = [FP, ctypes.c_int, ctypes.c_int, ctypes.c_int, FP, FP]
    L.orc_q4k_quantize.argtypes = [FP, ctypes.POINTER(ctypes.c_uint8), ctypes.c_size_t]
    bad = []
    for name, (x, sb, mb) in FITS.items():
        a = np.array(x, dtype=np.float32)
        s, m = ctypes.c_float(), ctypes.c_float()
        L.orc_make_qkx1_quants(a.ctypes.data_as(FP), a.size, 15, 5, ctypes.byref(s), ctypes.byref(m))
        got = tuple(int(np.array([v.value], dtype=np.float32).view(np.uint32)[0]) for v in (s, m))
        if got != (sb, mb):
            bad.append(name)
    a = np.array(BLOCK_PQ_X, dtype=np.float32)
    b = np.zeros(144, dtype=np.uint8)
    L.orc_q4k_quantize(a.ctypes.data_as(FP), b.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), 256)
    if list(b[:16]) != BLOCK_PQ_HEADER or list(b[16:]) != BLOCK_PQ_QS:
        bad.append("block")
    return bad


@pytest.fixture(scope="module")
def tmpdir_mut(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc is not available")
    return str(tmp_path_factory.mktemp("mutants"))


def test_unmutated_build_passes(tmpdir_mut):
    assert _failures(_build(tmpdir_mut, 0)) == []


@pytest.mark.parametrize("m", sorted(MUTANTS))
def test_mutant_is_caught(tmpdir_mut, m):
    bad = _failures(_build(tmpdir_mut, m))
    assert bad, f"planted mistake '{MUTANTS[m]}' passes every known answer"
