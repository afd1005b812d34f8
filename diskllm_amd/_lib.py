"""ctypes binding of libdiskllm_amd.so (include/diskllm_amd.h, include/sampler.h,
include/grammar.h).

The library is built in-tree by diskllm_amd/csrc/Makefile (see build()).  Loading
fails loudly if it is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libdiskllm_amd.so")
CSRC = os.path.join(HERE, "csrc")

DLK_OK = 0
DLK_ERR_INVALID = -1
DLK_ERR_UNSUPPORTED = -2
DLK_ERR_HIP = -3
DLK_STATUS_HISTORY_TOO_LONG = 1
PATH_AUTO, PATH_ROW, PATH_FULL_EXACT = 0, 1, 2

OP_REPETITION, OP_FREQUENCY, OP_PRESENCE = 1, 2, 3
ORDER_REFERENCE = OP_PRESENCE | (OP_REPETITION << 4)
ORDER_REP_FREQ_PRES = OP_REPETITION | (OP_FREQUENCY << 4) | (OP_PRESENCE << 8)


class SampleParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("frequency_penalty", C.c_float), ("presence_penalty", C.c_float),
                ("penalty_order", C.c_uint32), ("max_history", C.c_int), ("n_out", C.c_int),
                ("path", C.c_int)]


class Batch(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("ld", C.c_int64), ("hist_off", C.c_void_p), ("hist_ids", C.c_void_p),
                ("mask", C.c_void_p), ("mask_ld", C.c_int64), ("mask_row", C.c_void_p), ("rng", C.c_void_p),
                ("out_ids", C.c_void_p), ("out_cand_ids", C.c_void_p), ("out_cand_probs", C.c_void_p),
                ("out_cand_logprobs", C.c_void_p), ("status", C.c_void_p)]


class SamplerConfig(C.Structure):
    """include/sampler.h:10-16."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("seed", C.c_uint64)]


# Every symbol the public headers declare (checked by the CPU test suite).
EXPORTS = [
    # include/diskllm_amd.h
    "dlk_seed_state", "dlk_sample", "dlk_dfa_mask", "dlk_expf",
]


def build(quiet: bool = True) -> None:
    """Compile every HIP source for gfx950 and link the shared library in-tree."""
    jobs = str(min(16, os.cpu_count() or 4))
    r = subprocess.run(["make", "-C", CSRC, "-j", jobs], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("libdiskllm_amd build failed:\n" + r.stdout[-4000:] + r.stderr[-8000:])
    if not quiet:
        print(r.stdout)


_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run diskllm_amd._lib.build() (no fallback path exists)")
        L = C.CDLL(LIB_PATH)
        L.dlk_seed_state.restype = C.c_uint64
        L.dlk_seed_state.argtypes = [C.c_uint64]
        L.dlk_sample.restype = C.c_int
        L.dlk_sample.argtypes = [C.POINTER(Batch), C.c_int, C.c_int, C.POINTER(SampleParams), C.c_void_p]
        L.dlk_dfa_mask.restype = C.c_int
        L.dlk_dfa_mask.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                   C.c_int, C.c_uint64, C.c_void_p, C.c_int64, C.c_void_p]
        L.dlk_expf.restype = C.c_int
        L.dlk_expf.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]
        _LIB = L
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != DLK_OK:
        raise RuntimeError(f"{what} failed with status {rc}")
