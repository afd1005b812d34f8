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
DLK_ERR_FORMAT = -4
DLK_STATUS_HISTORY_TOO_LONG = 1
DLK_STATUS_SYNC_TIMEOUT = 2
DLK_STATUS_UNSUPPORTED_ROW = 4
PATH_AUTO, PATH_ROW, PATH_FULL_EXACT, PATH_FULL_NO_WAIT = 0, 1, 2, 3

OP_REPETITION, OP_FREQUENCY, OP_PRESENCE = 1, 2, 3
ORDER_REFERENCE = OP_PRESENCE | (OP_REPETITION << 4)
ORDER_REP_FREQ_PRES = OP_REPETITION | (OP_FREQUENCY << 4) | (OP_PRESENCE << 8)


class SampleParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("frequency_penalty", C.c_float), ("presence_penalty", C.c_float),
                ("penalty_order", C.c_uint32), ("max_history", C.c_int), ("n_out", C.c_int),
                ("path", C.c_int), ("softcap", C.c_float)]


class Batch(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("ld", C.c_int64), ("hist_off", C.c_void_p), ("hist_ids", C.c_void_p),
                ("mask", C.c_void_p), ("mask_ld", C.c_int64), ("mask_row", C.c_void_p), ("rng", C.c_void_p),
                ("out_ids", C.c_void_p), ("out_cand_ids", C.c_void_p), ("out_cand_probs", C.c_void_p),
                ("out_cand_logprobs", C.c_void_p), ("status", C.c_void_p)]


class SamplerConfig(C.Structure):
    """include/sampler.h:10-16."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("seed", C.c_uint64)]


GRAMMAR_NONE, GRAMMAR_JSON, GRAMMAR_RECEIPT = 0, 1, 2


class ScanState(C.Structure):
    _fields_ = [("mode", C.c_int32), ("pc", C.c_int32), ("n", C.c_int32), ("m", C.c_int32), ("prev", C.c_uint8),
                ("flag", C.c_uint8), ("pad", C.c_uint8 * 2)]


class BalanceState(C.Structure):
    _fields_ = [("braces", C.c_int32), ("brackets", C.c_int32), ("len", C.c_int32), ("in_str", C.c_uint8),
                ("prev", C.c_uint8), ("pad", C.c_uint8 * 2)]


class GrammarRow(C.Structure):
    """dlk_grammar_row (include/diskllm_amd.h)."""
    _fields_ = [("scan", ScanState), ("bal", BalanceState)]


class CsrVocab(C.Structure):
    """dlk_csr_vocab (include/diskllm_amd.h)."""
    _fields_ = [("off", C.c_void_p), ("bytes", C.c_void_p), ("vocab", C.c_int), ("scratch", C.c_void_p),
                ("scratch_cap", C.c_int)]


# Every symbol the public headers declare (checked by the CPU test suite).
EXPORTS = [
    # include/diskllm_amd.h
    "dlk_seed_state", "dlk_sample", "dlk_sample_noalloc", "dlk_release_stream", "dlk_dfa_mask", "dlk_expf", "dlk_apply_penalties", "dlk_grammar_mode_of",
    "dlk_grammar_row_init", "dlk_grammar_row_feed", "dlk_grammar_mask", "dlk_grammar_advance", "dlk_sample_grammar",
    "dlk_vocab_csr_from_gguf", "dlk_csr_token_str", "dlk_softcap",
    # include/sampler.h
    "sampler_create", "sampler_free", "sampler_apply_repetition_penalty", "sampler_apply_presence_penalty",
    "sampler_sample", "greedy_sample",
    # include/grammar.h
    "diskllm_grammar_init_from_file", "diskllm_grammar_init_from_str", "diskllm_grammar_init_json",
    "diskllm_grammar_free", "diskllm_grammar_reset", "diskllm_grammar_accept_str", "diskllm_grammar_advance",
    "diskllm_grammar_is_finished", "diskllm_grammar_apply_mask",
]


def source_stamp() -> str:
    """First 16 hex digits of a SHA-256 over the library's sources (csrc/hip,
    csrc/host, the Makefile, the export map and include/*.h, by relative path
    and content): the build a measurement was taken on.  Committed profile
    summaries record it, so a figure is only reused for the sources it measured."""
    import glob
    import hashlib
    h = hashlib.sha256()
    root = os.path.dirname(HERE)
    files = sorted(glob.glob(os.path.join(CSRC, "hip", "*")) + glob.glob(os.path.join(CSRC, "host", "*")) +
                   [os.path.join(CSRC, "Makefile"), os.path.join(CSRC, "exports.map")] +
                   glob.glob(os.path.join(root, "include", "*.h")))
    for f in files:
        if os.path.isfile(f):
            h.update(os.path.relpath(f, root).encode() + b"\0")
            with open(f, "rb") as fh:
                h.update(fh.read())
            h.update(b"\0")
    return h.hexdigest()[:16]


def build(quiet: bool = True) -> None:
    """Compile every HIP source for gfx950 and link the shared library in-tree
    (always from scratch: every call compiles, also over an existing build)."""
    jobs = str(min(16, len(os.sched_getaffinity(0)) or 4))
    r = subprocess.run(["make", "-B", "-C", CSRC, "-j", jobs], capture_output=True, text=True)
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
        L.dlk_sample_noalloc.restype = C.c_int
        L.dlk_sample_noalloc.argtypes = [C.POINTER(Batch), C.c_int, C.c_int, C.POINTER(SampleParams), C.c_void_p]
        L.dlk_release_stream.restype = C.c_int
        L.dlk_release_stream.argtypes = [C.c_void_p]
        L.dlk_dfa_mask.restype = C.c_int
        L.dlk_dfa_mask.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                   C.c_int, C.c_uint64, C.c_void_p, C.c_int64, C.c_void_p]
        L.dlk_expf.restype = C.c_int
        L.dlk_expf.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]
        L.dlk_apply_penalties.restype = C.c_int
        L.dlk_apply_penalties.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                          C.c_uint32, C.c_float, C.c_float, C.c_float, C.c_void_p]
        L.dlk_grammar_mode_of.restype = C.c_int
        L.dlk_grammar_mode_of.argtypes = [C.c_char_p]
        L.dlk_grammar_row_init.argtypes = [C.POINTER(GrammarRow), C.c_int]
        L.dlk_grammar_row_feed.argtypes = [C.POINTER(GrammarRow), C.c_char_p, C.c_int]
        L.dlk_grammar_mask.restype = C.c_int
        L.dlk_grammar_mask.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                       C.c_int64, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p]
        L.dlk_grammar_advance.restype = C.c_int
        L.dlk_grammar_advance.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                          C.c_void_p]
        L.dlk_sample_grammar.restype = C.c_int
        L.dlk_sample_grammar.argtypes = [C.POINTER(Batch), C.c_int, C.c_int, C.POINTER(SampleParams), C.c_void_p,
                                         C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]
        L.dlk_softcap.restype = C.c_int
        L.dlk_softcap.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_float, C.c_void_p]
        L.dlk_vocab_csr_from_gguf.restype = C.c_int
        L.dlk_vocab_csr_from_gguf.argtypes = [C.c_char_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int64,
                                              C.POINTER(C.c_int32), C.POINTER(C.c_int64)]
        # include/sampler.h
        L.sampler_create.restype = C.c_void_p
        L.sampler_create.argtypes = [C.POINTER(SamplerConfig)]
        L.sampler_free.argtypes = [C.c_void_p]
        L.sampler_sample.restype = C.c_int
        L.sampler_sample.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
        L.greedy_sample.restype = C.c_int
        L.greedy_sample.argtypes = [C.c_void_p, C.c_int]
        for fn in ("sampler_apply_repetition_penalty", "sampler_apply_presence_penalty"):
            getattr(L, fn).argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_float]
        # include/grammar.h
        for fn in ("diskllm_grammar_init_from_file", "diskllm_grammar_init_from_str"):
            getattr(L, fn).restype = C.c_void_p
            getattr(L, fn).argtypes = [C.c_char_p]
        L.diskllm_grammar_init_json.restype = C.c_void_p
        L.diskllm_grammar_init_json.argtypes = []
        L.diskllm_grammar_free.argtypes = [C.c_void_p]
        L.diskllm_grammar_reset.argtypes = [C.c_void_p]
        L.diskllm_grammar_accept_str.restype = C.c_bool
        L.diskllm_grammar_accept_str.argtypes = [C.c_void_p, C.c_char_p]
        L.diskllm_grammar_advance.argtypes = [C.c_void_p, C.c_char_p]
        L.diskllm_grammar_is_finished.restype = C.c_bool
        L.diskllm_grammar_is_finished.argtypes = [C.c_void_p]
        L.dlk_csr_token_str.restype = C.c_char_p
        L.dlk_csr_token_str.argtypes = [C.c_void_p, C.c_int]
        L.diskllm_grammar_apply_mask.restype = C.c_int
        L.diskllm_grammar_apply_mask.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_int]
        _LIB = L
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != DLK_OK:
        raise RuntimeError(f"{what} failed with status {rc}")


def vocab_csr_from_gguf(path: str, vocab: int = 0):
    """(off uint32[ids+1], bytes uint8[n], n_tokens) of a GGUF file's token
    strings, through dlk_vocab_csr_from_gguf's sizing and filling calls."""
    import numpy as np
    L = lib()
    nt, nb = C.c_int32(0), C.c_int64(0)
    p = os.fsencode(path)
    check(L.dlk_vocab_csr_from_gguf(p, vocab, None, None, 0, C.byref(nt), C.byref(nb)), "dlk_vocab_csr_from_gguf")
    ids = vocab if vocab > 0 else nt.value
    off = np.zeros(ids + 1, np.uint32)
    data = np.zeros(max(nb.value, 1), np.uint8)
    check(L.dlk_vocab_csr_from_gguf(p, vocab, off.ctypes.data, data.ctypes.data, data.size, C.byref(nt),
                                    C.byref(nb)), "dlk_vocab_csr_from_gguf")
    return off, data[:nb.value], nt.value
