"""ctypes bindings for the checker.  TEST INFRASTRUCTURE ONLY.

Loads oracle/_build/liboracle.so (the C restatement in oracle.c) and, when built,
oracle/_ref/libref_{strict,fast}.so (the reference's own src/sampler.c and
src/core/grammar.c compiled from its sources).  Only tests/, the smoke check and
bench.py's cpu_baseline leg import this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(HERE, "_build")
REF = os.path.join(HERE, "_ref")

OP_REPETITION, OP_FREQUENCY, OP_PRESENCE = 1, 2, 3

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


class OrcCfg(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float)]


class OrcTrace(C.Structure):
    _fields_ = [("idx", C.POINTER(C.c_int)), ("val", C.POINTER(C.c_float)), ("p", C.POINTER(C.c_float)),
                ("greedy", C.c_int), ("k", C.c_int), ("k_minp", C.c_int), ("nk", C.c_int), ("pos", C.c_int),
                ("r", C.c_float), ("inv_sum", C.c_float), ("inv_s2", C.c_float), ("inv_s3", C.c_float),
                ("sum", C.c_double), ("s2", C.c_double), ("s3", C.c_double)]


class OrcGrammar(C.Structure):
    _fields_ = [("buf", C.c_char * 8192), ("len", C.c_int), ("is_json", C.c_bool), ("is_receipt", C.c_bool)]


class SamplerConfig(C.Structure):
    """include/sampler.h:10-16."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("seed", C.c_uint64)]


def build(quiet: bool = True) -> None:
    subprocess.run(["make", "-C", HERE, "-s"], check=True,
                   stdout=subprocess.DEVNULL if quiet else None)


_LIB: Optional[C.CDLL] = None
_REFS: dict = {}


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(BUILD, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        L.orc_seed_state.restype = C.c_uint64
        L.orc_seed_state.argtypes = [C.c_uint64]
        L.orc_xorshift64.restype = C.c_uint64
        L.orc_xorshift64.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_rand_f32.restype = C.c_float
        L.orc_rand_f32.argtypes = [C.POINTER(C.c_uint64)]
        L.orc_greedy.argtypes = [_f32p, C.c_int]
        for fn in ("orc_repetition", "orc_presence", "orc_frequency"):
            getattr(L, fn).argtypes = [_f32p, C.c_int, _i32p, C.c_int, C.c_float]
        L.orc_penalties.argtypes = [_f32p, C.c_int, _i32p, C.c_int, C.c_uint32, C.c_float, C.c_float, C.c_float]
        L.orc_apply_packed_mask.argtypes = [_f32p, C.c_int, _u32p]
        L.orc_sample.argtypes = [C.POINTER(OrcCfg), C.POINTER(C.c_uint64), _f32p, C.c_int, C.POINTER(OrcTrace)]
        L.orc_dfa_mask.argtypes = [_u32p, _u8p, C.c_int, _u8p, C.c_int, C.c_int, C.c_uint64, _u32p]
        L.orc_receipt_prefix.restype = C.c_bool
        L.orc_receipt_prefix.argtypes = [C.c_char_p, C.c_int]
        L.orc_json_prefix.restype = C.c_bool
        L.orc_json_prefix.argtypes = [C.c_char_p, C.c_int]
        L.orc_expf_bits.argtypes = [C.c_uint32, C.c_long, _f32p, C.c_int]
        L.orc_softcap.argtypes = [_f32p, _f32p, C.c_long, C.c_float]
        L.orc_tanhf_bits.argtypes = [C.c_uint32, C.c_long, _f32p, C.c_int]
        L.orc_grammar_init.argtypes = [C.POINTER(OrcGrammar), C.c_char_p]
        L.orc_grammar_accept.restype = C.c_bool
        L.orc_grammar_accept.argtypes = [C.POINTER(OrcGrammar), C.c_char_p]
        L.orc_grammar_advance.argtypes = [C.POINTER(OrcGrammar), C.c_char_p]
        L.orc_grammar_finished.restype = C.c_bool
        L.orc_grammar_finished.argtypes = [C.POINTER(OrcGrammar)]
        L.orc_grammar_mask.argtypes = [C.POINTER(OrcGrammar), _f32p, C.c_int, _u32p, _u8p, C.c_int]
        _LIB = L
    return _LIB


def ref(kind: str = "strict") -> Optional[C.CDLL]:
    """The reference build (kind 'strict' or 'fast'), or None if not built."""
    if kind not in _REFS:
        path = os.path.join(REF, f"libref_{kind}.so")
        if not os.path.exists(path):
            return None
        L = C.CDLL(path)
        L.refh_sample_trace.argtypes = [C.POINTER(SamplerConfig), C.POINTER(C.c_uint64), _f32p, C.c_int, C.c_int,
                                        _i32p, _f32p]
        L.refh_time_batch.argtypes = [_f32p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                      C.c_uint32, C.c_float, C.c_float, C.c_float, C.POINTER(SamplerConfig),
                                      _u64p, C.c_int, C.c_int, _f64p, _i32p]
        L.refh_expf_many.argtypes = [_f32p, _f32p, C.c_long]
        L.refh_softcap.argtypes = [_f32p, C.c_int, C.c_float]
        L.sampler_apply_repetition_penalty.argtypes = [_f32p, C.c_int, _i32p, C.c_int, C.c_float]
        L.sampler_apply_presence_penalty.argtypes = [_f32p, C.c_int, _i32p, C.c_int, C.c_float]
        L.greedy_sample.argtypes = [_f32p, C.c_int]
        L.diskllm_grammar_init_from_str.restype = C.c_void_p
        L.diskllm_grammar_init_from_str.argtypes = [C.c_char_p]
        L.diskllm_grammar_init_json.restype = C.c_void_p
        L.diskllm_grammar_free.argtypes = [C.c_void_p]
        L.diskllm_grammar_reset.argtypes = [C.c_void_p]
        L.diskllm_grammar_accept_str.restype = C.c_bool
        L.diskllm_grammar_accept_str.argtypes = [C.c_void_p, C.c_char_p]
        L.diskllm_grammar_advance.argtypes = [C.c_void_p, C.c_char_p]
        L.diskllm_grammar_is_finished.restype = C.c_bool
        L.diskllm_grammar_is_finished.argtypes = [C.c_void_p]
        L.diskllm_grammar_apply_mask.argtypes = [C.c_void_p, _f32p, C.c_int, C.c_void_p, C.c_void_p, C.c_int]
        _REFS[kind] = L
    return _REFS[kind]


# ---------------------------------------------------------------------------- rows

def rand_f32(state: int) -> tuple[float, int]:
    s = C.c_uint64(state)
    r = lib().orc_rand_f32(C.byref(s))
    return float(np.float32(r)), int(s.value)


def penalties(row: np.ndarray, hist: Optional[np.ndarray], order: int, rep: float, freq: float,
              pres: float) -> np.ndarray:
    out = np.ascontiguousarray(row, np.float32).copy()
    if hist is not None and len(hist):
        h = np.ascontiguousarray(hist, np.int32)
        lib().orc_penalties(out, out.size, h, h.size, order, rep, freq, pres)
    return out


def dfa_mask(dfa, state: int, vocab: Optional[int] = None) -> np.ndarray:
    V = len(dfa.offsets) - 1 if vocab is None else vocab
    out = np.zeros((V + 31) // 32, np.uint32)
    lib().orc_dfa_mask(np.ascontiguousarray(dfa.offsets, np.uint32), np.ascontiguousarray(dfa.data, np.uint8), V,
                       np.ascontiguousarray(dfa.trans, np.uint8), int(state), int(dfa.eos_id),
                       int(dfa.accept) & 0xFFFFFFFFFFFFFFFF, out)
    return out


def row_mask(w, r: int) -> Optional[np.ndarray]:
    if w.mask is not None:
        return np.ascontiguousarray(w.mask[r])
    if w.dfa is not None and w.dfa_states is not None:
        return dfa_mask(w.dfa, int(w.dfa_states[r]), w.vocab)
    return None


def prepared_row(w, r: int) -> np.ndarray:
    """Row r after the soft-cap (if the workload has one, src/core/context.c:873-876),
    the mask and the penalties: the logits sampler_sample sees
    (src/core/sampler_api.c:51-61, with the configured penalty order)."""
    row = np.ascontiguousarray(w.logits[r], np.float32).copy()
    if getattr(w, "softcap", 0.0) > 0.0:
        lib().orc_softcap(row, row, row.size, np.float32(w.softcap))
    m = row_mask(w, r)
    if m is not None:
        lib().orc_apply_packed_mask(row, row.size, m)
    hist = None
    if w.hist_ids is not None:
        hist = w.hist_ids[w.hist_off[r]:w.hist_off[r + 1]]
    return penalties(row, hist, w.order, w.repeat_penalty, w.frequency_penalty, w.presence_penalty)


def sample_row(row: np.ndarray, state: int, temperature: float, top_k: int, top_p: float, min_p: float,
               want_p: int = 0) -> dict:
    """orc_sample on one prepared row; returns token, new rng state and the trace."""
    V = row.size
    idx = np.zeros(V, np.int32)
    val = np.zeros(V, np.float32)
    p = np.zeros(V, np.float32)
    tr = OrcTrace()
    tr.idx = idx.ctypes.data_as(C.POINTER(C.c_int))
    tr.val = val.ctypes.data_as(C.POINTER(C.c_float))
    tr.p = p.ctypes.data_as(C.POINTER(C.c_float))
    cfg = OrcCfg(temperature, top_k, top_p, min_p)
    s = C.c_uint64(state)
    tok = lib().orc_sample(C.byref(cfg), C.byref(s), np.ascontiguousarray(row, np.float32), V, C.byref(tr))
    n = min(want_p, tr.k) if want_p else 0
    return dict(token=int(tok), state=int(s.value), greedy=tr.greedy, k=tr.k, k_minp=tr.k_minp, nk=tr.nk,
                pos=tr.pos, r=tr.r, inv_sum=tr.inv_sum, inv_s2=tr.inv_s2, inv_s3=tr.inv_s3, sum=tr.sum,
                s2=tr.s2, s3=tr.s3, cand_idx=idx[:n].copy(), cand_p=p[:n].copy(), final=val.copy(),
                final_idx=idx.copy())


def run_workload(w, rows: Optional[list] = None) -> dict:
    """The oracle on every (or the listed) row of a workload."""
    rows = list(range(w.rows)) if rows is None else rows
    ids, states, cand_idx, cand_p = [], [], [], []
    for r in rows:
        out = sample_row(prepared_row(w, r), int(w.seeds[r]), w.temperature, w.top_k, w.top_p, w.min_p,
                         want_p=w.n_out)
        ids.append(out["token"])
        states.append(out["state"])
        ci = np.full(w.n_out, -1, np.int32)
        cp = np.zeros(w.n_out, np.float32)
        ci[:len(out["cand_idx"])] = out["cand_idx"]
        cp[:len(out["cand_p"])] = out["cand_p"]
        cand_idx.append(ci)
        cand_p.append(cp)
    return dict(ids=np.array(ids, np.int32), states=np.array(states, np.uint64),
                cand_idx=np.array(cand_idx, np.int32).reshape(len(rows), w.n_out),
                cand_p=np.array(cand_p, np.float32).reshape(len(rows), w.n_out))


def ref_sample_row(kind: str, row: np.ndarray, state: int, temperature: float, top_k: int, top_p: float,
                   min_p: float, n_trace: int = 0) -> tuple[int, int, np.ndarray, np.ndarray]:
    """The reference sampler_sample (compiled from its sources) on one prepared row."""
    L = ref(kind)
    cfg = SamplerConfig(temperature, top_k, top_p, min_p, 1)
    s = C.c_uint64(state)
    n = max(n_trace, 1)
    oi = np.zeros(n, np.int32)
    ov = np.zeros(n, np.float32)
    work = np.ascontiguousarray(row, np.float32).copy()
    tok = L.refh_sample_trace(C.byref(cfg), C.byref(s), work, work.size, n_trace, oi, ov)
    return int(tok), int(s.value), oi[:n_trace], ov[:n_trace]


# ------------------------------------------------------------------------- grammar

def grammar(text: Optional[bytes]) -> OrcGrammar:
    g = OrcGrammar()
    lib().orc_grammar_init(C.byref(g), text)
    return g


def grammar_mask(g: OrcGrammar, offsets: np.ndarray, data: np.ndarray, eos_id: int,
                 logits: Optional[np.ndarray] = None) -> tuple[np.ndarray, int]:
    """orc_grammar_mask over a CSR vocabulary: the masked logits and the valid count."""
    V = len(offsets) - 1
    lg = np.zeros(V, np.float32) if logits is None else np.ascontiguousarray(logits, np.float32).copy()
    n = lib().orc_grammar_mask(C.byref(g), lg, V, np.ascontiguousarray(offsets, np.uint32),
                               np.ascontiguousarray(data, np.uint8), int(eos_id))
    return lg, int(n)
