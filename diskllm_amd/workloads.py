"""Synthetic workloads for the sampling / grammar-mask path (configs C1-C5).

The five configurations are the measurement contract of this package: bench.py
times C2 and the tests use all five as parity cases.  Everything is drawn from
numpy's PCG64 with a fixed seed, so a (config, seed) pair names one exact input.

Conventions the configuration text leaves open (stated once, used everywhere):
  * Zipf rank bias (C2): bias_i = -s * ln(rank_i), rank_i = perm[i] + 1 of a
    per-row random permutation; logits = N(0, sigma^2) + bias computed in float64
    and rounded once to float32.
  * Zipf history (C2): ranks drawn from Zipf(s) truncated to [1, V] by rejection,
    mapped to ids through the row's permutation, so repeats follow the Zipf law.
  * Token lengths (C4/C5): Geometric(p=1/4) (mean 4) clipped to [1, 16]; bytes
    uniform in [0, 255]; CSR = uint32 offsets[V+1] + uint8 bytes.
  * DFA (C4/C5): uint8 trans[64, 256]; state 0 is dead (row 0 all zeros); every
    other entry is 0 with probability 0.7, else uniform in [1, 63].
  * Per-row xorshift seeds: non-zero uint64 drawn from the config seed; the row's
    uniform is the first rand_f32 of that state (src/sampler.c:79-81, :225).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

# Penalty op codes packed low nibble first (same numbering as include/diskllm_amd.h).
OP_REPETITION, OP_FREQUENCY, OP_PRESENCE = 1, 2, 3


def pack_order(*ops: int) -> int:
    v = 0
    for i, op in enumerate(ops):
        v |= (op & 0xF) << (4 * i)
    return v


# North-star order (repetition -> frequency -> presence) and the reference caller
# order (presence -> repetition, src/core/sampler_api.c:55-61).
ORDER_NORTH_STAR = pack_order(OP_REPETITION, OP_FREQUENCY, OP_PRESENCE)
ORDER_REFERENCE = pack_order(OP_PRESENCE, OP_REPETITION)


@dataclass
class Workload:
    name: str
    rows: int
    vocab: int
    logits: np.ndarray                       # float32 [rows, vocab]
    seeds: np.ndarray                        # uint64 [rows]
    temperature: float = 1.0
    top_k: int = 0
    top_p: float = 1.0
    min_p: float = 0.0
    repeat_penalty: float = 1.0
    frequency_penalty: float = 0.0
    presence_penalty: float = 0.0
    order: int = ORDER_NORTH_STAR
    hist_off: Optional[np.ndarray] = None    # int32 [rows+1]
    hist_ids: Optional[np.ndarray] = None    # int32 [hist_off[-1]]
    mask: Optional[np.ndarray] = None        # uint32 [rows, ceil(V/32)] packed allow-mask
    dfa: Optional["DFA"] = None              # byte-DFA mask source
    dfa_states: Optional[np.ndarray] = None  # int32 [rows] active state per row
    n_out: int = 0                           # candidate outputs per row
    softcap: float = 0.0                     # > 0: logits capped, cap * tanhf(l / cap), before the mask
    extra: dict = field(default_factory=dict)

    @property
    def mask_words(self) -> int:
        return (self.vocab + 31) // 32


@dataclass
class DFA:
    offsets: np.ndarray   # uint32 [V+1]
    data: np.ndarray      # uint8 [offsets[-1]]
    trans: np.ndarray     # uint8 [n_states, 256]
    eos_id: int = -1
    accept: int = 0       # bit s set: EOS allowed in state s


def _row_seeds(rng: np.random.Generator, rows: int) -> np.ndarray:
    s = rng.integers(1, np.iinfo(np.uint64).max, size=rows, dtype=np.uint64, endpoint=True)
    s[s == 0] = 1
    return s


def _csr(lists) -> tuple[np.ndarray, np.ndarray]:
    off = np.zeros(len(lists) + 1, np.int32)
    off[1:] = np.cumsum([len(x) for x in lists])
    ids = np.concatenate([np.asarray(x, np.int32) for x in lists]) if lists else np.zeros(0, np.int32)
    return off, ids.astype(np.int32)


def _zipf_ranks(rng: np.random.Generator, s: float, n: int, vmax: int) -> np.ndarray:
    out = np.empty(0, np.int64)
    while out.size < n:
        z = rng.zipf(s, size=2 * n)
        out = np.concatenate([out, z[z <= vmax]])
    return out[:n]


def make_tokens(rng: np.random.Generator, vocab: int, max_len: int = 16, p: float = 0.25):
    lens = np.minimum(rng.geometric(p, size=vocab), max_len).astype(np.uint32)
    off = np.zeros(vocab + 1, np.uint32)
    off[1:] = np.cumsum(lens, dtype=np.uint64).astype(np.uint32)
    data = rng.integers(0, 256, size=int(off[-1]), dtype=np.uint8)
    return off, data


def make_dfa_table(rng: np.random.Generator, n_states: int = 64, dead_frac: float = 0.7) -> np.ndarray:
    t = rng.integers(1, n_states, size=(n_states, 256), dtype=np.uint8)
    t[rng.random((n_states, 256)) < dead_frac] = 0
    t[0, :] = 0
    return t


def c1(seed: int = 1) -> Workload:
    """Single row, Llama-3.2 vocab: N(0,3^2), 20 ids +8, rep 1.1 over 64 ids,
    T 0.8, top-k 40, top-p 0.95; outputs the token and the 40 candidate probs."""
    rng = np.random.Generator(np.random.PCG64(seed))
    V = 128256
    lg = rng.normal(0.0, 3.0, size=(1, V)).astype(np.float32)
    boost = rng.choice(V, 20, replace=False)
    lg[0, boost] += np.float32(8.0)
    off, ids = _csr([rng.integers(0, V, 64)])
    return Workload("C1", 1, V, lg, _row_seeds(rng, 1), temperature=0.8, top_k=40, top_p=0.95,
                    repeat_penalty=1.1, order=ORDER_REFERENCE, hist_off=off, hist_ids=ids, n_out=40)


def c2(seed: int = 2, rows: int = 64, vocab: int = 151936) -> Workload:
    """Batch-64 Qwen vocab nucleus sampling: N(0,2^2) + Zipf(1.1) rank bias;
    rep 1.15 / freq 0.3 / pres 0.5 over a 256-id Zipf history; T 1.0, top-p 0.9,
    no top-k (index-order nucleus, src/sampler.c:165-170, :205-216)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    V = vocab
    lg = np.empty((rows, V), np.float32)
    hist = []
    for r in range(rows):
        perm = rng.permutation(V)
        bias = -1.1 * np.log(perm.astype(np.float64) + 1.0)
        lg[r] = (rng.normal(0.0, 2.0, size=V) + bias).astype(np.float32)
        by_rank = np.argsort(perm)
        hist.append(by_rank[_zipf_ranks(rng, 1.1, 256, V) - 1])
    off, ids = _csr(hist)
    return Workload("C2", rows, V, lg, _row_seeds(rng, rows), temperature=1.0, top_k=0, top_p=0.9,
                    repeat_penalty=1.15, frequency_penalty=0.3, presence_penalty=0.5,
                    order=ORDER_NORTH_STAR, hist_off=off, hist_ids=ids)


def c3(seed: int = 3, rows: int = 32, vocab: int = 151936) -> Workload:
    """Batch-32 packed-mask sampling: N(0,3^2), ~2% allowed bits per row (row 3
    allows exactly one token), T 0.7, top-k 50, top-p 0.95."""
    rng = np.random.Generator(np.random.PCG64(seed))
    V = vocab
    W = (V + 31) // 32
    lg = rng.normal(0.0, 3.0, size=(rows, V)).astype(np.float32)
    mask = np.zeros((rows, W), np.uint32)
    for r in range(rows):
        n = 1 if r == 3 else int(round(0.02 * V))
        pos = rng.choice(V, n, replace=False)
        np.bitwise_or.at(mask[r], pos >> 5, (np.uint32(1) << (pos & 31).astype(np.uint32)))
    return Workload("C3", rows, V, lg, _row_seeds(rng, rows), temperature=0.7, top_k=50, top_p=0.95,
                    mask=mask, n_out=50)


def c4(seed: int = 4, rows: int = 16, vocab: int = 151936) -> Workload:
    """Per-token DFA validity mask: 151936 CSR tokens, 64-state byte DFA, 16 rows."""
    rng = np.random.Generator(np.random.PCG64(seed))
    off, data = make_tokens(rng, vocab)
    trans = make_dfa_table(rng)
    states = rng.integers(1, 64, size=rows).astype(np.int32)
    return Workload("C4", rows, vocab, np.zeros((rows, 0), np.float32), _row_seeds(rng, rows),
                    dfa=DFA(off, data, trans), dfa_states=states)


def c5(seed: int = 5, rows: int = 512, vocab: int = 262144) -> Workload:
    """Batch-512 Gemma vocab decode step: N(0,2.5^2), DFA mask (512 active
    states), rep 1.1 over 128 ids, T 1.0, top-k 64, top-p 0.95, top-20 log-probs."""
    rng = np.random.Generator(np.random.PCG64(seed))
    V = vocab
    lg = np.empty((rows, V), np.float32)
    for r in range(rows):
        lg[r] = rng.normal(0.0, 2.5, size=V).astype(np.float32)
    off, data = make_tokens(rng, V)
    trans = make_dfa_table(rng)
    states = rng.integers(1, 64, size=rows).astype(np.int32)
    hoff, hids = _csr([rng.integers(0, V, 128) for _ in range(rows)])
    return Workload("C5", rows, V, lg, _row_seeds(rng, rows), temperature=1.0, top_k=64, top_p=0.95,
                    repeat_penalty=1.1, order=ORDER_REFERENCE, hist_off=hoff, hist_ids=hids,
                    dfa=DFA(off, data, trans), dfa_states=states, n_out=20)


CAP_C5CAP = 30.0


def c5cap(seed: int = 5, rows: int = 512, vocab: int = 262144) -> Workload:
    """C5's decode step with the reference's final-logit soft-cap in front:
    cap * tanhf(l / cap), cap 30 (the Gemma cap), then mask, penalties and sampling
    as in C5; 512 x 262144 fp32."""
    w = c5(seed, rows, vocab)
    w.name = "C5CAP"
    w.softcap = CAP_C5CAP
    return w


def cap(seed: int = 5, rows: int = 512, vocab: int = 262144) -> Workload:
    """The reference's decode epilogue alone on C5's logits: soft-cap
    cap * tanhf(x / cap) with cap 30, in place, 512 x 262144 fp32."""
    w = c5(seed, rows, vocab)
    w.name = "CAP"
    return w


CONFIGS = {"C1": c1, "C2": c2, "C3": c3, "C4": c4, "C5": c5, "C5CAP": c5cap, "CAP": cap}
