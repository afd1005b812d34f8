"""GPU parity over the reference's whole configuration space at the boundary:
temperatures whose reciprocal is negative, zero or infinite (src/sampler.c:154
uses 1/temperature as it is), any 0 < top_k < V (src/sampler.c:166), histories
of any length (src/sampler.c:21-52), the soft-cap folded into dlk_sample
(src/core/context.c:873-876 before src/core/sampler_api.c:51-63), and drop-in
sampler objects used from two threads at once.

Token ids and rng states are compared bit for bit with the reference compiled
from its sources (oracle/_ref, through the drop-in) and with the oracle
(batched entry point).  Every case prints its name before touching the GPU.
"""
import ctypes as C
import threading

import numpy as np
import pytest

from diskllm_amd import _lib
from diskllm_amd import workloads as W
from oracle import oracle as O
from test_gpu_sampler import assert_rows_match

pytestmark = pytest.mark.gpu
REF = O.ref("strict")
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _ref_sampler_api():
    REF.sampler_create.restype = C.c_void_p
    REF.sampler_create.argtypes = [C.POINTER(O.SamplerConfig)]
    REF.sampler_free.argtypes = [C.c_void_p]
    REF.sampler_sample.restype = C.c_int
    REF.sampler_sample.argtypes = [C.c_void_p, C.c_void_p, C.c_int]


def fptr(a):
    return a.ctypes.data_as(C.c_void_p)


def _row(rng, V, kind):
    row = rng.normal(0, 3, V).astype(np.float32)
    if kind == 1:
        row = np.round(row)                                 # ties
    elif kind == 2:
        row[rng.random(V) < 0.3] = -np.inf                  # masked: +inf under a negative temperature
    return row


BOUNDARY = [(-0.5, 0, 0.9, 0.0), (-0.5, 40, 0.95, 0.0), (-2.0, 0, 1.0, 0.05), (1e-40, 0, 0.9, 0.0),
            (1e-40, 7, 1.0, 0.0), (float("inf"), 0, 0.9, 0.0), (0.8, 5000, 0.95, 0.0), (-0.7, 5000, 0.9, 0.0),
            (1.0, 100000, 0.9, 0.0), (1e-40, 5000, 0.9, 0.0), (float("inf"), 6000, 0.9, 0.0)]


@needs_ref
@pytest.mark.parametrize("V", [1000, 151936])
@pytest.mark.parametrize("cfg", BOUNDARY, ids=[f"T{c[0]}-k{c[1]}" for c in BOUNDARY])
def test_dropin_boundary_vs_reference(cuda, V, cfg):
    """sampler_sample on configurations the reference accepts but the usual
    range leaves out, two steps per row kind, against the reference's."""
    T, k, p, mp = cfg
    if k >= V:
        pytest.skip("top_k >= V is the no-top-k case")
    L = _lib.lib()
    _ref_sampler_api()
    rng = np.random.default_rng(V + k)
    seed = int(rng.integers(1, 2 ** 63))
    _announce(f"drop-in V={V} T={T} k={k} p={p} minp={mp} seed={seed}")
    cfgc = _lib.SamplerConfig(T, k, p, mp, seed)
    rcfg = O.SamplerConfig(T, k, p, mp, seed)
    s, r = L.sampler_create(C.byref(cfgc)), REF.sampler_create(C.byref(rcfg))
    assert s and r
    try:
        kinds = (0, 2) if k >= 50000 else (0, 1, 2)            # the reference sorts O(V k) on the host
        for kind in kinds:
            row = _row(rng, V, kind)
            a, b = row.copy(), row.copy()
            ta = L.sampler_sample(s, fptr(a), V)
            tb = REF.sampler_sample(r, fptr(b), V)
            assert ta == tb, (V, cfg, kind, ta, tb)
    finally:
        L.sampler_free(s)
        REF.sampler_free(r)


NAN_ROWS = ["nan-inside-k", "nan-at-k-1", "nan-at-0", "nan-past-k", "pinf", "two-nans", "all-masked-one-nan"]


@needs_ref
@pytest.mark.parametrize("V,k", [(20000, 5000), (151936, 9000)])
@pytest.mark.parametrize("kind", NAN_ROWS)
def test_nan_rows_large_k_vs_reference(cuda, V, k, kind):
    """Rows whose s = (l - max) / T holds NaN with top_k above 4096 (the
    one-thread emulation's limit): the reference's insertion sort in closed form
    (the window after the last NaN among the first k), or, with every NaN past
    the first k, the ordinary selection with NaN keys last.  Token and rng
    sequence through the drop-in against the reference build, two steps."""
    L = _lib.lib()
    _ref_sampler_api()
    rng = np.random.default_rng(V + k + len(kind))
    seed = int(rng.integers(1, 2 ** 63))
    cfgc, rcfg = _lib.SamplerConfig(0.9, k, 0.95, 0.0, seed), O.SamplerConfig(0.9, k, 0.95, 0.0, seed)
    s, r = L.sampler_create(C.byref(cfgc)), REF.sampler_create(C.byref(rcfg))
    assert s and r
    try:
        for step in range(2):
            _announce(f"NaN row V={V} k={k} kind={kind} step={step}")
            row = rng.normal(0, 3, V).astype(np.float32)
            if kind == "nan-inside-k":
                row[rng.integers(0, k - 1, 3)] = np.nan
            elif kind == "nan-at-k-1":
                row[k - 1] = np.nan
            elif kind == "nan-at-0":
                row[0] = np.nan
            elif kind == "nan-past-k":
                row[rng.integers(k, V, 5)] = np.nan
            elif kind == "pinf":
                row[rng.integers(0, V, 2)] = np.inf
            elif kind == "two-nans":
                row[[rng.integers(0, k // 2), k - 2]] = np.nan
            else:
                row[:] = -np.inf
                row[rng.integers(1, V)] = np.nan
            a, b = row.copy(), row.copy()
            ta = L.sampler_sample(s, fptr(a), V)
            tb = REF.sampler_sample(r, fptr(b), V)
            assert ta == tb, (V, k, kind, step, ta, tb)
    finally:
        L.sampler_free(s)
        REF.sampler_free(r)


def _batched(w, path=0, softcap=0.0, max_history=0):
    from diskllm_amd import api
    db = api.to_device(w)
    prm = api.params_of(w, max_history=max_history, path=path)
    prm.softcap = softcap
    api.sample(db, prm)
    return api.results(db)


@pytest.mark.parametrize("path", [0, 1])
@pytest.mark.parametrize("T,k", [(-0.6, 0), (-0.6, 50), (1e-40, 0), (float("inf"), 50), (0.7, 6000),
                                 (-1.3, 6000)])
def test_batched_boundary_vs_oracle(cuda, path, T, k):
    """dlk_sample on masked rows (C3's packed masks, 8 rows) with these
    temperatures and top-k values: ids, rng states and candidate outputs equal
    the oracle's."""
    w = W.c3(rows=8)
    w.temperature, w.top_k = T, k
    with np.errstate(over="ignore"):
        inv_t = np.float32(1.0) / np.float32(T)
    w.n_out = 16 if 0 < inv_t < np.inf else 0                # candidate outputs where they are numbers
    _announce(f"batched boundary T={T} k={k} path={path} rows={w.rows}")
    res = _batched(w, path)
    assert_rows_match(w, res, list(range(w.rows)))


@pytest.mark.parametrize("n_hist", [3000, 10000])
@pytest.mark.parametrize("k", [0, 40])
def test_long_history_vs_oracle(cuda, n_hist, k):
    """Histories longer than the fused kernels' LDS staging (penalties applied to
    a scratch copy first), with repetition, frequency and presence penalties in
    both orders: ids and rng states equal the oracle's."""
    rng = np.random.default_rng(n_hist + k)
    w = W.c2(rows=4)
    hist = [rng.integers(0, w.vocab, n_hist) if r % 2 == 0 else rng.integers(0, 500, n_hist) for r in range(w.rows)]
    w.hist_off, w.hist_ids = W._csr(hist)
    w.top_k = k
    for order in (W.ORDER_NORTH_STAR, W.ORDER_REFERENCE):
        w.order = order
        _announce(f"long history n={n_hist} k={k} order={order:#x}")
        res = _batched(w, max_history=n_hist)
        assert_rows_match(w, res, list(range(w.rows)))


@pytest.mark.parametrize("vocab,n_hist", [(32768, 1000), (151936, 1024), (151936, 700), (151936, 512),
                                          (151936, 513)])
def test_fused_history_hash(cuda, vocab, n_hist):
    """The fused full-vocabulary kernel's history table at its largest direct
    history (up to 1,024 ids; longer ones are applied to a scratch copy first):
    many repeats of few ids (long probe chains), ids on both sides of every
    slice edge, all-distinct ids; both penalty orders.  512 ids is the largest
    history of the instance that loads one id per thread, 513 the smallest of
    the one that loads two.  Ids and rng states equal the oracle's."""
    rng = np.random.default_rng(vocab + n_hist)
    w = W.c2(rows=4, vocab=vocab)
    edges = [0, vocab - 1] + [e + d for e in range(4096, vocab, 4096) for d in (-1, 0)]
    hist = []
    for r in range(w.rows):
        if r == 0:
            h = rng.integers(0, vocab, n_hist)
        elif r == 1:
            h = rng.integers(0, 40, n_hist)                   # few distinct ids, many repeats
        elif r == 2:
            e = np.array(edges[:n_hist // 2])
            h = np.concatenate([e, rng.integers(0, vocab, n_hist - len(e))])
        else:
            h = rng.permutation(vocab)[:n_hist]               # distinct ids
        hist.append(h)
    w.hist_off, w.hist_ids = W._csr(hist)
    for order in (W.ORDER_NORTH_STAR, W.ORDER_REFERENCE):
        w.order = order
        _announce(f"fused history V={vocab} n={n_hist} order={order:#x}")
        res = _batched(w, max_history=n_hist)
        assert_rows_match(w, res, list(range(w.rows)))


@pytest.mark.parametrize("path", [0, 1])
def test_softcap_param_vs_oracle(cuda, path):
    """dlk_sample with softcap 30 on C5 rows (DFA mask, repetition penalty,
    top-k 64, top-p 0.95, top-20 log-probs) and on C2 rows (full vocabulary):
    equal to the oracle's soft-cap followed by its sampling."""
    for w in (W.c5(rows=24), W.c2(rows=8)):
        _announce(f"softcap param 30 {w.name} rows={w.rows} path={path}")
        res = _batched(w, path, softcap=30.0)
        capped = w.logits.copy()
        O.lib().orc_softcap(capped.reshape(-1), capped.reshape(-1), capped.size, np.float32(30.0))
        w.logits = capped
        assert_rows_match(w, res, list(range(w.rows)))


@needs_ref
def test_dropin_two_threads(cuda):
    """Two sampler objects driven from two threads at once (the reference's
    objects are independent, each with its own state): each thread's tokens
    equal the reference's for its own sequence."""
    L = _lib.lib()
    _ref_sampler_api()
    V = 151936
    errors = []

    def worker(tid):
        try:
            rng = np.random.default_rng(100 + tid)
            T, k, p = (1.0, 0, 0.9) if tid == 0 else (0.8, 40, 0.95)
            cfgc = _lib.SamplerConfig(T, k, p, 0.0, 1000 + tid)
            s = L.sampler_create(C.byref(cfgc))
            rows = [_row(rng, V, i % 3) for i in range(24)]
            got = [L.sampler_sample(s, fptr(x.copy()), V) for x in rows]
            L.sampler_free(s)
            r = REF.sampler_create(C.byref(O.SamplerConfig(T, k, p, 0.0, 1000 + tid)))
            want = [REF.sampler_sample(r, fptr(x.copy()), V) for x in rows]
            REF.sampler_free(r)
            if got != want:
                errors.append((tid, [(i, a, b) for i, (a, b) in enumerate(zip(got, want)) if a != b][:5]))
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append((tid, repr(e)))

    _announce("drop-in from two threads, 24 steps each")
    th = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errors, errors
