"""CPU checks of the oracle (oracle/oracle.c), which the GPU parity tests trust.

Each part of the oracle is pinned by something other than a retyping of its own
formula: a closed form computed here from the definition, a brute force on tiny
inputs, the reference's own grammar unit test (tools/test_grammar_unit.c:17-24),
and -- where oracle/_ref was built from the reference sources -- a differential
test against the reference compiled as it lies (src/sampler.c, src/core/grammar.c).
"""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from diskllm_amd import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_STRICT = O.ref("strict")
needs_ref = pytest.mark.skipif(REF_STRICT is None, reason="oracle/_ref not built (no reference tree here)")

M64 = (1 << 64) - 1


# --------------------------------------------------------------------------- A2

def xorshift_py(x: int) -> int:
    x ^= (x << 13) & M64
    x ^= x >> 7
    x ^= (x << 17) & M64
    return x & M64


def f32_rne_of_int(v: int) -> np.float32:
    """The float32 nearest to the integer v (ties to even), by integer arithmetic."""
    if v == 0:
        return np.float32(0.0)
    e = v.bit_length() - 24
    if e <= 0:
        return np.float32(v)
    q, rem = divmod(v, 1 << e)
    half = 1 << (e - 1)
    if rem > half or (rem == half and q & 1):
        q += 1
    return np.float32(np.ldexp(np.float64(q), e))


def rand_py(state: int) -> tuple[np.float32, int]:
    x = xorshift_py(state)
    return np.float32(f32_rne_of_int(x >> 11) * np.float32(2.0 ** -53)), x


def unxorshift(y: int) -> int:
    """Inverse of xorshift_py (each xor-shift step is a bijection)."""
    def inv_left(y, s):
        x = y
        for _ in range(64 // s + 1):
            x = y ^ ((x << s) & M64)
        return x

    def inv_right(y, s):
        x = y
        for _ in range(64 // s + 1):
            x = y ^ (x >> s)
        return x
    return inv_left(inv_right(inv_left(y, 17), 7), 13)


def test_xorshift_and_rand_closed_form():
    L = O.lib()
    assert L.orc_seed_state(0) == 0xDEADBEEF12345678          # src/sampler.c:87
    assert L.orc_seed_state(12345) == 12345
    rng = np.random.default_rng(1)
    for s in list(rng.integers(1, 2 ** 63, 2000, dtype=np.uint64)) + [1, 2, M64, 0xDEADBEEF12345678]:
        s = int(s)
        r, st = O.rand_f32(s)
        rp, stp = rand_py(s)
        assert st == stp and np.float32(r) == rp, (hex(s), r, rp)
    # the u64 -> f32 conversion rounds: r == 1.0 is reachable, r == 0 only from x>>11 == 0
    for top in (M64, (1 << 64) - (1 << 39), ((1 << 53) - (1 << 28)) << 11):
        s = unxorshift(top)
        assert xorshift_py(s) == top
        r, _ = O.rand_f32(s)
        assert r == 1.0, (hex(top), r)
    s = unxorshift(((1 << 53) - (1 << 28) - 1) << 11)              # just below the rounding boundary
    assert O.rand_f32(s)[0] < 1.0
    s = unxorshift(0x7FF)                                          # x >> 11 == 0
    assert O.rand_f32(s)[0] == 0.0


# --------------------------------------------------------------------------- A3

def test_greedy_is_first_argmax():
    L = O.lib()
    rng = np.random.default_rng(2)
    for V in (1, 2, 5, 1000):
        for _ in range(50):
            x = np.round(rng.normal(0, 1, V) * 2).astype(np.float32) / 2    # many ties
            assert L.orc_greedy(x, V) == int(np.argmax(x))
    x = np.array([np.nan, 1.0, 5.0], np.float32)
    assert L.orc_greedy(x, 3) == 0                                  # src/sampler.c:11-17
    x = np.full(7, -np.inf, np.float32)
    assert L.orc_greedy(x, 7) == 0
    if REF_STRICT is not None:
        for _ in range(100):
            x = np.round(rng.normal(0, 1, 300)).astype(np.float32)
            assert REF_STRICT.greedy_sample(x, x.size) == L.orc_greedy(x, x.size)


# ------------------------------------------------------------------------ A4-A6

def penalties_py(row, hist, order, rep, freq, pres):
    out = row.astype(np.float32).copy()
    V = out.size
    ids, counts = np.unique(np.asarray([h for h in hist if 0 <= h < V], np.int64), return_counts=True)
    for s in range(8):
        op = (order >> (4 * s)) & 0xF
        if op == 0:
            break
        for t, c in zip(ids, counts):
            x = out[t]
            if op == W.OP_REPETITION and rep > 1.0:
                for _ in range(c):
                    x = np.float32(x * np.float32(rep)) if x < 0 else np.float32(x / np.float32(rep))
            elif op == W.OP_FREQUENCY and freq != 0.0:
                x = np.float32(x - np.float32(np.float32(freq) * np.float32(c)))
            elif op == W.OP_PRESENCE and pres != 0.0:
                x = np.float32(x - np.float32(pres))
            out[t] = x
    return out


@pytest.mark.parametrize("order", [W.ORDER_REFERENCE, W.ORDER_NORTH_STAR,
                                   W.pack_order(W.OP_FREQUENCY, W.OP_PRESENCE, W.OP_REPETITION)])
def test_penalties_closed_form(order):
    rng = np.random.default_rng(order)
    for V, n in ((10, 40), (1000, 256), (50000, 300)):
        row = rng.normal(0, 3, V).astype(np.float32)
        hist = list(rng.integers(-3, V + 3, n)) + [0, 0, V - 1]
        got = O.penalties(row, np.array(hist, np.int32), order, 1.3, 0.25, -0.6)
        np.testing.assert_array_equal(got, penalties_py(row, hist, order, 1.3, 0.25, -0.6))


@needs_ref
def test_penalties_vs_reference():
    """Repetition and presence against the reference functions (src/sampler.c:21-52)."""
    rng = np.random.default_rng(3)
    for V, n in ((50, 100), (151936, 256)):
        row = rng.normal(0, 2, V).astype(np.float32)
        hist = rng.integers(-2, V + 2, n).astype(np.int32)
        a = row.copy()
        REF_STRICT.sampler_apply_presence_penalty(a, V, hist, n, np.float32(0.5))
        REF_STRICT.sampler_apply_repetition_penalty(a, V, hist, n, np.float32(1.15))
        np.testing.assert_array_equal(a, O.penalties(row, hist, W.ORDER_REFERENCE, 1.15, 0.0, 0.5))


# ---------------------------------------------------------------------- A7-A12

def test_top_k_is_order_statistic():
    """The k candidates are the first k under (s desc, index asc), by brute force."""
    rng = np.random.default_rng(4)
    for V in (1, 3, 17, 64, 200):
        for k in (1, 2, 5, 16):
            if k >= V:
                continue
            row = (rng.integers(-3, 4, V) * 0.5).astype(np.float32)        # heavy ties
            o = O.sample_row(row, 99, 0.8, k, 1.0, 0.0, want_p=k)
            s = (row - row.max()) * np.float32(1.0 / np.float32(0.8))
            order = np.lexsort((np.arange(V), -s))[:k]
            np.testing.assert_array_equal(o["cand_idx"], order)


def test_sampling_invariants():
    rng = np.random.default_rng(5)
    for _ in range(30):
        V = int(rng.integers(2, 3000))
        row = rng.normal(0, 2, V).astype(np.float32)
        o = O.sample_row(row, int(rng.integers(1, 2 ** 62)), 1.0, 1, 0.9, 0.0)
        assert o["token"] == int(np.argmax(row))                      # top_k = 1 -> argmax
        one = np.full(V, -np.inf, np.float32)
        t = int(rng.integers(0, V))
        one[t] = 0.5
        for k in (0, 5):
            o = O.sample_row(one, int(rng.integers(1, 2 ** 62)), 0.7, k, 0.95, 0.0)
            assert o["token"] == t                                    # a single allowed token is returned
        o = O.sample_row(row, int(rng.integers(1, 2 ** 62)), 1.3, 0, 1.0, 0.0, want_p=V)
        assert abs(float(np.sum(o["cand_p"], dtype=np.float64)) - 1.0) < 1e-4
    # r == 0 returns the first candidate with q > 0
    s = unxorshift(0x7FF)
    row = np.array([-np.inf, 1.0, 2.0, 0.5], np.float32)
    assert O.sample_row(row, s, 1.0, 0, 1.0, 0.0)["token"] == 1
    # temperature 0 is greedy and consumes no random number (src/sampler.c:140-142)
    o = O.sample_row(row, 77, 0.0, 0, 0.9, 0.0)
    assert o["token"] == 2 and o["state"] == 77


def _configs():
    rng = np.random.default_rng(6)
    out = []
    for V in (1, 2, 7, 100, 1000, 4096, 50000):
        for (T, k, p, mp) in ((1.0, 0, 1.0, 0.0), (0.8, 40, 0.95, 0.0), (1.3, 0, 0.9, 0.0), (0.5, 5, 0.5, 0.02),
                              (1.0, 0, 0.0, 0.0), (0.7, 64, 1.0, 0.1), (2.0, 1, 0.9, 0.0), (0.0, 10, 0.9, 0.0)):
            out.append((V, T, k, p, mp, int(rng.integers(1, 2 ** 63))))
    return out


@needs_ref
@pytest.mark.parametrize("V,T,k,p,mp,seed", _configs())
def test_sample_vs_reference(V, T, k, p, mp, seed):
    """Token, rng state and the first candidates bit-identical to the reference's
    sampler_sample compiled strict (-std=c11 -O2)."""
    rng = np.random.default_rng(seed % 1000)
    for rep in range(6):
        row = (rng.normal(0, 3, V) + (rng.random(V) < 0.01) * 8).astype(np.float32)
        if rep == 1:
            row = np.round(row)                                        # ties
        if rep == 2 and V > 3:
            row[rng.random(V) < 0.3] = -np.inf                          # masked entries
        st = int(rng.integers(1, 2 ** 63))
        n = min(V, 64)
        tok, st_ref, ri, rv = O.ref_sample_row("strict", row, st, T, k, p, mp, n_trace=n)
        o = O.sample_row(row, st, T, k, p, mp)
        assert o["token"] == tok and o["state"] == st_ref, (rep, o["token"], tok)
        if T > 0:
            np.testing.assert_array_equal(o["final_idx"][:n], ri)
            np.testing.assert_array_equal(o["final"][:n].view(np.uint32), rv.view(np.uint32))


def _boundary_configs():
    """1/temperature negative, zero and infinite (src/sampler.c:154 uses it as
    is), and top-k far past LDS sizes (any 0 < top_k < V, :166)."""
    out = []
    for V in (7, 1000, 20000):
        for (T, k, p, mp) in ((-0.5, 0, 0.9, 0.0), (-2.0, 40, 0.95, 0.0), (-1.0, 0, 1.0, 0.05),
                              (1e-40, 0, 0.9, 0.0), (1e-40, 5, 1.0, 0.0), (float("inf"), 0, 0.9, 0.0),
                              (float("inf"), 3, 1.0, 0.0), (1.0, V // 2, 0.9, 0.0), (0.7, V - 1, 0.95, 0.0),
                              (-0.7, V - 1, 0.8, 0.0), (1.2, max(1, V - 5), 1.0, 0.01)):
            if 0 < k < V or k == 0:
                out.append((V, T, k, p, mp))
    return out


@needs_ref
@pytest.mark.parametrize("V,T,k,p,mp", _boundary_configs())
def test_sample_vs_reference_boundary(V, T, k, p, mp):
    """The oracle's token and rng state equal the strict reference build's on the
    configurations outside the usual range, over rows with ties, masked (-inf)
    entries (+inf under a negative temperature) and large spreads."""
    rng = np.random.default_rng(V * 7 + k)
    for rep in range(4):
        row = rng.normal(0, 3, V).astype(np.float32)
        if rep == 1:
            row = np.round(row)
        if rep == 2 and V > 3:
            row[rng.random(V) < 0.2] = -np.inf
        if rep == 3:
            row[: V // 2] *= 1e37                                      # (l - max) overflows to -inf
        st = int(rng.integers(1, 2 ** 63))
        tok, st_ref, _, _ = O.ref_sample_row("strict", row, st, T, k, p, mp, n_trace=1)
        o = O.sample_row(row, st, T, k, p, mp)
        assert o["token"] == tok and o["state"] == st_ref, (rep, o["token"], tok)


@needs_ref
def test_fast_build_agreement():
    """Agreement of the reference's Makefile build (-O3 -ffast-math, libmvec expf)
    with the strict build on C2 rows: reported, not a parity target."""
    if O.ref("fast") is None:
        pytest.skip("fast build missing")
    w = W.c2(rows=16)
    same = 0
    for r in range(w.rows):
        row = O.prepared_row(w, r)
        a = O.ref_sample_row("strict", row, int(w.seeds[r]), w.temperature, w.top_k, w.top_p, w.min_p)[0]
        b = O.ref_sample_row("fast", row, int(w.seeds[r]), w.temperature, w.top_k, w.top_p, w.min_p)[0]
        same += a == b
    print(f"fast-math build agrees with the strict build on {same}/{w.rows} C2 rows")
    assert same >= w.rows // 2


def _ref_batch_ids(w, rows):
    """Token ids of the strict reference build on rows of a workload: the
    reference's penalties (src/sampler.c:21-52, frequency as the harness states
    it), the mask as -inf, then sampler_sample (oracle/ref_harness.c
    refh_time_batch, one run)."""
    L = O.ref("strict")
    lg = np.ascontiguousarray(w.logits[rows])
    if w.softcap > 0.0:
        for r in range(len(rows)):
            L.refh_softcap(lg[r], w.vocab, np.float32(w.softcap))
    mask, mw = None, 0
    if w.mask is not None:
        mask = np.ascontiguousarray(w.mask[rows])
    elif w.dfa is not None:
        tab = {}
        mask = np.ascontiguousarray(np.stack([tab.setdefault(int(w.dfa_states[r]),
                                                             O.dfa_mask(w.dfa, int(w.dfa_states[r]), w.vocab))
                                              for r in rows]))
    if mask is not None:
        mw = mask.shape[1]
    hoff = hids = None
    if w.hist_off is not None:
        lists = [w.hist_ids[w.hist_off[r]:w.hist_off[r + 1]] for r in rows]
        hoff = np.zeros(len(rows) + 1, np.int32)
        hoff[1:] = np.cumsum([len(x) for x in lists])
        hids = np.concatenate(lists).astype(np.int32)
    cfg = O.SamplerConfig(w.temperature, w.top_k, w.top_p, w.min_p, 1)
    ids = np.zeros(len(rows), np.int32)
    ms = np.zeros(1, np.float64)
    rc = L.refh_time_batch(lg, len(rows), w.vocab, hoff.ctypes.data if hoff is not None else None,
                           hids.ctypes.data if hids is not None else None,
                           mask.ctypes.data if mask is not None else None, mw, w.order, w.repeat_penalty,
                           w.frequency_penalty, w.presence_penalty, C.byref(cfg),
                           np.ascontiguousarray(w.seeds[rows]), min(8, len(rows)), 1, ms, ids)
    assert rc == 0
    return ids


@needs_ref
@pytest.mark.parametrize("name,nrows", [("C1", None), ("C2", None), ("C3", None), ("C5", None), ("C5CAP", None)])
def test_configs_full_size_vs_reference(name, nrows):
    """The oracle equals the strict reference build at the configurations' full
    shapes, every row: C1, the 64 rows of C2, the 32 of C3, and the 512 of C5
    (DFA masks from the oracle's walk) and of C5CAP (the reference's soft-cap
    loop first)."""
    w = W.CONFIGS[name]()
    rows = list(range(w.rows if nrows is None else nrows))
    np.testing.assert_array_equal(O.run_workload(w, rows)["ids"], _ref_batch_ids(w, rows))


# ----------------------------------------------------------------- golden vectors

GOLDEN = os.path.join(ROOT, "tests", "golden", "sampler_small.npz")


def test_golden_sampler_fixtures():
    """The committed small-vocabulary vectors (tests/golden/make_golden.py)."""
    g = np.load(GOLDEN, allow_pickle=False)
    for i in range(len(g["V"])):
        V = int(g["V"][i])
        row = g["logits"][i, :V]
        o = O.sample_row(row, int(g["seed"][i]), float(g["T"][i]), int(g["k"][i]), float(g["p"][i]),
                         float(g["mp"][i]), want_p=V)
        assert o["token"] == int(g["token"][i]) and o["state"] == int(g["state"][i]), i
        n = len(o["cand_p"])
        np.testing.assert_array_equal(o["cand_p"].view(np.uint32), g["cand_p"][i, :n].view(np.uint32))


# ------------------------------------------------------------------ A14-A16

KAT_GBNF = (b'root ::= "{" ws "\\"bbox_2d\\":" ws "[" ws int "]" ws "}"\n'
            b'int ::= [0-9]+\n'
            b'ws ::= [ \\t\\n\\r]*\n')


def test_grammar_unit_kats_oracle():
    """tools/test_grammar_unit.c:17-24 on the restatement."""
    L = O.lib()
    g = O.grammar(KAT_GBNF)
    assert g.is_receipt
    assert L.orc_grammar_accept(C.byref(g), b"{")
    L.orc_grammar_advance(C.byref(g), b"{")
    assert L.orc_grammar_accept(C.byref(g), b'"bbox_2d":')
    assert not L.orc_grammar_accept(C.byref(g), b"invalid")
    L.orc_grammar_advance(C.byref(g), b'"bbox_2d": [123] }')
    assert L.orc_grammar_finished(C.byref(g))


def test_grammar_unit_binary():
    """The reference's own unit test, built from its source by oracle/Makefile."""
    exe = os.path.join(ROOT, "oracle", "_ref", "test_grammar_unit")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/test_grammar_unit not built")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=30)
    assert r.returncode == 0 and "PASSED" in r.stdout


ALPHABET = list(b'{}[]":,\\ \t\n0123456789abxt_-') + [0x80, 0xC4, 0xA0]


def _rand_piece(rng, maxlen=6):
    n = int(rng.integers(1, maxlen + 1))
    return bytes(int(b) for b in rng.choice(ALPHABET, n))


def _receipt_stream(rng):
    """Pieces that mostly follow the receipt schema, with random corruption."""
    text = b' {"bbox_2d": [12, 3 ,450,7] , "text_content": "a \\"q\\" b"} '
    cuts = sorted(set(int(c) for c in rng.integers(1, len(text), 8)))
    pieces = [text[a:b] for a, b in zip([0] + cuts, cuts + [len(text)])]
    if rng.random() < 0.5:
        i = int(rng.integers(0, len(pieces)))
        pieces[i] = _rand_piece(rng)
    return pieces


@needs_ref
@pytest.mark.parametrize("mode", [b"receipt bbox_2d", b"root ::= object | value", b"plain text grammar"])
def test_grammar_vs_reference(mode):
    """accept_str / advance / is_finished of the restatement against the reference
    (src/core/grammar.c:68-273) on random and schema-shaped piece streams."""
    L = O.lib()
    R = REF_STRICT
    rng = np.random.default_rng(len(mode))
    for trial in range(300):
        g = O.grammar(mode)
        h = R.diskllm_grammar_init_from_str(mode)
        try:
            pieces = _receipt_stream(rng) if trial % 2 else [_rand_piece(rng) for _ in range(10)]
            for pc in pieces:
                for probe in (pc, _rand_piece(rng), b"}", b"]", b'"', b" "):
                    assert L.orc_grammar_accept(C.byref(g), probe) == R.diskllm_grammar_accept_str(h, probe), \
                        (mode, g.buf[:g.len], probe)
                assert L.orc_grammar_finished(C.byref(g)) == R.diskllm_grammar_is_finished(h)
                L.orc_grammar_advance(C.byref(g), pc)
                R.diskllm_grammar_advance(h, pc)
        finally:
            R.diskllm_grammar_free(h)


def _csr(strings):
    off = np.zeros(len(strings) + 1, np.uint32)
    off[1:] = np.cumsum([len(s) for s in strings])
    data = np.frombuffer(b"".join(strings), np.uint8).copy() if off[-1] else np.zeros(1, np.uint8)
    return off, data


@needs_ref
def test_grammar_mask_vs_reference():
    """apply_mask (src/core/grammar.c:275-308) through a get_token_str callback."""
    rng = np.random.default_rng(8)
    vocab = [b""] + [_rand_piece(rng, 5) for _ in range(3000)] + [b"{", b"[", b"}", b"]", b'"', b" "]
    V = len(vocab)
    off, data = _csr(vocab)
    cbuf = [C.c_char_p(s) for s in vocab]
    CB = C.CFUNCTYPE(C.c_char_p, C.c_void_p, C.c_int)
    cb = CB(lambda ctx, i: C.cast(cbuf[i], C.c_void_p).value)
    for mode in (b"root ::= object | value", b"receipt bbox_2d"):
        for prefix in (b"", b" {", b'{"bbox_2d": [1,2', b'[{"a": "x}"', b'{"bbox_2d":[1,2,3,4],"text_content":"hi"}'):
            g = O.grammar(mode)
            O.lib().orc_grammar_advance(C.byref(g), prefix)
            h = REF_STRICT.diskllm_grammar_init_from_str(mode)
            REF_STRICT.diskllm_grammar_advance(h, prefix)
            for eos in (5, -1):
                lg = rng.normal(0, 1, V).astype(np.float32)
                a = lg.copy()
                n_ref = REF_STRICT.diskllm_grammar_apply_mask(h, a, V, None, C.cast(cb, C.c_void_p), eos)
                b, n = O.grammar_mask(g, off, data, eos, lg)
                np.testing.assert_array_equal(a, b)
                assert n == n_ref
            REF_STRICT.diskllm_grammar_free(h)


def test_dfa_mask_brute_force():
    """A16: token t allowed from state s iff walking its bytes never reaches state 0
    (EOS by the accept set), against a direct walk."""
    w = W.c4(rows=4)
    dfa = w.dfa
    V = len(dfa.offsets) - 1
    sel = np.random.default_rng(9).choice(V, 4000, replace=False)
    for r in range(w.rows):
        s0 = int(w.dfa_states[r])
        m = O.dfa_mask(dfa, s0, V)
        for t in list(sel) + [int(dfa.eos_id)]:
            t = int(t)
            if t == dfa.eos_id:
                ok = bool((int(dfa.accept) >> s0) & 1)
            else:
                b0, b1 = int(dfa.offsets[t]), int(dfa.offsets[t + 1])
                s, ok = s0, b1 > b0
                for b in dfa.data[b0:b1]:
                    s = int(dfa.trans[s, b])
                    if s == 0:
                        ok = False
                        break
            assert bool((m[t >> 5] >> (t & 31)) & 1) == ok, (r, t)


def test_packed_mask_semantics():
    rng = np.random.default_rng(10)
    V = 1000
    row = rng.normal(0, 1, V).astype(np.float32)
    m = rng.integers(0, 2 ** 32, (V + 31) // 32, dtype=np.uint64).astype(np.uint32)
    out = row.copy()
    O.lib().orc_apply_packed_mask(out, V, m)
    bits = (m[np.arange(V) >> 5] >> (np.arange(V) & 31).astype(np.uint32)) & 1
    np.testing.assert_array_equal(out, np.where(bits == 1, row, -np.inf).astype(np.float32))


# ------------------------------------------------------------------------ expf

def test_expf_restatement_vs_host_libm():
    """The device expf (diskllm_amd/csrc/hip/expf_glibc.h) compiled for the host,
    against this host's libm expf, on every 4099th float bit pattern, screened
    and unscreened-with-clamp (the exhaustive run is the same program with stride 1)."""
    exe = os.path.join(ROOT, "oracle", "_build", "expf_host_check")
    src = os.path.join(ROOT, "tests", "native", "expf_host_check.c")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm", "-lpthread"], check=True)
    for mode in ([], ["core"]):
        r = subprocess.run([exe, "0", str(1 << 32), "4099", "8"] + mode, capture_output=True, text=True,
                           timeout=300)
        checked, bad = map(int, r.stdout.split())
        assert checked > 500000 and bad == 0, (mode, r.stdout, r.stderr[:500])


@needs_ref
def test_sample_nan_and_inf_rows_vs_reference():
    """NaN and +inf logits (the softmax sum turns NaN and no comparison holds):
    the restatement follows the reference there too, with and without top-k."""
    rng = np.random.default_rng(13)
    for V in (5, 300, 20000):
        for (T, k, p) in ((1.0, 0, 0.9), (0.8, 4, 0.95), (1.0, 0, 1.0)):
            for case in range(5):
                row = rng.normal(0, 2, V).astype(np.float32)
                if case == 0:
                    row[0] = np.nan
                elif case == 1:
                    row[V // 2] = np.nan
                elif case == 2:
                    row[V - 1] = np.inf
                elif case == 3:
                    row[1] = np.inf
                    row[2] = np.nan
                else:
                    row[:] = -np.inf
                    row[V // 3] = np.inf
                st = int(rng.integers(1, 2 ** 63))
                tok, st_ref, _, _ = O.ref_sample_row("strict", row, st, T, k, p, 0.0)
                o = O.sample_row(row, st, T, k, p, 0.0)
                assert (o["token"], o["state"]) == (tok, st_ref), (V, T, k, p, case, o["token"], tok)


# ------------------------------------------------------------------------ tanhf / soft-cap

def test_tanhf_restatement_vs_host_libm():
    """The device tanhf (diskllm_amd/csrc/hip/tanhf_glibc.h) compiled for the host,
    against this host's libm tanhf, on every 1031st float bit pattern, and the
    soft-cap cap * tanhf(x / cap) for the Gemma cap 30 and two others (the
    exhaustive run is the same program with stride 1: 4,278,190,082 inputs, 0
    mismatches)."""
    exe = os.path.join(ROOT, "oracle", "_build", "tanhf_host_check")
    src = os.path.join(ROOT, "tests", "native", "tanhf_host_check.c")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm", "-lpthread"], check=True)
    for extra, stride in (([], 1031), (["cap=30"], 2053), (["cap=0.75"], 4099), (["cap=1e4"], 4099)):
        r = subprocess.run([exe, "0", str(1 << 32), str(stride), "8"] + extra, capture_output=True, text=True,
                           timeout=300)
        checked, bad = map(int, r.stdout.split())
        assert checked > 1000000 and bad == 0, (extra, r.stdout, r.stderr[:500])


def test_tanhf_monotone():
    """tanhf (the restatement, bit-identical to the host libm) never decreases
    from one float to the next, from -inf to +inf; hence x -> cap * tanhf(x / cap)
    is non-decreasing for every cap > 0, which is what lets the top-k kernel
    select soft-capped candidates on the raw logits.  Here every 97th pair of
    consecutive floats, and the composite for two caps; the exhaustive run is the
    same program with stride 1 (4,278,190,081 pairs, 0 decreases)."""
    exe = os.path.join(ROOT, "oracle", "_build", "tanhf_monotone_check")
    src = os.path.join(ROOT, "tests", "native", "tanhf_monotone_check.c")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm", "-lpthread"], check=True)
    for extra, stride in (([], 97), (["cap=30"], 1021), (["cap=0.75"], 2039)):
        r = subprocess.run([exe, str(stride), "8"] + extra, capture_output=True, text=True, timeout=300)
        checked, bad = map(int, r.stdout.split())
        assert checked > 1000000 and bad == 0, (extra, r.stdout, r.stderr[:500])


@needs_ref
def test_softcap_strict_and_fast_builds():
    """The reference's soft-cap loop (src/core/context.c:873-876) as the two builds
    compile it.  Strict ISO C: bit-identical to orc_softcap (and so to the
    kernels, which match orc_softcap bit for bit).  The reference Makefile's
    -O3 -ffast-math build (x * (1/cap), libmvec tanhf): within 4 ulp but not
    bit-identical, on about 41% of logits uniform in [-60, 60] -- the strict
    build is the parity target.  On 16 C5 rows the differences change no sampled
    token."""
    fast = O.ref("fast")
    if fast is None:
        pytest.skip("fast reference build absent")
    x = np.random.default_rng(1).uniform(-60.0, 60.0, 1 << 20).astype(np.float32)
    x[:6] = [0.0, -0.0, np.inf, -np.inf, 1e-30, 700.0]
    a, b, c = x.copy(), x.copy(), x.copy()
    REF_STRICT.refh_softcap(a, a.size, np.float32(30.0))
    fast.refh_softcap(b, b.size, np.float32(30.0))
    O.lib().orc_softcap(c, c, c.size, np.float32(30.0))
    np.testing.assert_array_equal(a.view(np.uint32), c.view(np.uint32))
    d = np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))
    assert 0.3 < np.count_nonzero(d) / d.size < 0.5 and d.max() <= 4
    w = W.c5cap(rows=16)
    strict_ids = O.run_workload(w)["ids"]
    lg = np.ascontiguousarray(w.logits)
    for r in range(w.rows):
        fast.refh_softcap(lg[r], w.vocab, np.float32(w.softcap))
    w.logits, w.softcap = lg, 0.0
    np.testing.assert_array_equal(O.run_workload(w)["ids"], strict_ids)


def test_oracle_softcap_known_values():
    """orc_softcap against values fixed by the mathematics: tanh(0) = 0 (sign
    kept), tanh saturates to +-1 at |x| >= 22 (so cap * 1 = cap), tanh(x) ~ x
    near 0, odd symmetry, no-op for cap <= 0 or NaN."""
    x = np.array([0.0, -0.0, 1e-30, 22.0 * 30, -1e30, np.inf, -np.inf, 15.0, -15.0, 3.0], np.float32)
    y = np.empty_like(x)
    O.lib().orc_softcap(x, y, x.size, np.float32(30.0))
    assert y[0] == 0.0 and not np.signbit(y[0]) and y[1] == 0.0 and np.signbit(y[1])
    assert y[2] == np.float32(1e-30)
    assert y[3] == 30.0 and y[4] == -30.0 and y[5] == 30.0 and y[6] == -30.0
    assert y[7] == -y[8]
    assert abs(float(y[9]) - 30.0 * np.tanh(0.1)) < 1e-5
    for cap in (0.0, -1.0, np.nan):
        O.lib().orc_softcap(x, y, x.size, np.float32(cap))
        np.testing.assert_array_equal(y.view(np.uint32), x.view(np.uint32))
