"""GPU parity of dlk_dfa_mask (A16: the byte-DFA allow-mask) with the oracle's
direct walk (oracle/oracle.c orc_dfa_mask), bit for bit, over the shapes that
select its kernels and paths: automata of up to 64 states (state-per-lane walk,
8/16/32/64 lanes of keys per wave, batches of more rows than states sharing
masks), larger automata (token-per-thread walk), the EOS rule, empty tokens,
start states outside the automaton or negative, and blocks whose tokens are
too long to stage in LDS (bytes read from memory)."""
import numpy as np
import pytest

from diskllm_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _expected(d, state, V, n_states):
    """The oracle's walk for a start state inside the automaton; outside it no
    token is allowed, and the EOS id follows the accept bit (0 < state < 64)."""
    if 0 < state < n_states:
        return O.dfa_mask(d, state, V)
    out = np.zeros((V + 31) // 32, np.uint32)
    if 0 <= d.eos_id < V and 0 < state < 64 and (int(d.accept) >> state) & 1:
        out[d.eos_id >> 5] |= np.uint32(1) << np.uint32(d.eos_id & 31)
    return out


CASES = [
    # (V, rows, n_states, dead_frac, max_len, eos, label)
    (1, 3, 64, 0.7, 16, -1, "one token"),
    (33, 5, 64, 0.7, 16, 0, "two words, 5 rows"),
    (1000, 16, 64, 0.7, 16, 999, "16 rows"),
    (20011, 17, 17, 0.5, 16, 7, "17 rows, 17 states"),
    (20011, 64, 64, 0.3, 16, 123, "64 rows, live automaton"),
    (70000, 130, 64, 0.7, 16, 69999, "three row groups"),
    (5000, 8, 2, 0.0, 16, -1, "two states"),
    (9000, 40, 200, 0.7, 16, 11, "200 states (token-per-thread kernel)"),
    (9000, 64, 65, 0.6, 16, -1, "65 states (token-per-thread kernel)"),
    (3000, 12, 64, 0.02, 300, 5, "long tokens: unstaged blocks"),
    (40000, 700, 5, 0.3, 16, 17, "700 rows over 5 states: shared masks"),
    (262144, 512, 64, 0.7, 16, 262143, "C5 shape: 512 rows, 64 states"),
    (1000, 9, 40, 0.5, 16, 3, "9 rows: states negative, at 40..63 and above 63"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[-1] for c in CASES])
def test_dfa_mask_vs_oracle(cuda, case):
    from diskllm_amd import api
    V, rows, n_states, dead, max_len, eos, label = case
    rng = np.random.default_rng(V + rows + n_states)
    if max_len > 16:
        lens = rng.integers(0, max_len + 1, V).astype(np.uint32)
    else:
        lens = np.minimum(rng.geometric(0.25, V), max_len).astype(np.uint32)
        lens[rng.random(V) < 0.01] = 0                                     # empty tokens
    off = np.zeros(V + 1, np.uint32)
    off[1:] = np.cumsum(lens, dtype=np.uint64).astype(np.uint32)
    data = rng.integers(0, 256, int(off[-1]) or 1, dtype=np.uint8)
    trans = W.make_dfa_table(rng, n_states, dead)
    accept = int(rng.integers(0, 2 ** 63)) * 2 + 1
    d = W.DFA(off, data, trans, eos_id=eos, accept=accept)
    states = rng.integers(1, n_states, rows).astype(np.int32)
    states[rng.random(rows) < 0.1] = 0                                     # dead start
    if rows > 2:
        states[1] = n_states + 1                                           # outside the automaton
    if rows == 9:
        states[2:8] = [-1, -70000, 45, 63, 64, 1000]                       # keys 0, 45, 63, 0, 0
    _announce(f"dfa {label}: V={V} rows={rows} n_states={n_states}")
    got = api.dfa_masks(off, data, trans, states, V, eos, accept).cpu().numpy().view(np.uint32)
    for r in range(rows):
        np.testing.assert_array_equal(got[r], _expected(d, int(states[r]), V, n_states),
                                      err_msg=f"{label}: row {r} state {states[r]}")
