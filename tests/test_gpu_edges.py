"""GPU parity on edge cases, through both paths of dlk_sample (automatic dispatch
and the forced one-workgroup-per-row kernel): greedy, masked rows, fewer finite
entries than k, long runs of equal logits at the k-th value, min-p, top-p <= 0 /
= 1, tiny vocabularies, out-of-range and repeated history ids.
"""
import numpy as np
import pytest

from oracle import oracle as O
from diskllm_amd import workloads as W

pytestmark = pytest.mark.gpu

PATHS = [0, 1]   # automatic dispatch, forced row kernel


def make(name, rows, V, seed=0, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, rep=1.0, freq=0.0, pres=0.0,
         order=W.ORDER_REFERENCE, hist=None, mask=None, logits=None, n_out=0):
    rng = np.random.Generator(np.random.PCG64(seed))
    lg = logits if logits is not None else rng.normal(0, 3, size=(rows, V)).astype(np.float32)
    hoff = hids = None
    if hist is not None:
        hoff = np.zeros(rows + 1, np.int32)
        hoff[1:] = np.cumsum([len(h) for h in hist])
        hids = np.concatenate([np.asarray(h, np.int32) for h in hist]).astype(np.int32)
    seeds = rng.integers(1, 2 ** 63, size=rows, dtype=np.uint64)
    return W.Workload(name, rows, V, np.ascontiguousarray(lg, np.float32), seeds, temperature=temperature,
                      top_k=top_k, top_p=top_p, min_p=min_p, repeat_penalty=rep, frequency_penalty=freq,
                      presence_penalty=pres, order=order, hist_off=hoff, hist_ids=hids, mask=mask, n_out=n_out)


def run_and_check(w, path):
    from diskllm_amd import api
    print(f"[case] {w.name} rows={w.rows} V={w.vocab} k={w.top_k} p={w.top_p} minp={w.min_p} T={w.temperature} "
          f"path={path}", flush=True)
    db = api.to_device(w)
    api.sample(db, api.params_of(w, path=path))
    res = api.results(db)
    for r in range(w.rows):
        o = O.sample_row(O.prepared_row(w, r), int(w.seeds[r]), w.temperature, w.top_k, w.top_p, w.min_p,
                         want_p=w.n_out)
        assert int(res["ids"][r]) == o["token"], (w.name, r, int(res["ids"][r]), o["token"])
        assert int(res["states"][r]) == o["state"], (w.name, r)
        # (candidate outputs are the softmax stage's entries in buffer order; the
        # oracle's trace is the buffer after min-p's compaction)
        if w.n_out and w.min_p == 0.0 and o["k"] and not o["greedy"] and np.all(np.isfinite(o["cand_p"])):
            n = min(w.n_out, o["k"])
            np.testing.assert_array_equal(res["cand_ids"][r, :n], o["cand_idx"][:n])
            np.testing.assert_allclose(res["cand_probs"][r, :n], o["cand_p"][:n], rtol=1e-5)
    assert res["status"] == 0
    return res


def mask_rows(rows, V, allowed_lists):
    m = np.zeros((rows, (V + 31) // 32), np.uint32)
    for r, al in enumerate(allowed_lists):
        al = np.asarray(al, np.int64)
        if al.size:
            np.bitwise_or.at(m[r], al >> 5, (np.uint32(1) << (al & 31).astype(np.uint32)))
    return m


@pytest.mark.parametrize("path", PATHS)
def test_greedy(cuda, path):
    w = make("greedy", 6, 50000, seed=1, temperature=0.0, top_k=40, hist=[[1, 2, 3]] * 6, rep=1.3)
    w.logits[2, 777] = w.logits[2].max() + 1
    w.logits[2, 9000] = w.logits[2, 777]          # tie: lowest index wins
    w.logits[3, :] = -np.inf                      # all -inf: index 0
    w.logits[4, 0] = np.nan                       # NaN at 0: index 0 (src/sampler.c:11-17)
    res = run_and_check(w, path)
    assert res["ids"][2] == 777 and res["ids"][3] == 0 and res["ids"][4] == 0


@pytest.mark.parametrize("path", PATHS)
def test_masked_rows_topk(cuda, path):
    V = 40000
    rng = np.random.default_rng(5)
    allowed = [[], [1234], list(rng.choice(V, 7, replace=False)), list(rng.choice(V, 300, replace=False)),
               list(range(V - 5, V)), [0]]
    w = make("masked", len(allowed), V, seed=2, temperature=0.7, top_k=20, top_p=0.9,
             mask=mask_rows(len(allowed), V, allowed), n_out=24)
    res = run_and_check(w, path)
    assert res["ids"][0] == 19                    # all masked: candidate k-1 in index order
    assert res["ids"][1] == 1234 and res["ids"][5] == 0


@pytest.mark.parametrize("path", PATHS)
def test_masked_rows_full_vocab(cuda, path):
    V = 30000
    allowed = [[], [4321], list(range(0, V, 97))]
    w = make("masked-full", 3, V, seed=3, temperature=1.0, top_p=0.95, mask=mask_rows(3, V, allowed))
    res = run_and_check(w, path)
    assert res["ids"][0] == V - 1 and res["ids"][1] == 4321


@pytest.mark.parametrize("path", PATHS)
def test_ties_at_kth(cuda, path):
    V = 70000
    rows = 4
    lg = np.random.default_rng(7).normal(0, 1, size=(rows, V)).astype(np.float32)
    lg[0, :] = 1.5                                # every entry equal: first k by index
    lg[1, ::3] = 4.0                              # 23k-way tie above the rest
    lg[2, 10:5000] = 9.0                          # contiguous tie block
    lg[3, :] = np.round(lg[3] * 4) / 4            # quantised logits: many s ties
    w = make("ties", rows, V, seed=4, temperature=0.9, top_k=50, top_p=0.8, logits=lg, n_out=50)
    res = run_and_check(w, path)


@pytest.mark.parametrize("path", PATHS)
def test_min_p_and_top_p_edges(cuda, path):
    V = 20000
    for tp, mp, k in [(0.0, 0.0, 30), (-1.0, 0.0, 0), (1.0, 0.0, 30), (0.5, 0.02, 0), (0.9, 0.001, 64),
                      (0.9, 0.9, 16), (1.0, 0.05, 0)]:
        w = make(f"edges-p{tp}-minp{mp}-k{k}", 5, V, seed=11, temperature=0.6, top_k=k, top_p=tp, min_p=mp)
        w.logits[:, 17] += 12.0                   # one dominant token
        run_and_check(w, path)


@pytest.mark.parametrize("path", PATHS)
def test_tiny_vocab_and_history(cuda, path):
    for V in (1, 2, 3, 63, 64, 65, 4095, 4097):
        hist = [[0, 0, V - 1, V + 5, -3, 1, 1, 1], [], [V // 2] * 40]
        w = make(f"tiny{V}", 3, V, seed=V, temperature=1.3, top_k=min(5, V), top_p=0.97, rep=1.2, pres=0.4,
                 freq=0.1, order=W.ORDER_NORTH_STAR, hist=hist)
        run_and_check(w, path)
        w2 = make(f"tiny{V}-full", 3, V, seed=V + 1, temperature=0.5, top_p=0.9, rep=1.5, hist=hist)
        run_and_check(w2, path)


@pytest.mark.parametrize("path", PATHS)
def test_penalty_orders(cuda, path):
    V = 50000
    rng = np.random.default_rng(9)
    hist = [list(rng.integers(0, 50, 200)), list(rng.integers(0, V, 300))]
    for order in (W.ORDER_REFERENCE, W.ORDER_NORTH_STAR, W.pack_order(W.OP_FREQUENCY, W.OP_PRESENCE,
                                                                        W.OP_REPETITION)):
        w = make(f"order{order:x}", 2, V, seed=12, temperature=1.0, top_k=100, top_p=0.95, rep=1.3, freq=0.2,
                 pres=-0.7, order=order, hist=hist)
        w.logits[:, :50] = np.linspace(-6, 6, 50, dtype=np.float32)
        run_and_check(w, path)


@pytest.mark.parametrize("path", PATHS)
def test_penalties_on_the_top_entries(cuda, path):
    """History ids that are each row's best logits (5 to 1000 of them), with
    penalties strong enough to move them below the rest: the top-k kernel takes
    its threshold from raw logits before the patches, finds fewer than k + 16
    entries above it and recomputes it from exact values.  Negative presence
    lifts ids instead; the last case repeats the first under a soft-cap."""
    V, rows = 120000, 6
    rng = np.random.default_rng(77)
    lg = rng.normal(0, 3, size=(rows, V)).astype(np.float32)
    best = np.argsort(-lg, axis=1, kind="stable")
    hist = [list(best[r, :n]) for r, n in enumerate([60, 150, 300, 40, 1000, 5])]
    for rep, freq, pres, cap in ((50.0, 0.0, 0.0, 0.0), (1.0, 0.0, 25.0, 0.0), (1.3, 0.5, -8.0, 0.0),
                                 (50.0, 0.0, 0.0, 30.0)):
        w = make(f"toppen-{rep}-{pres}-{cap}", rows, V, seed=5, temperature=0.9, top_k=40, top_p=0.95, rep=rep,
                 freq=freq, pres=pres, hist=hist, logits=lg.copy(), n_out=8)
        w.softcap = cap
        run_and_check(w, path)


@pytest.mark.parametrize("path", [0, 1, 2])
def test_full_vocab_min_p(cuda, path):
    """Min-p without top-k at Qwen vocab through the fused kernel (0), the row
    kernel (1) and the fused kernel's exact fallbacks on every row (2: the split
    softmax, survivors' and top-p sums, the draw re-walked per slice): survivors p >= min_p in
    index order, renormalised (src/sampler.c:188-202), then top-p and the draw;
    min_p 0.5 leaves no survivor, so every entry stays (:195)."""
    V = 151936
    for (T, tp, mp, sd) in [(1.0, 0.9, 1e-6, 51), (1.0, 1.0, 1e-5, 52), (0.7, 0.95, 1e-4, 53), (1.3, 0.9, 0.01, 54),
                            (1.0, 0.9, 0.5, 55), (0.5, 1.0, 0.5, 56)]:
        w = W.c2(seed=sd, rows=8, vocab=V)
        w.temperature, w.top_p, w.min_p = T, tp, mp
        w.n_out = 16
        res = run_and_check(w, path)
        if path != 1:
            # the candidate outputs (softmax stage, buffer order, final log-probabilities)
            # equal the row kernel's
            ref = run_and_check(w, 1)
            for key in ("cand_ids", "cand_probs", "cand_logprobs"):
                np.testing.assert_array_equal(res[key].view(np.uint32), ref[key].view(np.uint32), err_msg=key)
    w = W.c2(seed=57, rows=4, vocab=V)
    w.min_p = 2e-5
    m = np.zeros((4, (V + 31) // 32), np.uint32)
    rng = np.random.default_rng(57)
    for r in range(4):
        al = rng.choice(V, [3, 1000, 50000, V][r], replace=False)
        np.bitwise_or.at(m[r], al >> 5, (np.uint32(1) << (al & 31).astype(np.uint32)))
    w.mask = m
    run_and_check(w, path)


@pytest.mark.parametrize("path", [0, 1, 2])
def test_full_vocab_variants(cuda, path):
    """Full-vocabulary sampling at Qwen vocab through the fused kernel (0), the
    row kernel (1) and the fused kernel's exact fallbacks on every row (2)."""
    V = 151936
    rng = np.random.default_rng(21)
    for (T, tp, sd) in [(1.0, 0.9, 31), (0.7, 0.95, 32), (1.3, 1.0, 33), (0.5, 0.0, 34), (2.0, 0.5, 35)]:
        w = W.c2(seed=sd, rows=8, vocab=V)
        w.temperature, w.top_p = T, tp
        w.n_out = 16
        run_and_check(w, path)
    w = W.c2(seed=36, rows=6, vocab=V)
    m = np.zeros((6, (V + 31) // 32), np.uint32)
    for r in range(6):
        al = rng.choice(V, [1, 5, 1000, 20000, 100000, V][r], replace=False)
        np.bitwise_or.at(m[r], al >> 5, (np.uint32(1) << (al & 31).astype(np.uint32)))
    w.mask = m
    run_and_check(w, path)


@pytest.mark.parametrize("V,rows", [(151936, 64), (50004, 8), (262144, 3), (8192, 40), (100004, 1)])
def test_split_sums_shapes(cuda, V, rows):
    """The fused kernel's exact fallbacks on every row (path 2: the softmax,
    survivors' and top-p sums by all of the row's workgroups, the draw walked
    slice by slice from each slice's exact start) over vocabularies and batch
    sizes that change the slices (1 to 16 workgroups per row; a last chunk and
    a last group that end inside the vocabulary), top-p off, on, at 0 and below
    the row's mass, min-p with and without survivors: tokens against the oracle
    and every candidate output bit-equal to the row kernel's."""
    from diskllm_amd import api
    for (T, tp, mp) in [(1.0, 0.9, 0.0), (0.6, 1.0, 0.0), (1.4, 0.0, 0.0), (0.9, 0.999999, 0.0), (1.0, 0.9, 1e-5),
                        (0.8, 1.0, 0.5)]:
        w = W.c2(seed=V % 1000 + rows, rows=rows, vocab=V)
        w.temperature, w.top_p, w.min_p = T, tp, mp
        w.n_out = 24
        w.name = f"split-V{V}-T{T}-p{tp}-mp{mp}"
        res = run_and_check(w, 2)
        ref = run_and_check(w, 1)
        for key in ("ids", "states", "cand_ids", "cand_probs", "cand_logprobs"):
            a, b = np.asarray(res[key]), np.asarray(ref[key])
            if a.dtype.kind == "f":
                a, b = a.view(np.uint32), b.view(np.uint32)
            np.testing.assert_array_equal(a, b, err_msg=f"{w.name}: {key}")


@pytest.mark.parametrize("rows,V,k", [(300, 131072, 40), (1030, 65536, 8)])
def test_topk_slice_major_grid(cuda, rows, V, k):
    """The top-k kernel's slice-major grid (four or more blocks per CU: grid
    (rows, G), row blockIdx.x, slice blockIdx.y, raised wave priority for each
    slice's tail) at row counts that are not multiples of 8, with a history
    and penalties on every row: tokens, rng states and the candidates against
    the oracle."""
    rng = np.random.default_rng(rows)
    hist = [rng.integers(0, V, 48) for _ in range(rows)]
    w = make(f"spread-{rows}-{V}", rows, V, seed=rows, temperature=0.9, top_k=k, top_p=0.95, rep=1.2, freq=0.1,
             pres=0.3, hist=hist, n_out=8)
    run_and_check(w, 0)


@pytest.mark.parametrize("rows,V", [(16, 151936), (256, 32768), (40, 151936), (24, 151936), (5, 151936)])
def test_fused_block_to_slice_mappings(cuda, rows, V):
    """The fused kernel's block -> (row, slice) mappings on the automatic path:
    16 rows (G 16: a row's slices from both halves of each XCD's blocks), 256
    rows of a small vocabulary (G 2: one slice from each half), 40 rows (G 13,
    odd: rows on one XCD, slices in order), 24 rows (G 22: two launches of 23
    and 1 rows, grids of no whole eight-row groups, consecutive blocks) and 5
    rows (consecutive blocks).  Tokens and rng states against the oracle."""
    w = W.c2(seed=100 + rows, rows=rows, vocab=V)
    w.name = f"mapping-rows{rows}-V{V}"
    run_and_check(w, 0)


@pytest.mark.parametrize("T", [0.5, 0.6, 0.8, 1.3])
def test_fresh_batches_natural_fallbacks(cuda, T):
    """Fresh C2 batches through the automatic path at temperatures where rows
    meet the fused kernel's fallbacks without forcing: sums the certified
    bounds leave open (split sums) and slices whose candidate chains miss the
    composition's value (re-walks, mostly at T 0.6 and below).  Every token
    and rng state against the oracle, over four launches of 64 rows each."""
    from diskllm_amd import api
    for b in range(4):
        w = W.c2(seed=90001 + 131 * b + int(T * 10))
        w.temperature = T
        w.name = f"fresh-T{T}-b{b}"
        print(f"[case] {w.name} rows={w.rows} V={w.vocab}", flush=True)
        db = api.to_device(w)
        api.sample(db, api.params_of(w))
        res = api.results(db)
        assert res["status"] == 0
        for r in range(w.rows):
            o = O.sample_row(O.prepared_row(w, r), int(w.seeds[r]), w.temperature, w.top_k, w.top_p, w.min_p)
            assert int(res["ids"][r]) == o["token"], (w.name, r, int(res["ids"][r]), o["token"])
            assert int(res["states"][r]) == o["state"], (w.name, r)


@pytest.mark.parametrize("path", [0, 2])
def test_full_vocab_many_rows(cuda, path):
    """More rows than one cooperative launch holds: the host splits the batch."""
    w = W.c2(seed=41, rows=300, vocab=16384)
    run_and_check(w, path)


@pytest.mark.parametrize("path", [0, 1, 2])
def test_nan_and_inf_rows(cuda, path):
    """NaN / +inf logits make the reference's softmax sum NaN: every comparison
    after it fails and the draw falls through (src/sampler.c:226-233)."""
    for V, k, tp, mp in ((20000, 0, 0.9, 0.0), (20000, 0, 1.0, 0.0), (9000, 7, 0.95, 0.0), (9000, 50, 0.9, 0.01),
                         (300, 20, 1.0, 0.0)):
        if path == 2 and k:
            continue
        rows = 6
        lg = np.random.default_rng(V + k).normal(0, 2, size=(rows, V)).astype(np.float32)
        lg[0, 0] = np.nan
        lg[1, V // 2] = np.nan
        lg[2, V - 1] = np.inf
        lg[3, 1] = np.inf
        lg[3, 2] = np.nan
        lg[4, :] = -np.inf
        lg[4, V // 3] = np.inf
        lg[5, 3] = np.nan                            # NaN late in the first k: a barrier for the insertion sort
        w = make(f"nan-inf-k{k}-p{tp}-mp{mp}", rows, V, seed=5, temperature=1.0, top_k=k, top_p=tp, min_p=mp,
                 logits=lg, n_out=12)
        run_and_check(w, path)


def test_sync_timeout_path(cuda):
    """The fused kernel's bounded cross-workgroup waits, made to give up at their
    first poll that finds a word not yet written (DLK_PATH_FULL_NO_WAIT, set from
    the host; every launch still runs to its end): the call completes, sets
    DLK_STATUS_SYNC_TIMEOUT and writes ids inside the vocabulary.  The timed-out
    launch returns the row's published words to zero like any other, so the next
    ordinary call on the same stream and workspace is exact again."""
    from diskllm_amd import _lib, api
    w = W.c2(rows=16)
    db = api.to_device(w)
    ref = [O.sample_row(O.prepared_row(w, r), int(w.seeds[r]), w.temperature, w.top_k, w.top_p, w.min_p)
           for r in range(w.rows)]
    for cycle in range(2):
        print(f"[case] no-wait launch, cycle {cycle}", flush=True)
        db.reset_rng()
        db.status.zero_()
        api.sample(db, api.params_of(w, path=_lib.PATH_FULL_NO_WAIT))
        res = api.results(db)
        assert res["status"] & 2, "no wait gave up"
        assert np.all((res["ids"] >= 0) & (res["ids"] < w.vocab)), res["ids"]
        print(f"[case] ordinary launch after it, cycle {cycle}", flush=True)
        db.reset_rng()
        db.status.zero_()
        api.sample(db, api.params_of(w))
        res = api.results(db)
        assert res["status"] == 0
        for r in range(w.rows):
            assert int(res["ids"][r]) == ref[r]["token"], (cycle, r)
            assert int(res["states"][r]) == ref[r]["state"], (cycle, r)


@pytest.mark.parametrize("path", PATHS)
def test_topk_sums_both_ways(cuda, path):
    """Top-k rows whose k candidates' softmax terms either are all whole
    multiples of the running sum's ulp (the one-wave pipeline sums them by a
    wave scan) or are not (terms down to 2^-40 of the maximum: it runs the
    reference's loops); min-p and top-p on both, against the oracle."""
    V, k = 40000, 48
    rng = np.random.default_rng(11)
    lg = rng.normal(0, 1, size=(6, V)).astype(np.float32)
    top = rng.choice(V, size=(6, k), replace=False)
    for r in range(6):
        if r % 2 == 0:
            lg[r, top[r]] = 20.0 + rng.normal(0, 0.5, size=k).astype(np.float32)       # close together
        else:
            lg[r, top[r]] = 20.0 + np.linspace(0.0, -28.0, k).astype(np.float32)      # spread far apart
    for top_p, min_p in ((0.9, 0.0), (1.0, 1e-6), (0.95, 1e-7)):
        w = make("topk_sums", 6, V, seed=12, temperature=1.0, top_k=k, top_p=top_p, min_p=min_p, logits=lg, n_out=8)
        run_and_check(w, path)
