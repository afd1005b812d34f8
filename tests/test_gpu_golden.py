"""The committed golden vectors (tests/golden/sampler_small.npz: 48 rows, V 1 to
4096, written by tests/golden/make_golden.py from the oracle after checking it
against the reference build) through dlk_sample, on the automatic path and on
the one-workgroup-per-row kernel: token, rng state and the first candidates'
softmax probabilities (src/sampler.c:183-185) bit-identical."""
import os

import numpy as np
import pytest

from diskllm_amd import workloads as W

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sampler_small.npz")


@pytest.mark.parametrize("path", [0, 1])
def test_golden_vectors_through_dlk_sample(cuda, path):
    from diskllm_amd import api
    g = np.load(GOLDEN, allow_pickle=False)
    print(f"[case] golden vectors, {len(g['V'])} rows, path={path}", flush=True)
    bad = []
    for i in range(len(g["V"])):
        V, k = int(g["V"][i]), int(g["k"][i])
        n_out = min(V, 64)
        w = W.Workload(f"golden{i}", 1, V, np.ascontiguousarray(g["logits"][i:i + 1, :V]), g["seed"][i:i + 1].copy(),
                       temperature=float(g["T"][i]), top_k=k, top_p=float(g["p"][i]), min_p=float(g["mp"][i]),
                       n_out=n_out)
        db = api.to_device(w)
        api.sample(db, api.params_of(w, path=path))
        res = api.results(db)
        if int(res["ids"][0]) != int(g["token"][i]) or int(res["states"][0]) != int(g["state"][i]):
            bad.append((i, "token/state", int(res["ids"][0]), int(g["token"][i])))
            continue
        n = min(n_out, k if 0 < k < V else V)
        got = np.ascontiguousarray(res["cand_probs"][0, :n]).view(np.uint32)
        want = np.ascontiguousarray(g["cand_p"][i, :n]).view(np.uint32)
        if not np.array_equal(got, want):
            bad.append((i, "cand_p", int(np.sum(got != want))))
        assert res["status"] == 0
    assert not bad, bad[:8]
