"""Writes tests/golden/sampler_small.npz: small-vocabulary sampling vectors
(inputs and outputs) from the C oracle, checked first against the reference
compiled from its sources (oracle/_ref) when that is built.  Run from the repo
root: python tests/golden/make_golden.py"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

VMAX = 4096


def main() -> None:
    rng = np.random.default_rng(20261201)
    cases = []
    for V in (1, 2, 3, 31, 64, 257, 1000, 4096):
        for (T, k, p, mp) in ((1.0, 0, 1.0, 0.0), (0.8, 40, 0.95, 0.0), (1.2, 0, 0.9, 0.0), (0.6, 8, 0.5, 0.05),
                              (1.0, 0, 0.0, 0.0), (0.9, 100, 0.97, 0.0)):
            row = (rng.normal(0, 3, V) + (rng.random(V) < 0.02) * 6).astype(np.float32)
            if V > 8 and rng.random() < 0.3:
                row[rng.random(V) < 0.2] = -np.inf
            cases.append((V, T, k, p, mp, int(rng.integers(1, 2 ** 63)), row))
    n = len(cases)
    logits = np.zeros((n, VMAX), np.float32)
    cand_p = np.zeros((n, VMAX), np.float32)
    out = {k: [] for k in ("V", "T", "k", "p", "mp", "seed", "token", "state")}
    for i, (V, T, k, p, mp, seed, row) in enumerate(cases):
        o = O.sample_row(row, seed, T, k, p, mp, want_p=V)
        if O.ref("strict") is not None:
            tok, st, _, _ = O.ref_sample_row("strict", row, seed, T, k, p, mp)
            assert (tok, st) == (o["token"], o["state"]), i
        logits[i, :V] = row
        cand_p[i, :len(o["cand_p"])] = o["cand_p"]
        for key, val in (("V", V), ("T", T), ("k", k), ("p", p), ("mp", mp), ("seed", seed),
                         ("token", o["token"]), ("state", o["state"])):
            out[key].append(val)
    np.savez_compressed(os.path.join(ROOT, "tests", "golden", "sampler_small.npz"), logits=logits, cand_p=cand_p,
                        V=np.array(out["V"], np.int32), T=np.array(out["T"], np.float32),
                        k=np.array(out["k"], np.int32), p=np.array(out["p"], np.float32),
                        mp=np.array(out["mp"], np.float32), seed=np.array(out["seed"], np.uint64),
                        token=np.array(out["token"], np.int32), state=np.array(out["state"], np.uint64))
    print(f"wrote {n} cases")


if __name__ == "__main__":
    main()
