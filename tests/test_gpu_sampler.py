"""GPU parity: libdiskllm_amd.so against the oracle, bit-exact on token ids,
RNG states and mask bits; candidate probabilities within 1e-5 relative.

Every case prints its name, seed and shape before touching the GPU.
"""
import numpy as np
import pytest

from oracle import oracle as O
from diskllm_amd import workloads as W

pytestmark = pytest.mark.gpu

PROB_RTOL = 1e-5   # candidate probabilities / log-probs vs the oracle


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def run_gpu(w, rows=None, path=0):
    from diskllm_amd import api
    db = api.to_device(w, rows=rows)
    api.sample(db, api.params_of(w, path=path))
    return api.results(db)


def oracle_rows(w, rows):
    out = []
    for r in rows:
        out.append(O.sample_row(O.prepared_row(w, r), int(w.seeds[r]), w.temperature, w.top_k, w.top_p, w.min_p,
                                want_p=w.n_out))
    return out


def final_probs(o, n_out):
    """Final sampling probability of the first n_out candidates (0 if cut)."""
    k = o["k"]
    p = o["cand_p"]
    out = np.zeros(min(n_out, k), np.float32)
    for j in range(min(n_out, k)):
        v = np.float32(p[j])
        if o["inv_s2"] != 0.0:          # min-p active
            raise AssertionError("use min_p = 0 in candidate-output tests")
        if o["inv_s3"] != 0.0:          # top-p active: kept iff j < nk
            v = np.float32(v * np.float32(o["inv_s3"])) if j < o["nk"] else np.float32(0.0)
        out[j] = v
    return out


def assert_rows_match(w, res, rows, check_cands=True):
    orc = oracle_rows(w, rows)
    bad = [(r, int(res["ids"][j]), o["token"]) for j, (r, o) in enumerate(zip(rows, orc)) if res["ids"][j] != o["token"]]
    assert not bad, f"{w.name}: token mismatches (row, gpu, oracle): {bad[:10]} of {len(bad)}"
    st = [(r, int(res["states"][j]), o["state"]) for j, (r, o) in enumerate(zip(rows, orc))
          if int(res["states"][j]) != o["state"]]
    assert not st, f"{w.name}: rng state mismatches {st[:5]}"
    assert res["status"] == 0
    if check_cands and w.n_out and "cand_ids" in res:
        for j, (r, o) in enumerate(zip(rows, orc)):
            n = min(w.n_out, o["k"])
            np.testing.assert_array_equal(res["cand_ids"][j, :n], o["cand_idx"][:n])
            np.testing.assert_allclose(res["cand_probs"][j, :n], o["cand_p"][:n], rtol=PROB_RTOL, atol=0)
            fp = final_probs(o, w.n_out)
            with np.errstate(divide="ignore"):
                lp = np.where(fp > 0, np.log(fp.astype(np.float64)), -np.inf).astype(np.float32)
            got = res["cand_logprobs"][j, :n]
            assert np.array_equal(np.isinf(got), np.isinf(lp)), f"row {r}: cut pattern differs"
            fin = np.isfinite(lp)
            np.testing.assert_allclose(got[fin], lp[fin], rtol=PROB_RTOL, atol=1e-7)
    return orc


def test_device_expf_exhaustive(cuda):
    """dlk_expf == host libm expf on every non-NaN float (2^32 inputs, 2^26 per slice)."""
    import torch
    from diskllm_amd import _lib
    _announce("expf exhaustive, 64 slices of 2^26")
    n = 1 << 26
    xs = torch.empty(n, dtype=torch.int32, device="cuda")
    ys = torch.empty(n, dtype=torch.float32, device="cuda")
    host = np.empty(n, np.float32)
    base = torch.arange(n, dtype=torch.int64, device="cuda")
    bad_total = 0
    for s in range(64):
        first = s * n
        v = base + first
        xs.copy_(torch.where(v >= 2 ** 31, v - 2 ** 32, v).to(torch.int32))
        _lib.check(_lib.lib().dlk_expf(xs.data_ptr(), ys.data_ptr(), n, torch.cuda.current_stream().cuda_stream),
                   "dlk_expf")
        O.lib().orc_expf_bits(first, n, host, 16)
        g = ys.cpu().numpy().view(np.uint32)
        h = host.view(np.uint32)
        xin = (np.arange(n, dtype=np.uint64) + first).astype(np.uint32)
        nan_in = ((xin & 0x7F800000) == 0x7F800000) & ((xin & 0x007FFFFF) != 0)
        bad = np.nonzero((g != h) & ~nan_in)[0]
        if bad.size:
            print("mismatch", hex(int(xin[bad[0]])), hex(int(g[bad[0]])), hex(int(h[bad[0]])))
        bad_total += bad.size
    assert bad_total == 0


@pytest.mark.parametrize("path", [0, 1])
def test_c1_single_row(cuda, path):
    w = W.c1()
    _announce(f"C1 V={w.vocab} path={path}")
    res = run_gpu(w, path=path)
    assert_rows_match(w, res, [0])


def test_c2_batch64_full_vocab(cuda):
    w = W.c2()
    _announce(f"C2 rows={w.rows} V={w.vocab}")
    res = run_gpu(w)
    assert_rows_match(w, res, list(range(w.rows)))


def test_c2_reference_order(cuda):
    w = W.c2(seed=12, rows=16)
    w.order = W.ORDER_REFERENCE
    _announce(f"C2 reference penalty order rows={w.rows}")
    res = run_gpu(w)
    assert_rows_match(w, res, list(range(w.rows)))


@pytest.mark.parametrize("path", [0, 1])
def test_c3_packed_mask(cuda, path):
    w = W.c3()
    _announce(f"C3 rows={w.rows} V={w.vocab} path={path}")
    res = run_gpu(w, path=path)
    orc = assert_rows_match(w, res, list(range(w.rows)))
    # row 3 allows exactly one token: it must be returned
    allowed = np.nonzero(np.unpackbits(w.mask[3].view(np.uint8), bitorder="little")[:w.vocab])[0]
    assert len(allowed) == 1 and res["ids"][3] == allowed[0]
    assert orc[3]["token"] == allowed[0]


def test_c4_dfa_masks(cuda):
    from diskllm_amd import api
    w = W.c4()
    _announce(f"C4 V={w.vocab} rows={w.rows}")
    got = api.dfa_masks(w.dfa.offsets, w.dfa.data, w.dfa.trans, w.dfa_states, w.vocab).cpu().numpy().view(np.uint32)
    for r in range(w.rows):
        ref = O.dfa_mask(w.dfa, int(w.dfa_states[r]), w.vocab)
        np.testing.assert_array_equal(got[r], ref, err_msg=f"row {r} state {w.dfa_states[r]}")


@pytest.mark.parametrize("path", [0, 1])
def test_c5_gemma_dfa_topk(cuda, path):
    w = W.c5()
    _announce(f"C5 rows={w.rows} V={w.vocab} path={path}")
    res = run_gpu(w, path=path)
    assert_rows_match(w, res, list(range(w.rows)))


def test_device_tanhf_exhaustive(cuda):
    """dlk_softcap with cap 1 (1 * tanhf(x / 1) = tanhf(x) bit for bit) == host libm
    tanhf on every non-NaN float (2^32 inputs, 2^26 per slice)."""
    import torch
    from diskllm_amd import _lib
    _announce("tanhf exhaustive through dlk_softcap(cap=1), 64 slices of 2^26")
    n = 1 << 26
    xs = torch.empty(n, dtype=torch.int32, device="cuda")
    host = np.empty(n, np.float32)
    base = torch.arange(n, dtype=torch.int64, device="cuda")
    bad_total = 0
    for s in range(64):
        first = s * n
        v = base + first
        xs.copy_(torch.where(v >= 2 ** 31, v - 2 ** 32, v).to(torch.int32))
        _lib.check(_lib.lib().dlk_softcap(xs.data_ptr(), n, 1, n, 1.0, torch.cuda.current_stream().cuda_stream),
                   "dlk_softcap")
        O.lib().orc_tanhf_bits(first, n, host, 16)
        g = xs.cpu().numpy().view(np.uint32)
        h = host.view(np.uint32)
        xin = (np.arange(n, dtype=np.uint64) + first).astype(np.uint32)
        nan_in = ((xin & 0x7F800000) == 0x7F800000) & ((xin & 0x007FFFFF) != 0)
        bad = np.nonzero((g != h) & ~nan_in)[0]
        if bad.size:
            print("mismatch", hex(int(xin[bad[0]])), hex(int(g[bad[0]])), hex(int(h[bad[0]])))
        bad_total += bad.size
    assert bad_total == 0


@pytest.mark.parametrize("rows,vocab,ld,offset,cap", [(3, 262144, 262144, 0, 30.0), (5, 1001, 1003, 1, 30.0),
                                                      (2, 151936, 152000, 0, 50.0), (1, 7, 7, 3, 0.5),
                                                      (4, 4096, 4100, 0, 0.0),
                                                      # float4 path (ld % 4 == 0, aligned) with ragged row ends
                                                      (2, 1001, 1004, 0, 30.0), (1, 151937, 151940, 0, 30.0)])
def test_softcap_rows_vs_oracle(cuda, rows, vocab, ld, offset, cap):
    """dlk_softcap over strided rows (float4 and scalar paths, ragged tails) ==
    the oracle's cap * tanhf(x / cap), bit for bit; the padding past vocab and
    the rows for cap <= 0 are left alone."""
    import torch
    from diskllm_amd import _lib
    _announce(f"softcap rows={rows} vocab={vocab} ld={ld} offset={offset} cap={cap}")
    rng = np.random.default_rng(vocab + rows)
    buf = rng.normal(0.0, 40.0, size=rows * ld + offset).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-38, -1e-45, 22.0 * 30, 3.4e38, -3.4e38], np.float32)
    buf[offset:offset + min(special.size, vocab)] = special[:vocab]
    d = torch.from_numpy(buf.copy()).cuda()
    _lib.check(_lib.lib().dlk_softcap(d.data_ptr() + 4 * offset, ld, rows, vocab, cap,
                                      torch.cuda.current_stream().cuda_stream), "dlk_softcap")
    got = d.cpu().numpy()
    want = buf.copy()
    for r in range(rows):
        seg = want[offset + r * ld: offset + r * ld + vocab]
        O.lib().orc_softcap(seg, seg, vocab, np.float32(cap))
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("path", [0, 1])
def test_softcap_then_sample_vs_oracle(cuda, path):
    """The reference's decode epilogue order on the device: soft-cap (cap 30, the
    Gemma value) in place, then the C5 sampling step (DFA mask, repetition
    penalty, top-k 64, top-p 0.95) on 48 rows; token ids and rng states equal to
    the oracle's on the capped logits."""
    from diskllm_amd import api, _lib
    import torch
    w = W.c5(rows=48)
    _announce(f"softcap 30 -> C5 rows={w.rows} V={w.vocab} path={path}")
    db = api.to_device(w)
    _lib.check(_lib.lib().dlk_softcap(db.logits.data_ptr(), w.vocab, w.rows, w.vocab, 30.0,
                                      torch.cuda.current_stream().cuda_stream), "dlk_softcap")
    api.sample(db, api.params_of(w, path=path))
    res = api.results(db)
    capped = w.logits.copy()
    O.lib().orc_softcap(capped.reshape(-1), capped.reshape(-1), capped.size, np.float32(30.0))
    w.logits = capped
    assert_rows_match(w, res, list(range(w.rows)))
