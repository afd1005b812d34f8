"""GPU tests of the boundary's contracts: the drop-in always returns a token
(src/sampler.c:136-234 has no failure return), workspaces are released with
their stream, a history longer than max_history is flagged on every path, and
the vocabulary table read from a GGUF file drives the device grammar mask and
the device decoding step exactly as the reference's tokenizer_init ->
tokenizer_decode_raw -> diskllm_grammar_apply_mask chain does."""
import ctypes as C
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

from diskllm_amd import _lib
from diskllm_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = O.ref("strict")
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def fptr(a):
    return a.ctypes.data_as(C.c_void_p)


# --- workspace lifetime --------------------------------------------------------------------------------

def test_release_stream_frees_workspace(cuda):
    """dlk_sample on a stream of its own grows that stream's workspace;
    dlk_release_stream frees it (device free memory back up), and a later call
    on the stream allocates afresh and is still exact."""
    import torch
    from diskllm_amd import api
    L = _lib.lib()
    w = W.c2(rows=8, vocab=151936)
    db = api.to_device(w)
    prm = api.params_of(w)
    orc = O.run_workload(w)
    st = torch.cuda.Stream()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    api.sample(db, prm, st.cuda_stream)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 < free0, (free0, free1)                      # the stream's workspace was allocated
    assert L.dlk_release_stream(st.cuda_stream) == _lib.DLK_OK
    free2 = torch.cuda.mem_get_info()[0]
    assert free2 - free1 >= (1 << 20), (free1, free2)         # ... and freed
    assert L.dlk_release_stream(st.cuda_stream) == _lib.DLK_OK  # nothing left to free
    np.testing.assert_array_equal(api.results(db)["ids"], orc["ids"])
    db.reset_rng()
    api.sample(db, prm, st.cuda_stream)                        # allocates afresh
    np.testing.assert_array_equal(api.results(db)["ids"], orc["ids"])
    assert L.dlk_release_stream(st.cuda_stream) == _lib.DLK_OK


# --- histories over max_history ------------------------------------------------------------------------

@pytest.mark.parametrize("top_k", [0, 40])
def test_long_history_over_max_history(cuda, top_k):
    """max_history above 1024 (penalties on a scratch copy first): a row whose
    history exceeds max_history gets id -1, DLK_STATUS_HISTORY_TOO_LONG and keeps
    its rng state; the other rows are the oracle's."""
    from diskllm_amd import api
    rng = np.random.default_rng(31 + top_k)
    V, max_hist = 30000, 2000
    lens = [1500, 2500, 10, 2000, 0]
    rows = len(lens)
    hist = []
    for n in lens:
        h = rng.integers(0, V, n).astype(np.int32)
        if n > 100:
            h[: n // 3] = h[n // 3: 2 * (n // 3)]                  # repeats
        hist.append(h)
    off = np.zeros(rows + 1, np.int32)
    off[1:] = np.cumsum(lens)
    ids = np.concatenate(hist).astype(np.int32)
    lg = rng.normal(0, 2, (rows, V)).astype(np.float32)
    w = W.Workload("LONG", rows, V, lg, rng.integers(1, 2 ** 63, rows, dtype=np.uint64), temperature=0.9,
                   top_k=top_k, top_p=0.95, repeat_penalty=1.2, frequency_penalty=0.1, presence_penalty=0.4,
                   order=W.ORDER_NORTH_STAR, hist_off=off, hist_ids=ids)
    _announce(f"long history top_k={top_k} lens={lens} max_history={max_hist}")
    db = api.to_device(w)
    api.sample(db, api.params_of(w, max_history=max_hist))
    res = api.results(db)
    assert res["status"] == _lib.DLK_STATUS_HISTORY_TOO_LONG
    for r in range(rows):
        if lens[r] > max_hist:
            assert res["ids"][r] == -1
            assert int(res["states"][r]) == int(w.seeds[r])
        else:
            o = O.sample_row(O.prepared_row(w, r), int(w.seeds[r]), w.temperature, w.top_k, w.top_p, w.min_p)
            assert res["ids"][r] == o["token"], r
            assert int(res["states"][r]) == o["state"], r


def test_penalties_more_distinct_ids_than_slots(cuda):
    """dlk_apply_penalties with a row holding more distinct ids than its LDS
    hash table (16,384 slots): the counting scan takes over, same values as the
    oracle's per-id restatement."""
    import torch
    L = _lib.lib()
    rng = np.random.default_rng(41)
    V = 60000
    h0 = rng.permutation(V)[:20000].astype(np.int32)             # 20,000 distinct ids
    h0 = np.concatenate([h0, h0[:3000], [-1, V, V + 5]]).astype(np.int32)
    h1 = rng.integers(0, V, 9000).astype(np.int32)
    hist = [h0, h1]
    hoff = np.array([0, h0.size, h0.size + h1.size], np.int32)
    hids = np.concatenate(hist).astype(np.int32)
    logits = rng.normal(0, 2, (2, V)).astype(np.float32)
    dev = torch.device("cuda:0")
    d = torch.from_numpy(logits).to(dev)
    d_hoff, d_hids = torch.from_numpy(hoff).to(dev), torch.from_numpy(hids).to(dev)
    rc = L.dlk_apply_penalties(d.data_ptr(), V, 2, V, d_hoff.data_ptr(), d_hids.data_ptr(), W.ORDER_NORTH_STAR, 1.3,
                               0.2, 0.6, None)
    assert rc == _lib.DLK_OK
    got = d.cpu().numpy()
    for r in range(2):
        np.testing.assert_array_equal(got[r], O.penalties(logits[r], hist[r], W.ORDER_NORTH_STAR, 1.3, 0.2, 0.6))


# --- the drop-in always returns a token ----------------------------------------------------------------

DROPIN_TIMEOUT_CHILD = r"""
import ctypes as C, os, sys
import numpy as np
sys.path.insert(0, os.environ["DLK_ROOT"])
from diskllm_amd import _lib
from oracle import oracle as O
L, R = _lib.lib(), O.ref("strict")
R.sampler_create.restype = C.c_void_p
R.sampler_create.argtypes = [C.POINTER(O.SamplerConfig)]
R.sampler_sample.restype = C.c_int
R.sampler_sample.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
R.sampler_free.argtypes = [C.c_void_p]
rng = np.random.default_rng(51)
V = 151936
for (T, p, seed) in ((1.0, 0.9, 7), (0.7, 0.95, 0), (1.3, 1.0, 12345)):
    print(f"[case] drop-in sync-timeout recovery T={T} p={p} seed={seed}", flush=True)
    s = L.sampler_create(C.byref(_lib.SamplerConfig(T, 0, p, 0.0, seed)))
    r = R.sampler_create(C.byref(O.SamplerConfig(T, 0, p, 0.0, seed)))
    assert s and r
    for step in range(5):
        row = (rng.normal(0, 2, V) + (rng.random(V) < 0.001) * 9).astype(np.float32)
        a, b = row.copy(), row.copy()
        ta = L.sampler_sample(s, a.ctypes.data_as(C.c_void_p), V)
        tb = R.sampler_sample(r, b.ctypes.data_as(C.c_void_p), V)
        assert ta == tb, (T, p, seed, step, ta, tb)
    L.sampler_free(s)
    R.sampler_free(r)
print("child ok", flush=True)
"""


@needs_ref
def test_dropin_sync_timeout_recovery(cuda):
    """Every first attempt of sampler_sample forced onto the fused kernel
    instance whose cross-workgroup waits give up (DLK_DROPIN_PATH=3, read at
    sampler_create): the drop-in notices DLK_STATUS_SYNC_TIMEOUT, runs the row
    again on the row kernel from the same rng state, and returns the strict
    reference build's token sequence (which also checks the rng carried on).
    Run in a child process: the hook is read from its environment."""
    # the forced path does time out (the recovery is what is tested)
    from diskllm_amd import api
    w = W.c2(rows=16, vocab=151936)
    db = api.to_device(w)
    api.sample(db, api.params_of(w, path=_lib.PATH_FULL_NO_WAIT))
    assert api.results(db)["status"] & _lib.DLK_STATUS_SYNC_TIMEOUT
    env = dict(os.environ, DLK_DROPIN_PATH=str(_lib.PATH_FULL_NO_WAIT), DLK_ROOT=ROOT)
    r = subprocess.run([sys.executable, "-u", "-c", DROPIN_TIMEOUT_CHILD], env=env, capture_output=True, text=True,
                       timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "child ok" in r.stdout
    assert "could not reach the GPU" not in r.stderr


# --- GGUF vocabulary -> device grammar mask and decoding step ---------------------------------------------

def _gguf_str(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def _write_gguf_tokens(path, tokens):
    """A GGUF v3 file with an architecture string and the tokens string array
    (the layout tokenizer_init reads, src/tokenizer.c:247-300)."""
    kvs = _gguf_str(b"general.architecture") + struct.pack("<I", 8) + _gguf_str(b"qwen2")
    kvs += _gguf_str(b"tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, len(tokens))
    kvs += b"".join(_gguf_str(t) for t in tokens)
    kvs += _gguf_str(b"tokenizer.ggml.eos_token_id") + struct.pack("<II", 4, 3)
    with open(path, "wb") as f:
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 3) + kvs)


def _ref_tokenizer():
    path = os.path.join(ROOT, "oracle", "_ref", "libref_tokenizer.so")
    if not os.path.exists(path):
        return None
    T = C.CDLL(path)
    T.tokenizer_init.restype = C.c_void_p
    T.tokenizer_init.argtypes = [C.c_char_p]
    T.tokenizer_decode_raw.restype = C.c_void_p
    T.tokenizer_decode_raw.argtypes = [C.c_void_p, C.c_int32]
    T.tokenizer_free.argtypes = [C.c_void_p]
    return T


def _json_tokens(rng, n):
    alpha = list(b'{}[]":, 0123456789abcdefxyz_\\') + [0xC4, 0xA0]
    toks = [b"{", b"[", b"}", b"]", b'"', b" ", b'{"bbox_2d": [', b", ", b"", "Ġthe".encode(), b"<0x0A>"]
    while len(toks) < n:
        k = int(min(12, rng.geometric(0.35)))
        toks.append(bytes(int(c) for c in rng.choice(alpha, k)))
    return toks


@needs_ref
@pytest.mark.skipif(_ref_tokenizer() is None, reason="oracle/_ref/libref_tokenizer.so not built")
@pytest.mark.parametrize("path", [0, 1])
def test_gguf_vocab_drives_device_grammar(cuda, tmp_path, path):
    """A GGUF file's tokens -> dlk_vocab_csr_from_gguf -> the device grammar mask
    (dlk_grammar_mask) and a 12-step dlk_sample_grammar loop, against the
    reference's own chain on the same file: tokenizer_init, tokenizer_decode_raw
    as the mask callback of diskllm_grammar_apply_mask, sampler_sample and
    diskllm_grammar_advance (src/core/sampler_api.c:48-73,
    src/core/grammar.c:275-308, src/tokenizer.c:247-300,377-380).  The table
    covers 40 ids past the file's strings (NULL from tokenizer_decode_raw,
    empty entries here: masked either way)."""
    import torch
    L = _lib.lib()
    T = _ref_tokenizer()
    rng = np.random.default_rng(61 + path)
    n_file = 4000
    V = n_file + 40
    toks = _json_tokens(rng, n_file)
    gpath = str(tmp_path / "vocab.gguf")
    _write_gguf_tokens(gpath, toks)
    off, data, n = _lib.vocab_csr_from_gguf(gpath, V)
    assert n == n_file
    tok = T.tokenizer_init(gpath.encode())
    assert tok
    cb = C.cast(T.tokenizer_decode_raw, C.c_void_p)
    eos = 3
    dev = torch.device("cuda:0")
    d_off = torch.from_numpy(off.view(np.int32)).to(dev)
    d_bytes = torch.from_numpy(data if data.size else np.zeros(1, np.uint8)).to(dev)
    W_ = (V + 31) // 32
    try:
        # 1. masks at several grammar positions
        for mode in (b"root ::= object | value", b"receipt bbox_2d"):
            for buf in (b"", b" {", b'{"bbox_2d": [1, 2', b'{"a": [1, "x'):
                _announce(f"gguf mask path={path} mode={mode} buffer={buf!r}")
                st = _lib.GrammarRow()
                L.dlk_grammar_row_init(C.byref(st), L.dlk_grammar_mode_of(mode))
                L.dlk_grammar_row_feed(C.byref(st), buf, len(buf))
                d_st = torch.frombuffer(bytearray(bytes(st)), dtype=torch.uint8).to(dev)
                row = rng.normal(0, 1, V).astype(np.float32)
                d_lg = torch.from_numpy(row).to(dev)
                d_mask = torch.zeros(W_, dtype=torch.int32, device=dev)
                d_valid = torch.zeros(1, dtype=torch.int32, device=dev)
                rc = L.dlk_grammar_mask(d_off.data_ptr(), d_bytes.data_ptr(), V, d_st.data_ptr(), 1, eos,
                                        d_mask.data_ptr(), W_, d_lg.data_ptr(), V, d_valid.data_ptr(), None)
                assert rc == _lib.DLK_OK
                g = REF.diskllm_grammar_init_from_str(mode)
                REF.diskllm_grammar_advance(g, buf)
                want = row.copy()
                nv = REF.diskllm_grammar_apply_mask(g, want, V, C.c_void_p(tok), cb, eos)
                REF.diskllm_grammar_free(g)
                got = d_lg.cpu().numpy()
                np.testing.assert_array_equal(got, want)
                bits = (d_mask.cpu().numpy().view(np.uint32)[np.arange(V) >> 5] >>
                        (np.arange(V) & 31).astype(np.uint32)) & 1
                np.testing.assert_array_equal(bits.astype(bool), np.isfinite(want))
                assert int(d_valid.cpu().item()) == nv
        # 2. a decoding loop on the device against the reference's per-row chain
        modes = [b"root ::= object | value", b"receipt bbox_2d"]
        R, steps = len(modes), 12
        Tmp, K_, P_ = 0.9, (0 if path == 0 else 30), 0.95
        seeds = rng.integers(1, 2 ** 63, R, dtype=np.uint64)
        states = (_lib.GrammarRow * R)()
        for i, mode in enumerate(modes):
            L.dlk_grammar_row_init(C.byref(states[i]), L.dlk_grammar_mode_of(mode))
        d_states = torch.frombuffer(bytearray(bytes(states)), dtype=torch.uint8).to(dev)
        d_rng = torch.from_numpy(seeds.view(np.int64).copy()).to(dev)
        d_mask = torch.zeros((R, W_), dtype=torch.int32, device=dev)
        d_out = torch.zeros(R, dtype=torch.int32, device=dev)
        d_status = torch.zeros(1, dtype=torch.int32, device=dev)
        prm = _lib.SampleParams(Tmp, K_, P_, 0.0, 1.0, 0.0, 0.0, _lib.ORDER_REFERENCE, 1, 0, path)
        step_logits = [rng.normal(0, 2, (R, V)).astype(np.float32) for _ in range(steps)]
        for lg in step_logits:
            lg[:, :11] += 3.0                                      # the JSON pieces
        got = np.zeros((steps, R), np.int32)
        _announce(f"gguf decoding loop path={path} steps={steps}")
        for s_ in range(steps):
            d_lg = torch.from_numpy(step_logits[s_]).to(dev)
            b = _lib.Batch(logits=d_lg.data_ptr(), ld=V, hist_off=None, hist_ids=None, mask=d_mask.data_ptr(),
                           mask_ld=W_, mask_row=None, rng=d_rng.data_ptr(), out_ids=d_out.data_ptr(),
                           out_cand_ids=None, out_cand_probs=None, out_cand_logprobs=None,
                           status=d_status.data_ptr())
            assert L.dlk_sample_grammar(C.byref(b), R, V, C.byref(prm), d_off.data_ptr(), d_bytes.data_ptr(),
                                        d_states.data_ptr(), eos, None) == _lib.DLK_OK
            got[s_] = d_out.cpu().numpy()
        assert int(d_status.cpu().item()) == 0
        REF.sampler_create.restype = C.c_void_p
        REF.sampler_create.argtypes = [C.POINTER(O.SamplerConfig)]
        REF.sampler_sample.restype = C.c_int
        REF.sampler_sample.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
        REF.sampler_free.argtypes = [C.c_void_p]
        for i, mode in enumerate(modes):
            g = REF.diskllm_grammar_init_from_str(mode)
            # the reference seeds through sampler_create; the device rows start from the state itself
            smp = REF.sampler_create(C.byref(O.SamplerConfig(Tmp, K_, P_, 0.0, int(seeds[i]))))
            try:
                for s_ in range(steps):
                    row = step_logits[s_][i].copy()
                    REF.diskllm_grammar_apply_mask(g, row, V, C.c_void_p(tok), cb, eos)
                    t = REF.sampler_sample(smp, row.ctypes.data_as(C.c_void_p), V)
                    assert got[s_, i] == t, (mode, s_, got[:, i], t)
                    if t != eos:
                        p = T.tokenizer_decode_raw(tok, t)
                        if p:
                            REF.diskllm_grammar_advance(g, C.string_at(p))
            finally:
                REF.sampler_free(smp)
                REF.diskllm_grammar_free(g)
    finally:
        T.tokenizer_free(tok)
