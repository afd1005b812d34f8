"""GPU parity of the drop-in boundary (include/sampler.h, include/grammar.h) and
of the batched grammar / penalty entry points, against the reference compiled
from its sources (oracle/_ref) and the oracle."""
import ctypes as C

import numpy as np
import pytest

from diskllm_amd import _lib
from diskllm_amd import workloads as W
from oracle import oracle as O

pytestmark = pytest.mark.gpu
REF = O.ref("strict")
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built")


def _ref_sampler_api():
    REF.sampler_create.restype = C.c_void_p
    REF.sampler_create.argtypes = [C.POINTER(O.SamplerConfig)]
    REF.sampler_free.argtypes = [C.c_void_p]
    REF.sampler_sample.restype = C.c_int
    REF.sampler_sample.argtypes = [C.c_void_p, C.c_void_p, C.c_int]


def fptr(a):
    return a.ctypes.data_as(C.c_void_p)


@needs_ref
@pytest.mark.parametrize("V", [1, 3, 100, 4097, 50000, 151936])
def test_dropin_sampler_sequence(cuda, V):
    """sampler_create + repeated sampler_sample (the rng state carried between
    calls) against the reference's, on rows of every kind of configuration."""
    L = _lib.lib()
    _ref_sampler_api()
    rng = np.random.default_rng(V)
    for (T, k, p, mp) in ((1.0, 0, 1.0, 0.0), (0.8, 40, 0.95, 0.0), (1.2, 0, 0.9, 0.0), (0.6, 8, 0.5, 0.05),
                          (0.0, 0, 0.9, 0.0), (0.9, 300, 0.97, 0.0), (1.0, 0, 0.0, 0.0)):
        seed = int(rng.integers(0, 2 ** 63)) if rng.random() < 0.8 else 0
        print(f"[case] V={V} T={T} k={k} p={p} minp={mp} seed={seed}", flush=True)
        cfg = _lib.SamplerConfig(T, k, p, mp, seed)
        rcfg = O.SamplerConfig(T, k, p, mp, seed)
        s, r = L.sampler_create(C.byref(cfg)), REF.sampler_create(C.byref(rcfg))
        assert s and r
        try:
            for step in range(4):
                row = (rng.normal(0, 3, V) + (rng.random(V) < 0.01) * 6).astype(np.float32)
                if step == 2:
                    row = np.round(row)
                a, b = row.copy(), row.copy()
                ta = L.sampler_sample(s, fptr(a), V)
                tb = REF.sampler_sample(r, fptr(b), V)
                assert ta == tb, (V, T, k, p, mp, step, ta, tb)
                np.testing.assert_array_equal(a, row)                  # the row is read only
        finally:
            L.sampler_free(s)
            REF.sampler_free(r)


@needs_ref
def test_dropin_greedy_and_penalties(cuda):
    L = _lib.lib()
    rng = np.random.default_rng(3)
    for V in (1, 2, 1000, 151936):
        row = np.round(rng.normal(0, 2, V)).astype(np.float32)
        assert L.greedy_sample(fptr(row), V) == REF.greedy_sample(row, V)
        if V > 1:
            row[0] = np.nan
            assert L.greedy_sample(fptr(row), V) == REF.greedy_sample(row, V) == 0
        row = rng.normal(0, 2, V).astype(np.float32)
        seen = rng.integers(-3, V + 3, 300).astype(np.int32)
        seen[:40] = seen[40:80]                                        # repeats
        for pen in (1.3, 1.0, 0.7):
            a, b = row.copy(), row.copy()
            L.sampler_apply_repetition_penalty(fptr(a), V, fptr(seen), seen.size, pen)
            REF.sampler_apply_repetition_penalty(b, V, seen, seen.size, np.float32(pen))
            np.testing.assert_array_equal(a, b)
        for pp in (0.5, 0.0, -1.25):
            a, b = row.copy(), row.copy()
            L.sampler_apply_presence_penalty(fptr(a), V, fptr(seen), seen.size, pp)
            REF.sampler_apply_presence_penalty(b, V, seen, seen.size, np.float32(pp))
            np.testing.assert_array_equal(a, b)


ALPHABET = list(b'{}[]":,\\ \t\n0123456789abdextnco_') + [0x80, 0xC4, 0xA0]


def random_vocab(rng, V):
    toks = []
    for t in range(V):
        u = rng.random()
        if u < 0.003:
            toks.append(None)
        elif u < 0.006:
            toks.append(b"")
        else:
            n = int(min(16, rng.geometric(0.3)))
            toks.append(bytes(int(b) for b in rng.choice(ALPHABET, n)))
    toks[:8] = [b"{", b"[", b"}", b"]", b'"', b" ", b'{"bbox_2d": [', b", "]
    return toks


class Vocab:
    """A get_token_str callback over Python byte strings (NULL for None)."""
    CB = C.CFUNCTYPE(C.c_void_p, C.c_void_p, C.c_int)

    def __init__(self, toks):
        self.bufs = [None if t is None else C.create_string_buffer(t) for t in toks]
        self.addr = [None if b is None else C.addressof(b) for b in self.bufs]
        self.cb = self.CB(lambda ctx, i: self.addr[i])
        self.ptr = C.cast(self.cb, C.c_void_p)


BUFFERS = [b"", b"  ", b" {", b'{"bbox_2d": [1, 2', b'{"bbox_2d": [1,2,3,4], "text_content": "ab\\"',
           b'{"bbox_2d":[1,2,3,4],"text_content":"hi"}', b'[{"a": "x}"', b"x", b'{"a": [1, 2]}', b"}"]


@needs_ref
@pytest.mark.parametrize("mode", [b"receipt bbox_2d", b"root ::= object | value", b"free text"])
def test_dropin_apply_mask_vs_reference(cuda, mode):
    L = _lib.lib()
    rng = np.random.default_rng(len(mode))
    for V in (300, 151936):
        voc = Vocab(random_vocab(rng, V))
        # the callback runs in Python: the Qwen-sized vocabulary gets a few positions
        for buf in (BUFFERS if V < 1000 else BUFFERS[2:5]):
            print(f"[case] mode={mode} V={V} buffer={buf!r}", flush=True)
            g, h = L.diskllm_grammar_init_from_str(mode), REF.diskllm_grammar_init_from_str(mode)
            try:
                L.diskllm_grammar_advance(g, buf)
                REF.diskllm_grammar_advance(h, buf)
                for eos in ((3, -1, V - 1) if V < 1000 else (3,)):
                    row = rng.normal(0, 1, V).astype(np.float32)
                    a, b = row.copy(), row.copy()
                    na = L.diskllm_grammar_apply_mask(g, fptr(a), V, None, voc.ptr, eos)
                    nb = REF.diskllm_grammar_apply_mask(h, b, V, None, voc.ptr, eos)
                    assert na == nb, (mode, buf, eos, na, nb)
                    np.testing.assert_array_equal(a, b)
            finally:
                L.diskllm_grammar_free(g)
                REF.diskllm_grammar_free(h)


def test_grammar_mask_batched(cuda):
    """dlk_grammar_mask over many rows in different positions at once, against
    the oracle's apply_mask restatement (src/core/grammar.c:275-308)."""
    import torch
    L = _lib.lib()
    rng = np.random.default_rng(11)
    V = 20000
    toks = random_vocab(rng, V)
    strs = [t or b"" for t in toks]
    off = np.zeros(V + 1, np.uint32)
    off[1:] = np.cumsum([len(s) for s in strs])
    data = np.frombuffer(b"".join(strs), np.uint8).copy()
    rows = []
    for mode in (b"receipt bbox_2d", b"object", b"plain"):
        for buf in BUFFERS:
            rows.append((mode, buf))
    R = len(rows)
    states = (_lib.GrammarRow * R)()
    for i, (mode, buf) in enumerate(rows):
        L.dlk_grammar_row_init(C.byref(states[i]), L.dlk_grammar_mode_of(mode))
        L.dlk_grammar_row_feed(C.byref(states[i]), buf, len(buf))
    dev = torch.device("cuda:0")
    d_off = torch.from_numpy(off.view(np.int32)).to(dev)
    d_bytes = torch.from_numpy(data).to(dev)
    d_states = torch.frombuffer(bytearray(bytes(states)), dtype=torch.uint8).to(dev)
    W_ = (V + 31) // 32
    d_mask = torch.zeros((R, W_), dtype=torch.int32, device=dev)
    logits = rng.normal(0, 1, (R, V)).astype(np.float32)
    d_logits = torch.from_numpy(logits).to(dev)
    d_valid = torch.zeros(R, dtype=torch.int32, device=dev)
    eos = 7
    rc = L.dlk_grammar_mask(d_off.data_ptr(), d_bytes.data_ptr(), V, d_states.data_ptr(), R, eos, d_mask.data_ptr(),
                            W_, d_logits.data_ptr(), V, d_valid.data_ptr(), None)
    assert rc == 0
    torch.cuda.synchronize()
    mask = d_mask.cpu().numpy().view(np.uint32)
    got_logits = d_logits.cpu().numpy()
    valid = d_valid.cpu().numpy()
    for i, (mode, buf) in enumerate(rows):
        g = O.grammar(mode)
        O.lib().orc_grammar_advance(C.byref(g), buf)
        exp_logits, n = O.grammar_mask(g, off, data, eos, logits[i])
        np.testing.assert_array_equal(got_logits[i], exp_logits)
        bits = (mask[i][np.arange(V) >> 5] >> (np.arange(V) & 31).astype(np.uint32)) & 1
        np.testing.assert_array_equal(bits.astype(bool), np.isfinite(exp_logits))
        assert valid[i] == n


def test_apply_penalties_batched(cuda):
    import torch
    L = _lib.lib()
    rng = np.random.default_rng(12)
    rows, V = 6, 40000
    logits = rng.normal(0, 2, (rows, V)).astype(np.float32)
    hist = [rng.integers(-2, V + 2, n).astype(np.int32) for n in (0, 1, 50, 256, 5000, 300)]
    hist[3][:100] = hist[3][100:200]
    hoff = np.zeros(rows + 1, np.int32)
    hoff[1:] = np.cumsum([h.size for h in hist])
    hids = np.concatenate(hist).astype(np.int32)
    dev = torch.device("cuda:0")
    d_hoff = torch.from_numpy(hoff).to(dev)          # kept alive across the asynchronous call
    d_hids = torch.from_numpy(hids).to(dev)
    for order in (W.ORDER_REFERENCE, W.ORDER_NORTH_STAR):
        d = torch.from_numpy(logits).to(dev)
        rc = L.dlk_apply_penalties(d.data_ptr(), V, rows, V, d_hoff.data_ptr(), d_hids.data_ptr(), order, 1.2, 0.3,
                                   0.5, None)
        assert rc == 0
        torch.cuda.synchronize()
        got = d.cpu().numpy()
        for r in range(rows):
            np.testing.assert_array_equal(got[r], O.penalties(logits[r], hist[r], order, 1.2, 0.3, 0.5))


@pytest.mark.parametrize("path", [0, 1])
def test_sample_grammar_device_loop(cuda, path):
    """dlk_sample_grammar for a number of steps -- each row's grammar mask, the
    draw, and the row's state advanced by the drawn token, all on the device --
    against the oracle's apply_mask -> sample -> advance sequence per row
    (src/core/sampler_api.c:48-73), with the EOS rule and the rng carried on."""
    import torch
    L = _lib.lib()
    rng = np.random.default_rng(21)
    V = 3000
    toks = random_vocab(rng, V)
    strs = [t or b"" for t in toks]
    off = np.zeros(V + 1, np.uint32)
    off[1:] = np.cumsum([len(s) for s in strs])
    data = np.frombuffer(b"".join(strs), np.uint8).copy()
    eos = 9
    modes = [b"receipt bbox_2d", b"root ::= object | value", b"free text", b"root ::= object | value"]
    R, steps = len(modes), 16
    T_, K_, P_ = 0.9, (0 if path == 0 else 40), 0.95
    states = (_lib.GrammarRow * R)()
    for i, mode in enumerate(modes):
        L.dlk_grammar_row_init(C.byref(states[i]), L.dlk_grammar_mode_of(mode))
    seeds = rng.integers(1, 2**63, R, dtype=np.uint64)
    dev = torch.device("cuda:0")
    d_off = torch.from_numpy(off.view(np.int32)).to(dev)
    d_bytes = torch.from_numpy(data).to(dev)
    d_states = torch.frombuffer(bytearray(bytes(states)), dtype=torch.uint8).to(dev)
    d_rng = torch.from_numpy(seeds.view(np.int64).copy()).to(dev)
    W_ = (V + 31) // 32
    d_mask = torch.zeros((R, W_), dtype=torch.int32, device=dev)
    d_out = torch.zeros(R, dtype=torch.int32, device=dev)
    d_status = torch.zeros(1, dtype=torch.int32, device=dev)
    prm = _lib.SampleParams(T_, K_, P_, 0.0, 1.0, 0.0, 0.0, _lib.ORDER_REFERENCE, 1, 0, path)
    step_logits = [rng.normal(0, 2, (R, V)).astype(np.float32) for _ in range(steps)]
    for lg in step_logits:
        lg[:, :8] += 2.5                                        # the JSON pieces of random_vocab
    got = np.zeros((steps, R), np.int32)
    for s_ in range(steps):
        d_lg = torch.from_numpy(step_logits[s_]).to(dev)
        b = _lib.Batch(logits=d_lg.data_ptr(), ld=V, hist_off=None, hist_ids=None, mask=d_mask.data_ptr(), mask_ld=W_,
                       mask_row=None, rng=d_rng.data_ptr(), out_ids=d_out.data_ptr(), out_cand_ids=None,
                       out_cand_probs=None, out_cand_logprobs=None, status=d_status.data_ptr())
        rc = L.dlk_sample_grammar(C.byref(b), R, V, C.byref(prm), d_off.data_ptr(), d_bytes.data_ptr(),
                                  d_states.data_ptr(), eos, None)
        assert rc == 0
        got[s_] = d_out.cpu().numpy()
    end_states = d_rng.cpu().numpy().view(np.uint64)
    assert int(d_status.cpu().item()) == 0
    for i, mode in enumerate(modes):
        g = O.grammar(mode)
        st = int(seeds[i])
        for s_ in range(steps):
            masked, _ = O.grammar_mask(g, off, data, eos, step_logits[s_][i])
            o = O.sample_row(masked, st, T_, K_, P_, 0.0)
            st = o["state"]
            assert got[s_, i] == o["token"], (mode, s_, got[:, i], o["token"])
            if o["token"] != eos and 0 <= o["token"] < V:
                O.lib().orc_grammar_advance(C.byref(g), strs[o["token"]].split(b"\0")[0])
        assert int(end_states[i]) == st
