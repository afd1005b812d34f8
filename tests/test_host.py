"""CPU checks of libdiskllm_amd.so that need no GPU: it loads, exports exactly
what include/*.h declares, and its host-side code (seed, grammar modes, the
resumable validators behind accept_str / advance / is_finished) agrees with the
reference compiled from its sources."""
import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

from diskllm_amd import _lib
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = O.ref("strict")
needs_ref = pytest.mark.skipif(REF is None, reason="oracle/_ref not built (no reference tree here)")


def declared_functions():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \t\*]*?\b([a-z_][a-z0-9_]*)\s*\([^;{]*\)\s*;", text, flags=re.M):
            if not m.group(0).lstrip().startswith(("typedef", "return", "#")):
                names.add(m.group(1))
    return names


def test_library_loads_and_exports_every_declared_symbol():
    L = _lib.lib()
    decl = declared_functions()
    assert decl == set(_lib.EXPORTS), sorted(decl ^ set(_lib.EXPORTS))
    for name in decl:
        assert hasattr(L, name), name
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert exported == decl, sorted(exported ^ decl)


def test_seed_state():
    L = _lib.lib()
    assert L.dlk_seed_state(0) == 0xDEADBEEF12345678            # src/sampler.c:87
    assert L.dlk_seed_state(7) == 7


def test_csr_token_str():
    """dlk_csr_token_str: the entry as a NUL-terminated string, NULL outside
    [0, vocab) or without a scratch buffer, long entries cut at scratch_cap - 1."""
    L = _lib.lib()
    toks = [b"ab", b"", b"{\"x\":", b"0123456789"]
    off = np.zeros(len(toks) + 1, np.uint32)
    off[1:] = np.cumsum([len(x) for x in toks])
    data = np.frombuffer(b"".join(toks), np.uint8).copy()
    scratch = C.create_string_buffer(8)
    v = _lib.CsrVocab(off.ctypes.data, data.ctypes.data, len(toks), C.cast(scratch, C.c_void_p), 8)
    assert [L.dlk_csr_token_str(C.byref(v), i) for i in range(3)] == toks[:3]
    assert L.dlk_csr_token_str(C.byref(v), 3) == b"0123456"
    assert L.dlk_csr_token_str(C.byref(v), -1) is None and L.dlk_csr_token_str(C.byref(v), 4) is None
    v.scratch_cap = 0
    assert L.dlk_csr_token_str(C.byref(v), 0) is None


def test_grammar_modes():
    L = _lib.lib()
    assert L.dlk_grammar_mode_of(b'root ::= "{" "\\"bbox_2d\\":" ...') == _lib.GRAMMAR_RECEIPT
    assert L.dlk_grammar_mode_of(b"root ::= object | array") == _lib.GRAMMAR_JSON
    assert L.dlk_grammar_mode_of(b"value bbox_2d") == _lib.GRAMMAR_RECEIPT         # receipt first (:240)
    assert L.dlk_grammar_mode_of(b"root ::= [a-z]+") == _lib.GRAMMAR_NONE
    assert L.dlk_grammar_mode_of(None) == _lib.GRAMMAR_NONE


ALPHABET = list(b'{}[]":,\\ \t\n\r0123456789abdextnco_-') + [0x80, 0xC4, 0xA0, 0x0B, 0x0C]


def rand_piece(rng, maxlen=6):
    return bytes(int(b) for b in rng.choice(ALPHABET, int(rng.integers(1, maxlen + 1))))


def schema_pieces(rng):
    texts = [b' {"bbox_2d": [12, 3 ,450,7] , "text_content": "a \\"q\\" b"} ',
             b'{"bbox_2d" [1,2,3,4],"text_content":"x"}', b'{ "bbox_2d":[,,,],"text_content":  ""}\n',
             b'[{"k": "v}"}, [1, {"a": "\\\\"}]]', b'  {"a": [1, 2, {"b": "]"}], "c": "{"}']
    t = texts[int(rng.integers(0, len(texts)))]
    cuts = sorted(set(int(c) for c in rng.integers(1, len(t), 6)))
    ps = [t[a:b] for a, b in zip([0] + cuts, cuts + [len(t)])]
    if rng.random() < 0.4:
        ps[int(rng.integers(0, len(ps)))] = rand_piece(rng)
    return ps


@needs_ref
@pytest.mark.parametrize("text", [b"receipt bbox_2d", b"root ::= object | value", b"anything", None])
def test_dropin_grammar_host_calls_vs_reference(text):
    """accept_str / advance / is_finished / reset of the drop-in (host code over
    the resumable validators) against the reference's (src/core/grammar.c)."""
    L = _lib.lib()
    rng = np.random.default_rng(0 if text is None else len(text))
    for trial in range(400):
        if text is None:
            g, h = L.diskllm_grammar_init_json(), REF.diskllm_grammar_init_json()
        else:
            g, h = L.diskllm_grammar_init_from_str(text), REF.diskllm_grammar_init_from_str(text)
        try:
            for rnd in range(2):
                pieces = schema_pieces(rng) if trial % 2 else [rand_piece(rng) for _ in range(8)]
                for pc in pieces:
                    for probe in (pc, rand_piece(rng), b"}", b"]", b'"', b" ", b"", b"x" * 9000):
                        assert L.diskllm_grammar_accept_str(g, probe) == REF.diskllm_grammar_accept_str(h, probe), \
                            (text, pc, probe)
                    assert L.diskllm_grammar_is_finished(g) == REF.diskllm_grammar_is_finished(h)
                    L.diskllm_grammar_advance(g, pc)
                    REF.diskllm_grammar_advance(h, pc)
                L.diskllm_grammar_reset(g)
                REF.diskllm_grammar_reset(h)
        finally:
            L.diskllm_grammar_free(g)
            REF.diskllm_grammar_free(h)


@needs_ref
def test_dropin_grammar_buffer_limit():
    """Pieces that would overflow the 8191-byte buffer are refused by accept_str
    and dropped by advance (src/core/grammar.c:233, :251)."""
    L = _lib.lib()
    g, h = L.diskllm_grammar_init_from_str(b"object"), REF.diskllm_grammar_init_from_str(b"object")
    try:
        chunk = b"[" + b" " * 999
        for _ in range(12):
            for probe in (b" " * 190, b" " * 191, b" " * 192, b"]"):
                assert L.diskllm_grammar_accept_str(g, probe) == REF.diskllm_grammar_accept_str(h, probe)
            L.diskllm_grammar_advance(g, chunk)
            REF.diskllm_grammar_advance(h, chunk)
            assert L.diskllm_grammar_is_finished(g) == REF.diskllm_grammar_is_finished(h)
    finally:
        L.diskllm_grammar_free(g)
        REF.diskllm_grammar_free(h)


def test_grammar_from_file(tmp_path):
    L = _lib.lib()
    p = tmp_path / "receipt.gbnf"
    p.write_bytes(b'root ::= "{" ws "\\"bbox_2d\\":" ws "[" ws int "]" ws "}"\nint ::= [0-9]+\n')
    g = L.diskllm_grammar_init_from_file(str(p).encode())
    assert g
    assert L.diskllm_grammar_accept_str(g, b'{"bbox_2d":')
    assert not L.diskllm_grammar_accept_str(g, b"invalid")
    L.diskllm_grammar_free(g)
    assert not L.diskllm_grammar_init_from_file(str(tmp_path / "missing").encode())


def test_grammar_unit_kats_dropin():
    """tools/test_grammar_unit.c:17-24 on the drop-in."""
    L = _lib.lib()
    gbnf = (b'root ::= "{" ws "\\"bbox_2d\\":" ws "[" ws int "]" ws "}"\n'
            b'int ::= [0-9]+\nws ::= [ \\t\\n\\r]*\n')
    g = L.diskllm_grammar_init_from_str(gbnf)
    assert g
    assert L.diskllm_grammar_accept_str(g, b"{")
    L.diskllm_grammar_advance(g, b"{")
    assert L.diskllm_grammar_accept_str(g, b'"bbox_2d":')
    assert not L.diskllm_grammar_accept_str(g, b"invalid")
    L.diskllm_grammar_advance(g, b'"bbox_2d": [123] }')
    assert L.diskllm_grammar_is_finished(g)
    L.diskllm_grammar_free(g)


# --- vocabulary table from a GGUF file (dlk_vocab_csr_from_gguf) -------------------------------------------

def _gguf_str(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def _gguf_value(t: int, v) -> bytes:
    """One GGUF value of type t (the type ids and layouts of the GGUF format)."""
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
    if t in fmt:
        return struct.pack(fmt[t], v)
    if t == 8:
        return _gguf_str(v)
    et, items = v
    return struct.pack("<IQ", et, len(items)) + b"".join(_gguf_value(et, x) for x in items)


def _write_gguf(path, kvs, magic=b"GGUF"):
    out = magic + struct.pack("<IQQ", 3, 0, len(kvs))
    for key, t, v in kvs:
        out += _gguf_str(key) + struct.pack("<I", t) + _gguf_value(t, v)
    with open(path, "wb") as f:
        f.write(out)
    return out


GGUF_TOKENS = [b"!", b"\"", b"{", b"}", "Ġthe".encode(), b"<0x0A>", b"", b"<|im_end|>", b"a\x00b",
               "éè".encode(), b"[", b"]", b"12", b"\\", b" " * 300]
# Every value type before the tokens, including strings, scalar arrays, string arrays and an array of
# arrays, and a key that shares the tokens key's length.
GGUF_PREFIX = [
    (b"general.architecture", 8, b"qwen2"), (b"general.file_type", 4, 7), (b"a.u8", 0, 200), (b"a.i8", 1, -3),
    (b"a.u16", 2, 65000), (b"a.i16", 3, -2), (b"a.i32", 5, -9), (b"a.f32", 6, 0.5), (b"a.bool", 7, True),
    (b"a.u64", 10, 1 << 40), (b"a.i64", 11, -(1 << 40)), (b"a.f64", 12, 0.25),
    (b"tokenizer.ggml.model", 8, b"gpt2"), (b"tokenizer.ggml.tokenz", 8, b"not the tokens"),
    (b"tokenizer.ggml.scores", 9, (6, [0.5] * 7)), (b"tokenizer.ggml.token_type", 9, (5, [1, 2, 3])),
    (b"a.nested", 9, (9, [(8, [b"x", b"yz"]), (4, [1, 2])])),
]
GGUF_SUFFIX = [(b"tokenizer.ggml.merges", 9, (8, ["Ġ t".encode(), b"h e"])), (b"tokenizer.ggml.eos_token_id", 4, 7)]


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


def _entries(off, data):
    return [bytes(data[off[t]:off[t + 1]]) for t in range(len(off) - 1)]


@pytest.mark.parametrize("vocab", [0, len(GGUF_TOKENS), 5, len(GGUF_TOKENS) + 9])
def test_vocab_csr_from_gguf(tmp_path, vocab):
    path = str(tmp_path / "v.gguf")
    _write_gguf(path, GGUF_PREFIX + [(b"tokenizer.ggml.tokens", 9, (8, GGUF_TOKENS))] + GGUF_SUFFIX)
    off, data, n = _lib.vocab_csr_from_gguf(path, vocab)
    ids = vocab or len(GGUF_TOKENS)
    assert n == len(GGUF_TOKENS) and len(off) == ids + 1 and off[0] == 0
    want = (GGUF_TOKENS + [b""] * ids)[:ids]
    assert _entries(off, data) == want
    T = _ref_tokenizer()
    if T is not None:                                   # the reference's own load of the same file
        tok = T.tokenizer_init(path.encode())
        assert tok
        try:
            for t in range(ids):
                p = T.tokenizer_decode_raw(tok, t)
                got = _entries(off, data)[t].split(b"\x00")[0]
                assert (C.string_at(p) if p else b"") == got, t
                assert (p is None) == (t >= len(GGUF_TOKENS)), t
        finally:
            T.tokenizer_free(tok)


def test_vocab_csr_from_gguf_errors(tmp_path):
    L = _lib.lib()
    nt, nb = C.c_int32(-1), C.c_int64(-1)
    full = _write_gguf(str(tmp_path / "ok.gguf"), GGUF_PREFIX + [(b"tokenizer.ggml.tokens", 9, (8, GGUF_TOKENS))])
    call = lambda p, *a: L.dlk_vocab_csr_from_gguf(str(p).encode(), *a, C.byref(nt), C.byref(nb))
    assert call(tmp_path / "missing.gguf", 0, None, None, 0) == _lib.DLK_ERR_FORMAT
    _write_gguf(str(tmp_path / "magic.gguf"), GGUF_PREFIX, magic=b"GGUG")
    assert call(tmp_path / "magic.gguf", 0, None, None, 0) == _lib.DLK_ERR_FORMAT
    # Cut anywhere inside the metadata or the strings: a format error on both calls.
    for cut in (3, 20, 100, len(full) // 2, len(full) - 301, len(full) - 1):
        (tmp_path / "cut.gguf").write_bytes(full[:cut])
        assert call(tmp_path / "cut.gguf", 0, None, None, 0) == _lib.DLK_ERR_FORMAT, cut
        off, data = np.zeros(len(GGUF_TOKENS) + 1, np.uint32), np.zeros(4096, np.uint8)
        assert call(tmp_path / "cut.gguf", len(GGUF_TOKENS), off.ctypes.data, data.ctypes.data,
                    data.size) == _lib.DLK_ERR_FORMAT, cut
    # Cut after the strings the table covers: only those are read.
    (tmp_path / "cut.gguf").write_bytes(full[:len(full) - 308])
    assert call(tmp_path / "cut.gguf", 5, None, None, 0) == _lib.DLK_OK and nt.value == len(GGUF_TOKENS)
    # The tokens array holding something other than strings.
    _write_gguf(str(tmp_path / "ints.gguf"), [(b"tokenizer.ggml.tokens", 9, (4, [1, 2, 3]))])
    assert call(tmp_path / "ints.gguf", 0, None, None, 0) == _lib.DLK_ERR_FORMAT
    # bytes_cap one short of what the sizing call reported.
    assert call(tmp_path / "ok.gguf", 0, None, None, 0) == _lib.DLK_OK
    need = nb.value
    off, data = np.zeros(len(GGUF_TOKENS) + 1, np.uint32), np.zeros(need, np.uint8)
    assert call(tmp_path / "ok.gguf", 0, off.ctypes.data, data.ctypes.data, need - 1) == _lib.DLK_ERR_INVALID
    assert call(tmp_path / "ok.gguf", 0, off.ctypes.data, data.ctypes.data, need) == _lib.DLK_OK
    # No tokens array: an all-empty table, as the reference's vocab_size 0 decodes nothing.
    _write_gguf(str(tmp_path / "none.gguf"), GGUF_PREFIX)
    off, data, n = _lib.vocab_csr_from_gguf(str(tmp_path / "none.gguf"), 6)
    assert n == 0 and list(off) == [0] * 7 and data.size == 0


def test_softcap_argument_checks():
    """dlk_softcap's host-side checks (no device work is started by any of these):
    bad pointers and shapes are DLK_ERR_INVALID, a grid beyond the row limit is
    DLK_ERR_UNSUPPORTED, and cap <= 0 or NaN is the reference's no-op."""
    L = _lib.lib()
    fake = C.c_void_p(16)                     # never dereferenced: every call below returns first
    assert L.dlk_softcap(None, 8, 1, 8, 30.0, None) == _lib.DLK_ERR_INVALID
    assert L.dlk_softcap(fake, 7, 1, 8, 30.0, None) == _lib.DLK_ERR_INVALID          # ld < vocab
    assert L.dlk_softcap(fake, 8, -1, 8, 30.0, None) == _lib.DLK_ERR_INVALID
    assert L.dlk_softcap(fake, 8, 1, -1, 30.0, None) == _lib.DLK_ERR_INVALID
    assert L.dlk_softcap(fake, 8, 70000, 8, 30.0, None) == _lib.DLK_ERR_UNSUPPORTED
    for cap in (0.0, -3.0, float("nan")):
        assert L.dlk_softcap(fake, 8, 4, 8, cap, None) == _lib.DLK_OK
    assert L.dlk_softcap(fake, 8, 0, 8, 30.0, None) == _lib.DLK_OK
