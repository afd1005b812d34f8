"""CPU checks of libdiskllm_amd.so that need no GPU: it loads, exports exactly
what include/*.h declares, and its host-side code (seed, grammar modes, the
resumable validators behind accept_str / advance / is_finished) agrees with the
reference compiled from its sources."""
import ctypes as C
import os
import re

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
