"""dlk_sample_noalloc (the entry point whose workspace is a fixed per-device
scratch array) against dlk_sample: the same ids, rng states and candidate
outputs, bit for bit, on two calls in a row with the second one smaller, for
each kernel family; and the sizes it refuses."""
import ctypes as C

import numpy as np
import pytest

from diskllm_amd import _lib
from diskllm_amd import workloads as W

pytestmark = pytest.mark.gpu


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _call(fn_name, db, prm):
    from diskllm_amd import api
    b = api.batch_struct(db)
    rc = getattr(_lib.lib(), fn_name)(C.byref(b), db.logits.shape[0], db.w.vocab, C.byref(prm), api.stream_handle())
    return rc


def _run_pair(w, path=0):
    """(noalloc results, dlk_sample results) from identical inputs."""
    from diskllm_amd import api
    a, b = api.to_device(w), api.to_device(w)
    prm = api.params_of(w, path=path)
    assert _call("dlk_sample_noalloc", a, prm) == _lib.DLK_OK
    assert _call("dlk_sample", b, prm) == _lib.DLK_OK
    return api.results(a), api.results(b)


def _same(ra, rb):
    np.testing.assert_array_equal(ra["ids"], rb["ids"])
    np.testing.assert_array_equal(ra["states"], rb["states"])
    assert ra["status"] == 0 and rb["status"] == 0
    for key in ("cand_ids", "cand_probs", "cand_logprobs"):
        if key in rb:
            np.testing.assert_array_equal(ra[key].view(np.uint32), rb[key].view(np.uint32))


@pytest.mark.parametrize("make,big,small", [(W.c2, 64, 16), (W.c3, 32, 8)], ids=["full", "topk"])
def test_noalloc_matches_dlk_sample(cuda, make, big, small):
    """Fused full-vocabulary (C2) and top-k (C3) kernels: a call over `big`
    rows, then one over fewer rows, each equal to dlk_sample's."""
    for rows in (big, small):
        w = make(rows=rows)
        _announce(f"noalloc {w.name} rows={rows}")
        ra, rb = _run_pair(w)
        _same(ra, rb)


def test_noalloc_row_kernel_and_large_k(cuda):
    """The one-workgroup-per-row kernel (no workspace) and the global-memory
    top-k (workspace inside the scratch array): equal to dlk_sample's."""
    w = W.c3(rows=8)
    _announce("noalloc row kernel C3 rows=8")
    _same(*_run_pair(w, path=_lib.PATH_ROW))
    w = W.c3(rows=6)
    w.top_k = 6000
    w.n_out = 0
    _announce("noalloc top-k 6000 rows=6 then rows=3")
    _same(*_run_pair(w))
    w = W.c3(rows=3)
    w.top_k = 6000
    w.n_out = 0
    _same(*_run_pair(w))


def test_noalloc_softcap_matches_dlk_sample(cuda):
    """The soft-cap inside the sampling kernels (no second buffer): C5 rows with
    cap 30, two calls of decreasing size, equal to dlk_sample's."""
    from diskllm_amd import api
    for rows in (24, 8):
        w = W.c5(rows=rows)
        _announce(f"noalloc softcap 30 C5 rows={rows}")
        a, b = api.to_device(w), api.to_device(w)
        prm = api.params_of(w)
        prm.softcap = 30.0
        assert _call("dlk_sample_noalloc", a, prm) == _lib.DLK_OK
        assert _call("dlk_sample", b, prm) == _lib.DLK_OK
        _same(api.results(a), api.results(b))


def test_noalloc_refuses_what_needs_more(cuda):
    """Calls that would need a second buffer are refused with
    DLK_ERR_UNSUPPORTED: histories above 1024 ids (their penalties run on a
    scratch copy of the rows)."""
    from diskllm_amd import api
    w = W.c2(rows=2)
    db = api.to_device(w)
    prm = api.params_of(w, max_history=5000)
    _announce("noalloc refuses max_history 5000")
    assert _call("dlk_sample_noalloc", db, prm) == _lib.DLK_ERR_UNSUPPORTED


@pytest.mark.parametrize("make,rows", [(W.c2, 16), (W.c3, 8)], ids=["full", "topk"])
def test_noalloc_allocates_nothing_and_captures(cuda, make, rows):
    """Device free memory is unchanged across a dlk_sample_noalloc call, and the
    call captured into a HIP graph (torch.cuda.graph; the counters are cleared by
    a fill kernel, not a memset node) gives, on each of four replays with eager
    work and synchronisation between them, the ids and rng states dlk_sample
    gives for the same step.  The first call of a shape (outside the capture)
    fills the host-side occupancy tables."""
    import torch
    from diskllm_amd import api
    w = make(rows=rows)
    a, b = api.to_device(w), api.to_device(w)
    prm = api.params_of(w)
    _announce(f"noalloc {w.name} rows={rows}: warm-up, memory")
    assert _call("dlk_sample_noalloc", a, prm) == _lib.DLK_OK       # warm-up (host tables)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    assert _call("dlk_sample_noalloc", a, prm) == _lib.DLK_OK
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    a.reset_rng()
    g = torch.cuda.CUDAGraph()
    _announce(f"noalloc {w.name} rows={rows}: capture")
    with torch.cuda.graph(g):
        rc = _call("dlk_sample_noalloc", a, prm)
    assert rc == _lib.DLK_OK
    for rep in range(4):
        _announce(f"noalloc {w.name} rows={rows}: replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        ra = api.results(a)
        assert _call("dlk_sample", b, prm) == _lib.DLK_OK
        rb = api.results(b)
        _same(ra, rb)
