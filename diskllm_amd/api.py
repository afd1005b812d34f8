"""Python host side of the batched sampling path.

Mirrors the C ABI of include/diskllm_amd.h one-to-one; torch tensors are only
device-memory and stream plumbing.  Every call goes through libdiskllm_amd.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib
from .workloads import Workload


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _dev(a: np.ndarray, device) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(a).to(device)


def stream_handle(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


@dataclass
class DeviceBatch:
    """A workload's inputs resident in HBM plus output buffers."""
    w: Workload
    logits: torch.Tensor
    seeds: torch.Tensor            # int64 view of the per-row uint64 seeds (never mutated)
    rng: torch.Tensor              # int64 view of the per-row xorshift states (mutated)
    hist_off: Optional[torch.Tensor]
    hist_ids: Optional[torch.Tensor]
    mask: Optional[torch.Tensor]
    mask_row: Optional[torch.Tensor]
    out_ids: torch.Tensor
    cand_ids: Optional[torch.Tensor]
    cand_probs: Optional[torch.Tensor]
    cand_logprobs: Optional[torch.Tensor]
    status: torch.Tensor

    def reset_rng(self) -> None:
        self.rng.copy_(self.seeds)


def dfa_masks(offsets, data, trans, states, vocab: int, eos_id: int = -1, accept: int = 0,
              device="cuda", stream: Optional[int] = None) -> torch.Tensor:
    """Packed allow-masks [len(states), ceil(V/32)] (int32 view of uint32 words)."""
    W = (vocab + 31) // 32
    t_off = offsets if isinstance(offsets, torch.Tensor) else _dev(np.asarray(offsets, np.uint32), device)
    t_dat = data if isinstance(data, torch.Tensor) else _dev(np.asarray(data, np.uint8), device)
    tr = np.ascontiguousarray(trans, np.uint8)
    t_tr = _dev(tr, device)
    t_st = states if isinstance(states, torch.Tensor) else _dev(np.asarray(states, np.int32), device)
    out = torch.empty((t_st.numel(), W), dtype=torch.int32, device=device)
    rc = _lib.lib().dlk_dfa_mask(t_off.data_ptr(), t_dat.data_ptr(), vocab, t_tr.data_ptr(), tr.shape[0],
                                 t_st.data_ptr(), t_st.numel(), eos_id, accept & 0xFFFFFFFFFFFFFFFF, out.data_ptr(),
                                 W, stream if stream is not None else stream_handle())
    _lib.check(rc, "dlk_dfa_mask")
    return out


def to_device(w: Workload, device="cuda", rows: Optional[list] = None) -> DeviceBatch:
    sel = list(range(w.rows)) if rows is None else list(rows)
    lg = _dev(np.ascontiguousarray(w.logits[sel]), device)
    seeds = _dev(np.ascontiguousarray(w.seeds[sel]), device)
    hoff = hids = None
    if w.hist_ids is not None:
        lists = [w.hist_ids[w.hist_off[r]:w.hist_off[r + 1]] for r in sel]
        off = np.zeros(len(sel) + 1, np.int32)
        off[1:] = np.cumsum([len(x) for x in lists])
        ids = np.concatenate(lists).astype(np.int32) if lists else np.zeros(0, np.int32)
        hoff, hids = _dev(off, device), _dev(ids if ids.size else np.zeros(1, np.int32), device)
    mask = mask_row = None
    if w.mask is not None:
        mask = _dev(np.ascontiguousarray(w.mask[sel]), device)
    elif w.dfa is not None and w.dfa_states is not None:
        n_states = w.dfa.trans.shape[0]
        mask = dfa_masks(w.dfa.offsets, w.dfa.data, w.dfa.trans, np.arange(n_states, dtype=np.int32), w.vocab,
                         w.dfa.eos_id, w.dfa.accept, device)
        mask_row = _dev(np.asarray(w.dfa_states[sel], np.int32), device)
    n = len(sel)
    no = w.n_out
    return DeviceBatch(
        w=w, logits=lg, seeds=seeds, rng=seeds.clone(), hist_off=hoff, hist_ids=hids, mask=mask, mask_row=mask_row,
        out_ids=torch.full((n,), -7, dtype=torch.int32, device=device),
        cand_ids=torch.zeros((n, no), dtype=torch.int32, device=device) if no else None,
        cand_probs=torch.zeros((n, no), dtype=torch.float32, device=device) if no else None,
        cand_logprobs=torch.zeros((n, no), dtype=torch.float32, device=device) if no else None,
        status=torch.zeros(1, dtype=torch.int32, device=device))


def params_of(w: Workload, max_history: int = 0, path: int = 0) -> _lib.SampleParams:
    mh = max_history
    if mh <= 0 and w.hist_off is not None and len(w.hist_off) > 1:
        mh = int(np.max(np.diff(w.hist_off)))
    return _lib.SampleParams(w.temperature, w.top_k, w.top_p, w.min_p, w.repeat_penalty, w.frequency_penalty,
                             w.presence_penalty, w.order, max(mh, 1), w.n_out, path, w.softcap)


def batch_struct(db: DeviceBatch) -> _lib.Batch:
    w = db.w
    return _lib.Batch(
        logits=db.logits.data_ptr(), ld=db.logits.shape[1], hist_off=_ptr(db.hist_off), hist_ids=_ptr(db.hist_ids),
        mask=_ptr(db.mask), mask_ld=(db.mask.shape[1] if db.mask is not None else 0), mask_row=_ptr(db.mask_row),
        rng=db.rng.data_ptr(), out_ids=db.out_ids.data_ptr(), out_cand_ids=_ptr(db.cand_ids),
        out_cand_probs=_ptr(db.cand_probs), out_cand_logprobs=_ptr(db.cand_logprobs), status=db.status.data_ptr())


def sample(db: DeviceBatch, params: Optional[_lib.SampleParams] = None, stream: Optional[int] = None) -> None:
    """One dlk_sample call over the batch (asynchronous on the stream)."""
    w = db.w
    p = params if params is not None else params_of(w)
    b = batch_struct(db)
    rc = _lib.lib().dlk_sample(C.byref(b), db.logits.shape[0], w.vocab, C.byref(p),
                               stream if stream is not None else stream_handle())
    _lib.check(rc, "dlk_sample")


def sampler(db: DeviceBatch, params: Optional[_lib.SampleParams] = None, stream: Optional[int] = None):
    """A callable that makes the dlk_sample call of sample() with its argument
    structures built once: a loop of calls then costs the C call alone (timing
    loops; the batch's buffers must stay where they are)."""
    w = db.w
    p = params if params is not None else params_of(w)
    b = batch_struct(db)
    f = _lib.lib().dlk_sample
    rows, vocab = db.logits.shape[0], w.vocab
    sh = stream if stream is not None else stream_handle()
    bp, pp = C.byref(b), C.byref(p)

    def run() -> None:
        rc = f(bp, rows, vocab, pp, sh)
        if rc != 0:
            _lib.check(rc, "dlk_sample")
    run.keep = (b, p)
    return run


def results(db: DeviceBatch) -> dict:
    torch.cuda.synchronize()
    out = dict(ids=db.out_ids.cpu().numpy(), states=db.rng.cpu().numpy().view(np.uint64),
               status=int(db.status.cpu().item()))
    if db.cand_ids is not None:
        out.update(cand_ids=db.cand_ids.cpu().numpy(), cand_probs=db.cand_probs.cpu().numpy(),
                   cand_logprobs=db.cand_logprobs.cpu().numpy())
    return out
