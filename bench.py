#!/usr/bin/env python3
"""Benchmark of the MI355X sampling path on its headline configuration.

Workload C2 (the headline configuration): fp32 logits [64, 151936] (Qwen vocab),
N(0,2^2) + Zipf(1.1) rank bias, repetition 1.15 / frequency 0.3 / presence 0.5
over a 256-id Zipf history, temperature 1.0, top-p 0.9, no top-k -- one
dlk_sample() call over the batch is one step.  Inputs are resident in HBM before
the timed region; the rng states advance every step exactly as the reference's
would.

Prints one JSON line: rows/s, ms per step, the dominant kernel's roofline
(algorithmic HBM bytes per launch / its average duration from HIP events on the
launch stream) and the reference src/sampler.c timed on this host's cores.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0        # MI355X HBM3E
ROWS, VOCAB, HIST = 64, 151936, 256
# Algorithmic bytes per row: logits + history ids + rng state + token id.
BYTES_PER_ROW = VOCAB * 4 + HIST * 4 + 8 + 4      # 608,780 B
METRIC = "sampled rows/sec + achieved HBM GB/s (% of peak), batch 64, vocab 151936"


def fused_kernel_name(rows: int, vocab: int) -> str:
    """Template instance of the fused full-vocabulary kernel dlk_sample launches for
    this shape (the same selection as launch_full in diskllm_amd/csrc/hip/capi.hip:
    G = ceil(512 / rows) workgroups of 512 threads per row, elements per thread
    rounded up to a bucket; the bench's 256-id histories take the instance that
    loads one history id per thread)."""
    G = min(16, max(1, (512 + rows - 1) // rows))
    ept = (vocab + G * 512 - 1) // (G * 512)
    ept = next(e for e in (16, 24, 32, 40, 48) if ept <= e or e == 48)
    return f"dlk::full_kernel<{ept}, false, false, 1>"


# The dominant kernel of each workload and its committed traffic summary.
DOMINANT = {"C1": ("dlk::topk_kernel<false, false>", None),
            "C3": ("dlk::topk_kernel<false, false>", "topk_kernel_c3"),
            "C4": ("dlk::dfa_walk_kernel<16>", None),
            "C5": ("dlk::topk_kernel<false, false>", "topk_kernel_c5"),
            "C5CAP": ("dlk::topk_kernel<true, false>", None),
            "CAP": ("dlk::softcap_vec_kernel", "softcap_vec_kernel_cap")}


def profiled_traffic(kernel: str, tag: str = "full_kernel_c2"):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary
    profiles/<tag>_hbm_traffic.txt (FETCH_SIZE and WRITE_SIZE passes scaled by a
    copy of known size), or None when the summary is absent, was taken on
    another kernel, or on other library sources than the ones built here (its
    "library source stamp:" line against diskllm_amd._lib.source_stamp())."""
    if tag is None:
        return None
    path = os.path.join(ROOT, "profiles", f"{tag}_hbm_traffic.txt")
    try:
        text = open(path).read()
    except OSError:
        return None
    short = kernel.replace("dlk::", "")
    if short not in text:
        return None
    from diskllm_amd import _lib
    stamp = _lib.source_stamp()
    if not any(ln.startswith("library source stamp:") and ln.split(":", 1)[1].strip() == stamp
               for ln in text.splitlines()):
        return None
    for ln in text.splitlines():
        if ln.startswith("scaled traffic per launch:"):
            return int(round(float(ln.split("=")[-1].split()[0]) * 1e6))
    return None


def host_threads() -> int:
    """Host threads the CPU baseline may use: the CPUs this process may run on
    (the GPU box gives one GPU 16 of them)."""
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_baseline(w, runs: int, threads_all: int, kind: str = "strict") -> dict:
    """The reference src/sampler.c (strict ISO C build in oracle/_ref, or with
    kind "fast" the reference Makefile's -O3 -ffast-math build) on the host:
    penalties + sampler_sample for every row, rows split over pthreads."""
    import numpy as np
    from oracle import oracle as O
    L = O.ref(kind)
    if L is None:
        return None
    cfg = O.SamplerConfig(w.temperature, w.top_k, w.top_p, w.min_p, 1)
    out = {}
    for th in (sorted({1, threads_all}) if kind == "strict" else [threads_all]):
        ms = np.zeros(runs, np.float64)
        ids = np.zeros(w.rows, np.int32)
        rc = L.refh_time_batch(np.ascontiguousarray(w.logits), w.rows, w.vocab, w.hist_off.ctypes.data,
                               w.hist_ids.ctypes.data, None, 0, w.order, w.repeat_penalty, w.frequency_penalty,
                               w.presence_penalty, C.byref(cfg), np.ascontiguousarray(w.seeds), th, runs, ms, ids)
        assert rc == 0
        med = float(np.median(ms))
        out[th] = dict(value=w.rows / (med / 1e3), ms=med, ids=ids)
    return out


# Algorithmic HBM bytes of the other workloads of the scope table, per step
# (logits + per-row inputs + outputs; shared tables once per step).
def other_bytes(w) -> int:
    import numpy as np
    V, rows = w.vocab, w.rows
    W = (V + 31) // 32
    if getattr(w, "epilogue", False):
        return rows * V * 8                              # each logit read and written once
    if w.name == "C4":
        csr = (V + 1) * 4 + int(w.dfa.data.size) + int(w.dfa.trans.size)
        return csr + rows * (4 + W * 4)                 # CSR + table once, a state in and a mask row out per row
    per = V * 4 + 8 + 4                                 # logits, rng state in/out, token id
    if w.hist_off is not None:
        per += int(np.max(np.diff(w.hist_off))) * 4     # history ids
    if w.mask is not None or w.dfa is not None:
        per += W * 4                                    # the row's mask words
    per += w.n_out * 12                                 # candidate ids, probs, log-probs
    return rows * per


def run_other(name: str, args) -> int:
    """One JSON line for workload C1, C3, C4, C5, C5CAP or CAP (parity-test
    configurations; the headline line is C2): the step is one dlk_sample call
    (C5/C5CAP: the DFA mask pass, then dlk_sample; C4: one dlk_dfa_mask call for
    its 16 rows; CAP: the soft-cap epilogue alone), inputs resident in HBM, timed
    with HIP events on the launch stream."""
    import numpy as np
    import torch
    from diskllm_amd import _lib, api, workloads
    from oracle import oracle as O
    dev = torch.device("cuda:0")
    w = workloads.CONFIGS[name]()
    gpu_ids = None
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    if name == "CAP":
        from diskllm_amd import _lib
        w.epilogue = True
        cap = workloads.CAP_C5CAP
        lg = api._dev(np.ascontiguousarray(w.logits), dev)

        def step(ev=None):
            if ev: ev[0].record(stream)
            _lib.check(_lib.lib().dlk_softcap(lg.data_ptr(), w.vocab, w.rows, w.vocab, cap, sh), "dlk_softcap")
            if ev: ev[1].record(stream)
        step()
        torch.cuda.synchronize()
        got = lg.cpu().numpy()
        check = list(range(min(w.rows, 32)))
        want = np.ascontiguousarray(w.logits[check])
        O.lib().orc_softcap(want.reshape(-1), want.reshape(-1), want.size, np.float32(cap))
        n_ok = sum(int(np.array_equal(got[r].view(np.uint32), want[r].view(np.uint32))) for r in check)
        parity = f"{n_ok}/{len(check)} capped rows bit-identical to the oracle (rows 0..{len(check) - 1})"
        # the timed steps re-cap the capped rows in place: the same work per element
    elif name == "C4":
        d = w.dfa
        t_off = api._dev(np.asarray(d.offsets, np.uint32), dev)
        t_dat = api._dev(np.asarray(d.data, np.uint8), dev)
        t_st = api._dev(np.asarray(w.dfa_states, np.int32), dev)
        t_tr = api._dev(np.ascontiguousarray(d.trans, np.uint8), dev)
        W = (w.vocab + 31) // 32
        out = torch.empty((w.rows, W), dtype=torch.int32, device=dev)
        from diskllm_amd import _lib

        def step(ev=None):
            if ev: ev[0].record(stream)
            rc = _lib.lib().dlk_dfa_mask(t_off.data_ptr(), t_dat.data_ptr(), w.vocab, t_tr.data_ptr(), d.trans.shape[0],
                                         t_st.data_ptr(), w.rows, d.eos_id, d.accept & 0xFFFFFFFFFFFFFFFF,
                                         out.data_ptr(), W, sh)
            _lib.check(rc, "dlk_dfa_mask")
            if ev: ev[1].record(stream)
        step()
        torch.cuda.synchronize()
        got = out.cpu().numpy().view(np.uint32)
        n_ok = sum(int(np.array_equal(got[r], O.dfa_mask(d, int(w.dfa_states[r]), w.vocab))) for r in range(w.rows))
        parity = f"{n_ok}/{w.rows} mask rows bit-identical to the oracle"
    else:
        db = api.to_device(w, device=dev)
        params = api.params_of(w)
        if w.dfa is not None:
            # C5: the step includes the DFA pass, one mask row per DFA state (the rows
            # then pick theirs through mask_row), rebuilt into db.mask every step
            from diskllm_amd import _lib
            d = w.dfa
            t_off = api._dev(np.asarray(d.offsets, np.uint32), dev)
            t_dat = api._dev(np.asarray(d.data, np.uint8), dev)
            t_tr = api._dev(np.ascontiguousarray(d.trans, np.uint8), dev)
            n_st = d.trans.shape[0]
            t_all = api._dev(np.arange(n_st, dtype=np.int32), dev)
            W = db.mask.shape[1]
            run = api.sampler(db, params, sh)
            dfa_args = (t_off.data_ptr(), t_dat.data_ptr(), w.vocab, t_tr.data_ptr(), n_st, t_all.data_ptr(), n_st,
                        d.eos_id, d.accept & 0xFFFFFFFFFFFFFFFF, db.mask.data_ptr(), W, sh)
            dfa = _lib.lib().dlk_dfa_mask

            def step(ev=None):
                _lib.check(dfa(*dfa_args), "dlk_dfa_mask")
                if ev: ev[0].record(stream)
                run()
                if ev: ev[1].record(stream)
        else:
            run = api.sampler(db, params, sh)

            def step(ev=None):
                if ev: ev[0].record(stream)
                run()
                if ev: ev[1].record(stream)
        step()
        res = api.results(db)
        gpu_ids = res["ids"]
        check = list(range(min(w.rows, 32)))
        orc = O.run_workload(w, check)
        n_ok = int(np.sum(res["ids"][check] == orc["ids"]))
        parity = f"{n_ok}/{len(check)} token ids bit-identical to the oracle (rows 0..{len(check) - 1})"
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # HIP events on the launch stream: a step of one kernel (C1, C3, C4, CAP) is
    # timed by one pair around the whole loop (a pair per step would add its own
    # few microseconds to steps of this length); C5 and C5CAP, whose step also
    # runs the DFA pass, by a pair around the sampling call of each step
    single = w.dfa is None or name in ("C4", "CAP")
    if single:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for k in range(args.steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ms_dev = e0.elapsed_time(e1) / args.steps
    else:
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        t0 = time.perf_counter()
        for k in range(args.steps):
            step(evs[k])
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ms_dev = sum(a.elapsed_time(b) for a, b in evs) / args.steps
    ms_step = (t1 - t0) * 1e3 / args.steps
    nbytes = other_bytes(w)
    achieved = nbytes / (ms_dev * 1e-3) / 1e9
    kname, ktag = DOMINANT[name]
    line = {
        "metric": f"{name}: rows/sec + achieved HBM GB/s (% of peak), batch {w.rows}, vocab {w.vocab}",
        "value": round(w.rows / (ms_step * 1e-3), 1), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u8" if name == "C4" else "f32", "data": "synthetic",
        "config": {"workload": f"{name}: " + " ".join(workloads.CONFIGS[name].__doc__.split()), "rows": w.rows,
                   "vocab": w.vocab,
                   "parallelism": "none (1 GPU)"},
        "parity": parity,
        "library_source_stamp": _lib.source_stamp(),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": profiled_traffic(kname, ktag),
                     "bytes_per_launch": nbytes, "ms_per_launch": round(ms_dev, 5), "kernel": kname},
        "cpu_baseline": None,
    }
    if w.dfa is not None and name not in ("C4", "CAP"):
        line["config"]["step"] = ("dlk_dfa_mask over every DFA state (the mask table, rebuilt inside each timed "
                                  "step), then one dlk_sample call whose rows pick their state's mask row"
                                  + (f", with softcap {w.softcap:g} applied inside the sampling kernels"
                                     if w.softcap > 0.0 else ""))
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_other(w, args.cpu_runs, gpu_ids)
    print(json.dumps(line), flush=True)
    return 0


def cpu_other(w, runs: int, gpu_ids=None) -> dict:
    """CPU time of the same step: C1/C3 the reference src/sampler.c (strict
    build, masks applied as -inf first); C4 the oracle's byte-DFA walk (the DFA
    mask has no counterpart in the reference); C5 both, on a 32-row sample;
    C5CAP the reference's soft-cap loop (host libm tanhf, one thread) in front of
    C5's."""
    import numpy as np
    from oracle import oracle as O
    nthreads = host_threads()
    if getattr(w, "epilogue", False):
        rows = min(w.rows, 32)
        x = np.ascontiguousarray(w.logits[:rows]).reshape(-1)
        y = np.empty_like(x)
        ts = []
        for _ in range(max(1, runs // 4)):
            t0 = time.perf_counter()
            O.lib().orc_softcap(x, y, x.size, np.float32(30.0))
            ts.append(time.perf_counter() - t0)
        sec = float(np.median(ts))
        return {"value": round(rows / sec, 1), "unit": "rows/s", "cores": 1, "kind": "port",
                "sample": f"rows 0..{rows - 1}, the reference's loop cap * tanhf(x / cap) with the host libm "
                          f"(oracle/oracle.c orc_softcap; one thread, as in src/core/context.c:873-876), "
                          f"median of {len(ts)} passes"}
    if w.name == "C4":
        t0 = time.perf_counter()
        for r in range(w.rows):
            O.dfa_mask(w.dfa, int(w.dfa_states[r]), w.vocab)
        dt = time.perf_counter() - t0
        return {"value": round(w.rows / dt, 1), "unit": "rows/s", "cores": 1, "kind": "port",
                "sample": f"all {w.rows} rows, oracle/oracle.c orc_dfa_mask, one pass"}
    L = O.ref("strict")
    if L is None:
        return None
    rows = list(range(min(w.rows, 32)))
    lg = np.ascontiguousarray(w.logits[rows])
    cap_s = 0.0
    if w.softcap > 0.0:
        x = lg.reshape(-1)
        t0 = time.perf_counter()
        O.lib().orc_softcap(x, x, x.size, np.float32(w.softcap))
        cap_s = time.perf_counter() - t0
    mask = None
    mw = 0
    dfa_s = 0.0
    if w.mask is not None:
        mask = np.ascontiguousarray(w.mask[rows])
    elif w.dfa is not None:
        t0 = time.perf_counter()
        tab = {}
        for r in rows:
            st = int(w.dfa_states[r])
            if st not in tab:
                tab[st] = O.dfa_mask(w.dfa, st, w.vocab)
        dfa_s = time.perf_counter() - t0
        mask = np.ascontiguousarray(np.stack([tab[int(w.dfa_states[r])] for r in rows]))
    if mask is not None:
        mw = mask.shape[1]
    hoff = hids = None
    if w.hist_off is not None:
        lists = [w.hist_ids[w.hist_off[r]:w.hist_off[r + 1]] for r in rows]
        hoff = np.zeros(len(rows) + 1, np.int32)
        hoff[1:] = np.cumsum([len(x) for x in lists])
        hids = np.concatenate(lists).astype(np.int32)
    cfg = O.SamplerConfig(w.temperature, w.top_k, w.top_p, w.min_p, 1)
    th = min(nthreads, len(rows))
    ms = np.zeros(runs, np.float64)
    ids = np.zeros(len(rows), np.int32)
    rc = L.refh_time_batch(lg, len(rows), w.vocab, hoff.ctypes.data if hoff is not None else None,
                           hids.ctypes.data if hids is not None else None,
                           mask.ctypes.data if mask is not None else None, mw, w.order, w.repeat_penalty,
                           w.frequency_penalty, w.presence_penalty, C.byref(cfg),
                           np.ascontiguousarray(w.seeds[rows]), th, runs, ms, ids)
    if rc != 0:
        return None
    sec = float(np.median(ms)) / 1e3 + dfa_s + cap_s
    fast_cap = None
    F = O.ref("fast")
    if w.softcap > 0.0 and F is not None:
        # the reference Makefile's -O3 -ffast-math build of the soft-cap loop and of
        # the sampler on the same rows: bit agreement of the capped logits and of
        # the token ids with the strict build's
        raw = np.ascontiguousarray(w.logits[rows])
        fl = raw.copy()
        F.refh_softcap(fl.reshape(-1), fl.size, np.float32(w.softcap))
        same = int(np.count_nonzero(fl.view(np.uint32) == lg.view(np.uint32)))
        fids = np.zeros(len(rows), np.int32)
        fms = np.zeros(1, np.float64)
        rc = F.refh_time_batch(fl, len(rows), w.vocab, hoff.ctypes.data if hoff is not None else None,
                               hids.ctypes.data if hids is not None else None,
                               mask.ctypes.data if mask is not None else None, mw, w.order, w.repeat_penalty,
                               w.frequency_penalty, w.presence_penalty, C.byref(cfg),
                               np.ascontiguousarray(w.seeds[rows]), th, 1, fms, fids)
        if rc == 0:
            fast_cap = {"capped_logits_bit_identical": f"{same}/{fl.size}",
                        "ids_agree_with_strict": f"{int(np.sum(fids == ids))}/{len(rows)}"}
    out = {"value": round(len(rows) / sec, 1), "unit": "rows/s", "cores": th,
            "kind": "reference",
            "sample": f"rows 0..{len(rows) - 1}, median of {runs} runs, strict -std=c11 -O2 build"
                      + ("; DFA mask rows by oracle/oracle.c orc_dfa_mask, one per distinct state" if w.dfa is not None else "")
                      + (f"; soft-cap {w.softcap:g} first by oracle/oracle.c orc_softcap (host libm tanhf, one "
                         f"thread, src/core/context.c:873-876), one pass" if w.softcap > 0.0 else "")}
    if gpu_ids is not None:
        # the reference build's ids against the GPU's first-step ids (same seeds)
        out["ids_match_gpu"] = f"{int(np.sum(ids == np.asarray(gpu_ids)[rows]))}/{len(rows)}"
    if fast_cap is not None:
        out["fast_math_build"] = fast_cap
    return out


def dropin_vocab(V: int, seed: int = 7):
    """A synthetic vocabulary of JSON-ish token strings in CSR form (no NUL bytes)."""
    import numpy as np
    rng = np.random.Generator(np.random.PCG64(seed))
    alpha = np.frombuffer(b'{}[]":, 0123456789abcdefghijklmnopqrstuvwxyz', np.uint8)
    lens = np.minimum(rng.geometric(0.3, size=V), 12).astype(np.uint32)
    off = np.zeros(V + 1, np.uint32)
    off[1:] = np.cumsum(lens, dtype=np.uint64).astype(np.uint32)
    data = alpha[rng.integers(0, alpha.size, int(off[-1]))].astype(np.uint8)
    return off, np.ascontiguousarray(data)


def run_dropin(args) -> int:
    """One token through the drop-in C API in the order the reference's caller uses
    it (src/core/sampler_api.c:48-73): diskllm_grammar_apply_mask (JSON grammar,
    buffer reset before each token) -> sampler_apply_presence_penalty ->
    sampler_apply_repetition_penalty -> sampler_sample -> diskllm_grammar_advance,
    on row 0 of C2 (host logits, as the reference passes them; a fresh copy of the
    row before each token, outside the timed part).  Reports tokens/s, the PCIe
    bytes each token moves (from the copies the drop-ins make) and the strict
    reference build running the same sequence on one core."""
    import numpy as np
    from diskllm_amd import _lib, workloads
    L = _lib.lib()
    w = workloads.c2(rows=1)
    V = w.vocab
    off, data = dropin_vocab(V)
    scratch = C.create_string_buffer(256)
    voc = _lib.CsrVocab(off.ctypes.data, data.ctypes.data, V, C.cast(scratch, C.c_void_p), 256)
    get = C.cast(L.dlk_csr_token_str, C.c_void_p)
    hist = np.ascontiguousarray(w.hist_ids[w.hist_off[0]:w.hist_off[1]], np.int32)
    row0 = np.ascontiguousarray(w.logits[0])
    pres, rep, eos = 0.5, 1.15, V - 1
    cfg = _lib.SamplerConfig(1.0, 0, 0.9, 0.0, 12345)

    def run_seq(lib, steps, warm):
        s = lib.sampler_create(C.byref(cfg))
        g = lib.diskllm_grammar_init_json()
        logits = np.empty_like(row0)
        toks, ts = [], []
        for i in range(warm + steps):
            np.copyto(logits, row0)
            lib.diskllm_grammar_reset(g)
            t0 = time.perf_counter()
            lib.diskllm_grammar_apply_mask(g, logits.ctypes.data, V, C.byref(voc), get, eos)
            lib.sampler_apply_presence_penalty(logits.ctypes.data, V, hist.ctypes.data, hist.size, C.c_float(pres))
            lib.sampler_apply_repetition_penalty(logits.ctypes.data, V, hist.ctypes.data, hist.size, C.c_float(rep))
            tok = lib.sampler_sample(s, logits.ctypes.data, V)
            if tok != eos:
                piece = L.dlk_csr_token_str(C.byref(voc), tok)
                if piece:
                    lib.diskllm_grammar_advance(g, piece)
            t1 = time.perf_counter()
            if i >= warm:
                toks.append(tok)
                ts.append(t1 - t0)
        lib.diskllm_grammar_free(g)
        lib.sampler_free(s)
        return toks, ts

    toks, ts = run_seq(L, args.steps, args.warmup)
    med = float(np.median(ts))
    # bytes over PCIe per token, from the drop-ins' copies (host <-> device)
    ids = hist[(hist >= 0) & (hist < V)]
    nd, m = int(np.unique(ids).size), int(ids.size)
    words = (V + 31) // 32
    row_b = C.sizeof(_lib.GrammarRow)
    now = {"apply_mask": row_b + 4 * words + 4, "presence": 2 * 4 * nd + 4 * m + 8,
           "repetition": 2 * 4 * nd + 4 * m + 8, "sample": 4 * V + 8 + 4 + 4 + 8}
    before = {"apply_mask": row_b + 2 * 4 * V + 4, "presence": 2 * 4 * V + 4 * hist.size + 8,
              "repetition": 2 * 4 * V + 4 * hist.size + 8, "sample": 4 * V + 8 + 4 + 4 + 8}
    line = {
        "metric": "DROPIN: tokens/sec through the drop-in C API (mask -> presence -> repetition -> sample -> advance), "
                  "one row, vocab 151936",
        "value": round(1.0 / med, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(med * 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "DROPIN: row 0 of C2 (N(0,2^2) + Zipf bias, 256-id history, presence 0.5, "
                               "repetition 1.15, T 1.0, top-p 0.9), JSON grammar over a synthetic 151936-token "
                               "vocabulary (dlk_csr_token_str callback), host logits",
                   "rows": 1, "vocab": V, "parallelism": "none (1 GPU)",
                   "step": "median over steps of one token's calls, the logits copy before it excluded"},
        "pcie": {"bytes_per_token": sum(now.values()), "by_call": now,
                 "bytes_per_token_full_row_copies": sum(before.values()),
                 "note": "penalties move the touched ids only (12 bytes per distinct id each way + the history), "
                         "apply_mask brings back the packed mask, not the row"},
        "roofline": None,
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        from oracle import oracle as O
        R = O.ref("strict")
        if R is not None:
            for fn, at in (("sampler_create", [C.c_void_p]), ("sampler_free", [C.c_void_p]),
                           ("sampler_sample", [C.c_void_p, C.c_void_p, C.c_int]),
                           ("sampler_apply_presence_penalty", [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_float]),
                           ("sampler_apply_repetition_penalty", [C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_float]),
                           ("diskllm_grammar_apply_mask", [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p,
                                                           C.c_int])):
                getattr(R, fn).argtypes = at
            R.sampler_create.restype = C.c_void_p
            rtoks, rts = run_seq(R, min(args.steps, 50), args.warmup)   # the same rng steps as ours
            rmed = float(np.median(rts))
            same = sum(int(a == b) for a, b in zip(toks, rtoks))
            line["parity"] = f"{same}/{len(rtoks)} tokens identical to the strict reference build's sequence"
            line["cpu_baseline"] = {"value": round(1.0 / rmed, 1), "unit": "tokens/s", "cores": 1, "kind": "reference",
                                    "sample": f"the same sequence through the strict reference build "
                                              f"(src/core/grammar.c, src/sampler.c), median of {len(rts)} tokens"}
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-runs", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--temperature", type=float, default=1.0,
                    help="C2 at another temperature (the configuration's is 1.0; lower ones sharpen the rows)")
    ap.add_argument("--batches", type=int, default=12,
                    help="C2: distinct batches resident in HBM, one per step in turn (12 x 38.96 MB = 468 MB)")
    ap.add_argument("--config", default="C2", choices=["C1", "C2", "C3", "C4", "C5", "C5CAP", "CAP", "DROPIN"],
                    help="C2 (default) is the headline line; the others are the scope table's parity "
                         "configurations, measured the same way")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="instead of the benchmark, run --steps plain device-to-device copies of this many MiB "
                         "(the reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the rows of this path are independent and a multi-GPU run "
              "(row sharding) is not part of this build; run with --gpus 1", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    from diskllm_amd import _lib, api, workloads
    from oracle import oracle as O

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.config == "DROPIN":
        return run_dropin(args)
    if args.config != "C2":
        return run_other(args.config, args)
    dev = torch.device("cuda:0")
    if args.copy_probe_mib:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"probe": "copy", "bytes_read": n * 4, "bytes_written": n * 4, "launches": args.steps}))
        return 0
    # C2 over NB distinct batches resident at once (NB x 38.96 MB, past the
    # 256 MB Infinity Cache), one batch per step in turn: every step reads fresh
    # logits from HBM and meets its own rows' sums, as a decode loop does
    NB = max(1, args.batches)
    ws = [workloads.c2(seed=2 + 7919 * b) for b in range(NB)]
    for wb in ws:
        wb.temperature = args.temperature
    dbs = [api.to_device(w, device=dev) for w in ws]
    w, db = ws[0], dbs[0]
    params = api.params_of(w)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def parity_pass() -> tuple:
        """One dlk_sample call per batch from its rows' current rng states,
        checked against the oracle from the same states."""
        ok = tot = 0
        ids0 = None
        for wb, d in zip(ws, dbs):
            st = d.rng.cpu().numpy().view(np.uint64).copy()
            api.sample(d, params, sh)
            res = api.results(d)
            if ids0 is None:
                ids0 = res["ids"].copy()
            for r in range(wb.rows):
                ref = O.sample_row(O.prepared_row(wb, r), int(st[r]), wb.temperature, wb.top_k, wb.top_p,
                                   wb.min_p)
                ok += int(res["ids"][r] == ref["token"] and int(res["states"][r]) == ref["state"])
                tot += 1
        return ok, tot, ids0

    n_ok0, n_tot0, first_ids = parity_pass()       # from the seeds
    runs = [api.sampler(d, params, sh) for d in dbs]  # each call's structures built once
    for i in range(args.warmup):
        runs[i % NB]()
    torch.cuda.synchronize()

    def timed(seq) -> tuple:
        """Wall clock and one event pair on the launch stream around len(seq) calls."""
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        for f in seq:
            f()
        ev1.record(stream)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        return (t1 - t0) * 1e3 / len(seq), ev0.elapsed_time(ev1) / len(seq)

    ms_step, ms_kernel = timed([runs[i % NB] for i in range(args.steps)])
    ms_step_fixed, ms_kernel_fixed = timed([runs[0]] * args.steps)
    # per-launch spread: one event before each call, so consecutive events bracket
    # one launch (each interval also holds one event record)
    nl = min(args.steps, 2000)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(nl + 1)]
    torch.cuda.synchronize()
    for i in range(nl):
        evs[i].record(stream)
        runs[i % NB]()
    evs[nl].record(stream)
    torch.cuda.synchronize()
    per = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(nl)], np.float64)
    # parity again after the timed steps: every row's rng state has moved on
    n_ok1, n_tot1, _ = parity_pass()
    bytes_launch = BYTES_PER_ROW * ROWS
    achieved = bytes_launch / (ms_kernel * 1e-3) / 1e9
    rows_s = ROWS / (ms_step * 1e-3)

    line = {
        "metric": METRIC,
        "value": round(rows_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "C2: batch-64 full-vocab nucleus sampling, fp32 logits [64,151936], rep 1.15 / "
                               f"freq 0.3 / pres 0.5 over 256-id Zipf history, T {args.temperature:g}, top-p 0.9, "
                               "no top-k",
                   "rows": ROWS, "vocab": VOCAB, "history": HIST, "parallelism": "none (1 GPU)",
                   "batches": NB, "resident_bytes": NB * bytes_launch,
                   "step": f"one dlk_sample call on batch (step mod {NB}): {NB} distinct C2 batches "
                           f"(seeds 2 + 7919 b) resident in HBM, {NB * bytes_launch / 1e6:.0f} MB, "
                           f"past the 256 MB Infinity Cache"},
        "hbm_gbps": round(bytes_launch / (ms_step * 1e-3) / 1e9, 1),
        "hbm_frac": round(bytes_launch / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
        "parity": f"{n_ok0}/{n_tot0} token ids and rng states bit-identical to the oracle from the seeds, "
                  f"{n_ok1}/{n_tot1} after the timed steps ({NB} batches)",
        "roofline": {"bound": "hbm", "kernel": fused_kernel_name(ROWS, VOCAB), "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": profiled_traffic(fused_kernel_name(ROWS, VOCAB)), "bytes_per_launch": bytes_launch,
                     "ms_per_launch": round(ms_kernel, 5)},
        "library_source_stamp": _lib.source_stamp(),
        "launch_spread": {"n": nl, "mean_ms": round(float(per.mean()), 5),
                          "p50_ms": round(float(np.percentile(per, 50)), 5),
                          "p99_ms": round(float(np.percentile(per, 99)), 5), "max_ms": round(float(per.max()), 5),
                          "note": "an event before each launch; each interval holds one event record"},
        "fixed_batch": {"ms_per_step": round(ms_step_fixed, 5), "ms_per_launch": round(ms_kernel_fixed, 5),
                        "value": round(ROWS / (ms_step_fixed * 1e-3), 1),
                        "note": "batch 0 every step (39 MB, inside the Infinity Cache)"},
        "cpu_baseline": None,
    }
    res = {"ids": first_ids}
    if not args.no_cpu:
        nthreads = host_threads()
        cb = cpu_baseline(w, args.cpu_runs, nthreads)
        if cb is not None:
            top = cb[max(cb)]
            line["cpu_baseline"] = {
                "value": round(top["value"], 1), "unit": "rows/s", "cores": max(cb), "kind": "reference",
                "sample": f"full C2 batch (64 rows), median of {args.cpu_runs} runs, strict -std=c11 -O2 build",
                "single_thread": round(cb[1]["value"], 1),
                # the reference build's ids against the GPU's first-step ids (same seeds)
                "ids_match_gpu": bool(np.array_equal(top["ids"], res["ids"])),
            }
            fast = cpu_baseline(w, args.cpu_runs, nthreads, "fast")
            if fast is not None:
                ff = fast[nthreads]
                line["cpu_baseline"]["fast_math_build"] = {
                    "value": round(ff["value"], 1), "cores": nthreads,
                    "ids_agree_with_strict": f"{int(np.sum(ff['ids'] == top['ids']))}/{ROWS}"}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
