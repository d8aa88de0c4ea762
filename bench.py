#!/usr/bin/env python3
"""bench.py - batch-1 decode tokens/s of the 27B-shape W4A16 g64 model on one MI355X.

Workload (the metric's configuration): a dense 64-layer decoder,
hidden 5120, 40 q / 8 kv heads of 128, SwiGLU 17408, vocab 151936, int4 g64 weights for
every linear and the lm_head, fp16 KV cache pre-filled N(0,1) to 4096 positions, RoPE
theta 1e6, greedy argmax. Random-init weights of that architecture (no checkpoint).

A "step" is one replay of the captured decode step (one token). The timed region is K
back-to-back graph launches on the engine's stream, bracketed by device synchronisation,
timed with HIP events on that stream; inputs (weights, KV, control block) are resident in
HBM before it starts.

Also printed in the same JSON line:
  roofline     the int4 GEMV (the step's dominant kernel): algorithmic bytes of every GEMV
               launch of one step / their time, each linear's fused launch as the step issues
               it timed with HIP events on the engine's stream (beside it the same GEMVs as
               plain launches);
  cpu_baseline this repository's CPU oracle (the reference's scalar twins restated) running
               one full decode step of the same model on the host's cores;
  parity       GPU vs oracle logits of that same step (rel 2e-3 bar) and their argmax.
"""
import argparse
import hashlib
import ctypes as C
import importlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
mi = importlib.import_module("intel-arc-inference-server_amd")

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E vendor peak


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Events:
    def __init__(self, stream):
        self.L = mi.lib()
        self.stream = stream
        self.a, self.b = C.c_void_p(), C.c_void_p()
        mi.check(self.L.mi_event_create(C.byref(self.a)))
        mi.check(self.L.mi_event_create(C.byref(self.b)))

    def start(self):
        mi.check(self.L.mi_event_record(self.a, self.stream))

    def stop_ms(self):
        mi.check(self.L.mi_event_record(self.b, self.stream))
        ms = C.c_float()
        mi.check(self.L.mi_event_elapsed_ms(self.a, self.b, C.byref(ms)))
        return float(ms.value)


LINEARS = ["qkv", "o", "gate_up", "down", "lm_head"]
EPILOGUES = ["QKV (attn_prep fused)", "RESID (residual + next norm)", "SILU (silu * up)",
             "RESID (residual + next norm)", "LOGITS (+ argmax parts)"]


def linear_dims(d):
    qkv_n = (d.q_heads + 2 * d.kv_heads) * d.head_dim
    return [(d.hidden, qkv_n), (d.q_heads * d.head_dim, d.hidden), (d.hidden, 2 * d.inter),
            (d.inter, d.hidden), (d.hidden, d.vocab)]


def alg_bytes(K, N):
    """a GEMV launch's algorithmic bytes: int4 weights + fp16 scales + fp16 x in + fp32 y out"""
    return K * N // 2 + (K // 64) * N * 2 + 2 * K + 4 * N


def step_gemv_roofline(eng, reps=3):
    """The int4 GEMV launches the step runs: for each linear, `reps` rounds of its fused
    launch exactly as the step issues it (mi_engine_bench_linear: every layer's weights in
    turn, the engine's split-K width and epilogue), HIP events on the engine's stream. The
    step's GEMV time is sum over linears of (launches per step x time per launch); achieved =
    the step's GEMV algorithmic bytes / that time. Rewrites the engine's state (the caller
    resets it)."""
    L = mi.lib()
    d = eng.desc
    dims = linear_dims(d)
    per = []
    t_step = 0.0
    alg_step = 0
    for which, (K, N) in enumerate(dims):
        ms = C.c_float()
        mi.check(L.mi_engine_bench_linear(eng._h, which, reps, C.byref(ms)), "engine_bench_linear")
        n = 1 if which == 4 else d.layers
        a = alg_bytes(K, N)
        t_step += ms.value * n
        alg_step += a * n
        per.append({"linear": LINEARS[which], "epilogue": EPILOGUES[which], "K": K, "N": N,
                    "S": eng.linear_s(which), "launches_per_step": n,
                    "avg_launch_us": round(ms.value * 1e3, 3),
                    "gbs": round(a / (ms.value * 1e-3) / 1e9, 1),
                    "frac": round(a / (ms.value * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    launches = sum(x["launches_per_step"] for x in per)
    achieved = alg_step / (t_step * 1e-3) / 1e9
    return {
        "kernel": "gemv_w4a16_kernel, the step's fused launches (int4 g64 GEMV, M=1)",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": None,
        "launches_per_step": launches,
        "alg_bytes_per_step": alg_step,
        "gemv_ms_per_step": round(t_step, 4),
        "avg_launch_us": round(t_step / launches * 1e3, 3),
        "per_linear": per,
    }, alg_step


def gemv_roofline(eng, reps=3):
    """The plain sweep: every int4 GEMV of one step as a plain partials launch (no epilogue),
    each on the engine's own weights and split-K width, back to back on the engine's stream;
    HIP events around `reps` such sweeps (algorithmic bytes as alg_bytes)."""
    L = mi.lib()
    d = eng.desc
    st = eng.stream
    H, I, V = d.hidden, d.inter, d.vocab
    qkv_n = (d.q_heads + 2 * d.kv_heads) * d.head_dim
    dims = [(H, qkv_n), (d.q_heads * d.head_dim, H), (H, 2 * I), (I, H)]
    S = [eng.linear_s(w) for w in range(5)]
    kmax = max(H, I, d.q_heads * d.head_dim)
    nmax = max(s * n for s, (_, n) in zip(S, dims + [(H, V)]))
    xbuf, pbuf = C.c_void_p(), C.c_void_p()
    mi.check(L.mi_malloc(C.byref(xbuf), kmax * 2))
    mi.check(L.mi_malloc(C.byref(pbuf), nmax * 4))
    mi.check(L.mi_fill_f16(xbuf, kmax, 99, 1, 0.0, 1.0, st))
    launches = []
    for li in range(d.layers):
        for w, (K, N) in enumerate(dims):
            q, _ = eng.tensor(2 * w, li)
            s, _ = eng.tensor(2 * w + 1, li)
            launches.append((q, s, K, N, S[w]))
    lq, _ = eng.tensor(mi.T_LM_Q)
    ls, _ = eng.tensor(mi.T_LM_S)
    launches.append((lq, ls, H, V, S[4]))
    alg = sum(K * N // 2 + (K // 64) * N * 2 + 2 * K + 4 * N for _, _, K, N, _ in launches)

    def sweep():
        for q, s, K, N, Sx in launches:
            mi.check(L.mi_gemv_w4a16(q, s, xbuf, pbuf, 1, K, N, Sx, st))

    sweep()
    mi.check(L.mi_stream_sync(st))
    ev = Events(st)
    ev.start()
    for _ in range(reps):
        sweep()
    ms = ev.stop_ms()
    mi.check(L.mi_free(xbuf))
    mi.check(L.mi_free(pbuf))
    per_launch_s = ms * 1e-3 / (reps * len(launches))
    bytes_per_launch = alg / len(launches)
    achieved = bytes_per_launch / per_launch_s / 1e9
    return {
        "kernel": "gemv_w4a16_kernel (int4 g64 GEMV, M=1)",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": None,
        "launches_per_step": len(launches),
        "alg_bytes_per_step": alg,
        "gemv_ms_per_step": round(per_launch_s * len(launches) * 1e3, 4),
        "avg_launch_us": round(per_launch_s * 1e6, 3),
    }, alg


GEMV_SOURCES = ("gemv_w4a16.hip", "gemv_core.h", "mi_common.h")


def gemv_source_sha():
    """sha256 (16 hex) of the GEMV kernel's sources: a traffic profile is reported only for the
    kernel it measured."""
    h = hashlib.sha256()
    for f in GEMV_SOURCES:
        with open(os.path.join(ROOT, "intel-arc-inference-server_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def pmc_summary(fetch_dir, write_dir):
    """Reduces two rocprofv3 --pmc runs of `bench.py --only roofline` (FETCH_SIZE, then
    WRITE_SIZE) to HBM bytes per GEMV launch: each counter (KiB per dispatch) is scaled by what
    it reads for a kernel of known size in the same run - the 2 GiB stream read (fetch) and the
    2 GiB fill (write). Writes profiles/gemv_w4a16_27b_step_traffic.json (the step's fused
    launches) and profiles/gemv_w4a16_27b_traffic.json (the plain sweep), stamped with the
    GEMV sources' hash, and prints the per-epilogue table."""
    import csv
    import glob
    import re

    def load(d, ctr):
        path = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)[0]
        per, name, grid = {}, {}, {}
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] != ctr:
                    continue
                k = r["Dispatch_Id"]
                per[k] = per.get(k, 0.0) + float(r["Counter_Value"])
                name[k], grid[k] = r["Kernel_Name"], int(r["Grid_Size"])
        return per, name, grid
    fe, fn, fg = load(fetch_dir, "FETCH_SIZE")
    wr, wn, wg = load(write_dir, "WRITE_SIZE")
    two = float(2 << 30)
    fetch_factor = two / (1024.0 * max(v for k, v in fe.items() if "stream_read_kernel" in fn[k]))
    write_factor = two / (1024.0 * max(v for k, v in wr.items() if "fill_u32_kernel" in wn[k]))

    def epi(n):
        m = re.search(r"gemv_w4a16_kernel<\s*\d+,\s*\d+,\s*(\d+)", n)
        return None if m is None else int(m.group(1))
    sha = gemv_source_sha()
    shapes = {"qkv": (5120, 7168, 5), "o": (5120, 5120, 1), "gate_up": (5120, 34816, 2), "down": (17408, 5120, 1),
              "lm_head": (5120, 151936, 3)}
    # the engine's split-K widths (its fused epilogues' choice; the plain sweep launches at the same S)
    split = {lin: int(mi.lib().mi_gemv_pick_s_ex(K, N, e)) for lin, (K, N, e) in shapes.items()}
    per_step = {"qkv": 64, "o": 64, "gate_up": 64, "down": 64, "lm_head": 1}
    lines = [f"fetch factor {fetch_factor:.4f} (a 2 GiB stream read), write factor {write_factor:.4f} (a 2 GiB "
             f"fill), GEMV sources {sha}", "",
             "| launches | linear | EPI | S | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic MB | "
             "algorithmic MB | traffic / algorithmic |", "|---|---|---|---|---|---|---|---|---|---|"]
    for fused, fname, what in ((True, "gemv_w4a16_27b_step_traffic.json",
                                "27B-shape step GEMVs, the step's fused launches (EPI 1 RESID, 2 SILU, 3 LOGITS, 5 QKV)"),
                               (False, "gemv_w4a16_27b_traffic.json", "27B-shape GEMV sweep, plain launches (EPI 0)")):
        tot_t = tot_a = 0.0
        for lin, (K, N, e) in shapes.items():
            S = split[lin]
            e_run = e if fused else 0
            rows_g = S + 1 if fused and e in (1, 5) else S
            grid = N // 64 * rows_g * 256
            F = [v for k, v in fe.items() if epi(fn[k]) == e_run and fg[k] == grid]
            W = [v for k, v in wr.items() if epi(wn[k]) == e_run and wg[k] == grid]
            fk, wk = sum(F) / len(F), sum(W) / len(W)
            t = fk * 1024 * fetch_factor + wk * 1024 * write_factor
            a = K * N // 2 + (K // 64) * N * 2 + 2 * K + 4 * N
            tot_t += t * per_step[lin]
            tot_a += a * per_step[lin]
            lines.append(f"| {'fused' if fused else 'plain'} | {lin} | {e_run} | {S} | {len(F)} | {fk:.1f} | {wk:.1f} | "
                         f"{t / 1e6:.2f} | {a / 1e6:.2f} | {t / a:.3f} |")
        n = sum(per_step.values())
        lines.append(f"| {'fused' if fused else 'plain'} | per launch of the step's {n} | | | | | | "
                     f"{tot_t / n / 1e6:.3f} | {tot_a / n / 1e6:.3f} | {tot_t / tot_a:.3f} |")
        prof = {"kernel": "gemv_w4a16_kernel", "workload": what, "traffic_bytes_per_launch": int(tot_t / n),
                "alg_bytes_per_launch": int(tot_a / n), "fetch_factor": round(fetch_factor, 4),
                "write_factor": round(write_factor, 4), "split_k": split,
                "source_sha": sha, "sources": list(GEMV_SOURCES),
                "command": "rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) -- python3 bench.py --only roofline; "
                           "python3 bench.py --pmc-summary FETCH_DIR WRITE_DIR"}
        with open(os.path.join(ROOT, "profiles", fname), "w") as f:
            json.dump(prof, f, indent=1)
    print("\n".join(lines))


def profiled_traffic(eng, name="gemv_w4a16_27b_traffic.json"):
    """HBM bytes per GEMV launch from a committed PMC summary under profiles/ (FETCH_SIZE and
    WRITE_SIZE runs of the launches, each scaled by a kernel of known size), provided it was
    measured at the split-K widths this engine uses; else None. gemv_w4a16_27b_traffic.json:
    the plain sweep; gemv_w4a16_27b_step_traffic.json: the step's fused launches."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        prof = json.load(f)
    mine = dict(zip(["qkv", "o", "gate_up", "down", "lm_head"], [eng.linear_s(w) for w in range(5)]))
    if prof.get("split_k") != mine:
        log(f"bench: profiled traffic was measured at S {prof.get('split_k')}, engine uses {mine}: not reported")
        return None
    if prof.get("source_sha") != gemv_source_sha():
        log(f"bench: profiled traffic ({name}) was measured on other GEMV sources: not reported")
        return None
    return prof["traffic_bytes_per_launch"]


def stream_read_rate(st):
    L = mi.lib()
    nbytes = 2 << 30
    buf, sink = C.c_void_p(), C.c_void_p()
    mi.check(L.mi_malloc(C.byref(buf), nbytes))
    mi.check(L.mi_malloc(C.byref(sink), 8192 * 4))
    mi.check(L.mi_fill_u32(buf, nbytes // 4, 5, st))
    mi.check(L.mi_stream_read(buf, nbytes, sink, st))
    mi.check(L.mi_stream_sync(st))
    ev = Events(st)
    ev.start()
    for _ in range(5):
        mi.check(L.mi_stream_read(buf, nbytes, sink, st))
    ms = ev.stop_ms()
    mi.check(L.mi_free(buf))
    mi.check(L.mi_free(sink))
    return nbytes * 5 / (ms * 1e-3) / 1e9


class Dev:
    """Device buffers for the secondary measurements (freed together)."""

    def __init__(self):
        self.L = mi.lib()
        self.ptrs = []

    def alloc(self, nbytes):
        p = C.c_void_p()
        mi.check(self.L.mi_malloc(C.byref(p), nbytes))
        self.ptrs.append(p)
        return p

    def upload(self, arr):
        p = self.alloc(arr.nbytes)
        mi.check(self.L.mi_memcpy_h2d(p, arr.ctypes.data, arr.nbytes, None))
        return p

    def free(self):
        for p in self.ptrs:
            mi.check(self.L.mi_free(p))
        self.ptrs = []


def time_calls(st, fn, reps, warm=5):
    for i in range(warm):
        fn(i)
    mi.check(mi.lib().mi_stream_sync(st))
    ev = Events(st)
    ev.start()
    for i in range(reps):
        fn(i)
    return ev.stop_ms() / reps * 1e3  # us per call


def measure_cfg1(st):
    """one W4A16 GEMV, K = N = 4096, M = 1, x N(0,1), scales
    U(0.002, 0.02), out fp16; >= 100 launches cycling over 96 weight copies (> 3x the 256 MB
    MALL). A call = the split-K GEMV + the fold of its partials to fp16."""
    L, D = mi.lib(), Dev()
    K = N = 4096
    copies = 96
    S = L.mi_gemv_pick_s(K, N)
    qw, sc = [], []
    for c in range(copies):
        q = D.alloc(K // 8 * N * 4)
        s = D.alloc(K // 64 * N * 2)
        mi.check(L.mi_fill_u32(q, K // 8 * N, 1000 + c, st))
        mi.check(L.mi_fill_f16(s, K // 64 * N, 5000 + c, 0, 0.002, 0.02, st))
        qw.append(q)
        sc.append(s)
    x = D.alloc(K * 2)
    mi.check(L.mi_fill_f16(x, K, 1234, 1, 0.0, 1.0, st))
    part = D.alloc(S * N * 4)
    out = D.alloc(N * 2)
    gemv = lambda i: mi.check(L.mi_gemv_w4a16(qw[i % copies], sc[i % copies], x, part, 1, K, N, S, st))

    def call(i):
        gemv(i)
        mi.check(L.mi_fold_partials(part, out, None, S, 1, N, st))
    # one launch: the GEMV with the fp16 fold as its epilogue (split-K capped for the fold)
    S1 = L.mi_gemv_pick_s_ex(K, N, mi.EPI_F16OUT)
    part1 = D.alloc(S1 * N * 4)
    mi.check(L.mi_gemv_handoff_init(part1, S1 * N, st))  # hand-off words: empty on entry and after each call
    ep = mi.GemvEpilogue(kind=mi.EPI_F16OUT, out16=out.value)
    fused = lambda i: mi.check(L.mi_gemv_w4a16_ex(qw[i % copies], sc[i % copies], x, part1, 1, K, N, S1,
                                                  C.byref(ep), st))
    t_call = time_calls(st, call, 192)
    t_gemv = time_calls(st, gemv, 192)
    t_fused = time_calls(st, fused, 192)
    D.free()
    alg = K * N // 2 + (K // 64) * N * 2 + 2 * K + 2 * N  # 8,929,280 B
    return {"workload": "BASELINE configs[0]: W4A16 GEMV K=N=4096, M=1, fp16 out",
            "us_per_call": round(t_fused, 3), "split_k": S1, "gbs_per_call": round(alg / t_fused / 1e3, 1),
            "frac_of_peak_per_call": round(alg / t_fused / 1e3 / HBM_PEAK_GBS, 4),
            "two_launches": {"split_k": S, "us_per_call": round(t_call, 3), "us_gemv_kernel_only": round(t_gemv, 3),
                             "gbs_gemv_kernel": round(alg / t_gemv / 1e3, 1)},
            "alg_bytes": alg}


def measure_lm_head_int8(st):
    """The int8 lm_head (spec 9, gemv_i8w) at the 27B head's shape: K = 5120, N = 151936, M = 1,
    int8 uniform [-127, 127] with fp32 row scales; calls alternate between two copies
    (1.56 GB, past the 256 MB MALL). Algorithmic bytes = K N + 4 N (weights and scales) + 2 K
    (x) + 4 N (fp32 logits)."""
    L, D = mi.lib(), Dev()
    K, N, copies = 5120, 151936, 2
    ws, ss = [], []
    for c in range(copies):
        w = D.alloc(K * N)
        s = D.alloc(N * 4)
        mi.check(L.mi_fill_i8(w, K * N, 70 + c, -127, 127, st))
        mi.check(L.mi_fill_f32(s, N, 80 + c, 0, 2e-4, 1.2e-3, 0, st))
        ws.append(w)
        ss.append(s)
    x = D.alloc(K * 2)
    mi.check(L.mi_fill_f16(x, K, 90, 1, 0.0, 1.0, st))
    out = D.alloc(N * 4)
    call = lambda i: mi.check(L.mi_gemv_i8w(ws[i % copies], ss[i % copies], x, out, 1, K, N, st))
    t = time_calls(st, call, 40)
    D.free()
    alg = K * N + 4 * N + 2 * K + 4 * N
    return {"workload": "int8 lm_head GEMV (gemv_i8w) at the 27B head: K=5120, N=151936, M=1",
            "us_per_call": round(t, 2), "gbs": round(alg / t / 1e3, 1),
            "frac_of_peak": round(alg / t / 1e3 / HBM_PEAK_GBS, 4), "alg_bytes": alg}


def measure_mtp(args, moe=False, w16=False):
    """The MTP draft lists at the 27B shape (the head: one more dense layer at the model's
    shapes, sharing the embedding and lm_head; random-init; w16: its linears in 16 bits as the
    reference keeps a dense head, else int4) or, moe, on the configs[3] MoE model
    (the head: one MoE layer of its shape): the plain step with the head's K/V fill, one draft
    list (the head at one row: front, attention over its own cache, FFN, head) and the verify
    step at k = 3 (four rows, the fill over them), at context `--context`. The weights are
    random, so the acceptance rate says nothing about a trained head; the time per list is what
    the speculative loop pays."""
    ctx = args.context
    max_len = ((ctx + 64 + 1 + 63) // 64) * 64
    desc = mi.desc_moe_cfg4(max_len=max_len) if moe else mi.desc_27b(max_len=max_len)
    desc.mtp = 1
    desc.mtp_w16 = 1 if w16 else 0
    eng = mi.Engine(desc, seed=args.seed)  # the main model's weights are the bench engine's
    eng.capture(1)
    eng.capture(4)
    st = eng.stream
    eng.reset(ctx, 1000)
    eng.generate(2)
    pos = int(eng.ctrl()[mi.CTRL_POS])
    plain = time_calls(st, lambda i: eng.replay(1), 20)
    eng.reset(pos, 1000)
    eng.draft(1)  # captures the draft graph
    t0 = time.perf_counter()
    reps = 20
    for _ in range(reps):
        eng.draft(3)
    t_draft3 = (time.perf_counter() - t0) / reps * 1e3
    drafts = eng.draft(3)
    # the random-init model's fp16 activations can leave the range on some rows (the verify
    # call then fails loudly, after its step ran): the time is the same, the flag says so
    finite = True
    c0 = eng.ctrl()
    t_verify = 0.0
    for _ in range(reps):
        eng.reset(int(c0[mi.CTRL_POS]), int(c0[mi.CTRL_CUR]))  # (a failed verify leaves no valid cur)
        t0 = time.perf_counter()
        try:
            eng.verify(drafts)
        except mi.MiError as ex:
            if "not finite" not in str(ex):
                raise
            finite = False
        t_verify += time.perf_counter() - t0
    t_verify = t_verify / reps * 1e3
    eng.reset(int(c0[mi.CTRL_POS]), int(c0[mi.CTRL_CUR]))
    c = eng.ctrl()
    assert c[mi.CTRL_DEBUG] == 0, (hex(c[mi.CTRL_DEBUG]), list(drafts), [hex(v) for v in c[:20]],
                                   [hex(v) for v in eng.to_host(mi.T_MTP_CTRL, 0, np.uint32)[:20]])
    eng.close()
    return {"workload": ("configs[3] MoE model" if moe else "27B shape") +
                        f" with an MTP head ({'16-bit' if w16 else 'int4' if not moe else 'MoE'} linears, "
                        f"random-init), context {ctx}",
            "plain_step_with_fill_ms": round(plain / 1e3, 4),
            "draft_3_ms": round(t_draft3, 3), "draft_list_ms": round(t_draft3 / 3, 3),
            "verify_k3_ms": round(t_verify, 3), "verify_logits_finite": finite,
            "note": "draft and verify times are host wall clock around each call (one "
                    "synchronisation per call); the plain step is HIP-event timed"}


def measure_verify_steps(eng, ctx, tok0, rows=(1, 2, 3, 4, 5, 6, 7, 8), reps=20):
    """The small-M verify step (the reference's gemm_sm lists, docs/12-kernels.md:409-412): the
    captured M-row step with all M rows live at context `ctx` (mi_engine_bench_verify: per step
    the rows' control reset and the graph, HIP-event timed), and its cost in plain steps."""
    ms = {}
    for M in rows:
        eng.reset(ctx, tok0)
        t = C.c_float()
        mi.check(mi.lib().mi_engine_bench_verify(eng._h, M, reps, C.byref(t)), "engine_bench_verify")
        ms[M] = float(t.value)
    eng.reset(ctx, tok0)
    return {"workload": f"27B-shape verify step, M live rows at context {ctx} (ids: the current token in each)",
            "ms": {str(M): round(v, 4) for M, v in ms.items()},
            "plain_steps": {str(M): round(v / ms[1], 3) for M, v in ms.items()}}


def measure_cfg3(st, ctx, tgt=64):
    """one layer's decode attention at context `ctx`, 40 q / 8 kv heads
    of 128, int8 K/V uniform [-127, 127] with fp16 scales U(0.005, 0.05) per (pos, kv head),
    64-token pages in a shuffled table; attn_decode + attn_reduce per call at 64 blocks per kv
    head (the engine's blocking; 512 / 2048 positions per block). The calls cycle
    through enough cache copies (at least 4, at least 640 MB in all) that none is still in
    the 256 MB MALL when it is read again."""
    L, D = mi.lib(), Dev()
    QH, KVH, HD, P = 40, 8, 128, 64
    rng = np.random.default_rng(ctx)
    copy_bytes = 2 * KVH * ctx * HD + 2 * KVH * ctx * 2
    copies = max(4, -(-640 * 2**20 // copy_bytes))
    caches = []
    for c in range(copies):
        k8, v8 = D.alloc(KVH * ctx * HD), D.alloc(KVH * ctx * HD)
        ks, vs = D.alloc(KVH * ctx * 2), D.alloc(KVH * ctx * 2)
        mi.check(L.mi_fill_i8(k8, KVH * ctx * HD, 31 + 4 * c, -127, 127, st))
        mi.check(L.mi_fill_i8(v8, KVH * ctx * HD, 32 + 4 * c, -127, 127, st))
        mi.check(L.mi_fill_f16(ks, KVH * ctx, 33 + 4 * c, 0, 0.005, 0.05, st))
        mi.check(L.mi_fill_f16(vs, KVH * ctx, 34 + 4 * c, 0, 0.005, 0.05, st))
        caches.append((k8, v8, ks, vs))
    pages = D.upload(rng.permutation(ctx // P).astype(np.uint32))
    q = D.alloc(QH * HD * 4)
    mi.check(L.mi_fill_f32(q, QH * HD, 35, 1, 0.0, 1.0, 1, st))
    ctrl_h = np.zeros(64, np.uint32)
    ctrl_h[0], ctrl_h[1] = ctx - 1, 1
    ctrl = D.upload(ctrl_h)
    part = D.alloc(QH * tgt * (HD + 2) * 4)
    out = D.alloc(QH * HD * 2)
    sh = mi.AttnShape(QH, KVH, HD, HD, 0, (QH + 2 * KVH) * HD, QH * HD, (QH + KVH) * HD,
                      float(np.float32(1 / np.sqrt(HD))), 1e-6)

    def call(i):
        k8, v8, ks, vs = caches[i % copies]
        mi.check(L.mi_attn_decode(ctrl, q, 1, k8, v8, ks, vs, HD, ctx * HD, 1, ctx, pages, P, ctx, part, 1, tgt,
                                  C.byref(sh), st))
        mi.check(L.mi_attn_reduce(ctrl, part, None, out, 1, tgt, ctx, C.byref(sh), st))
    t = time_calls(st, call, 50)
    D.free()
    alg = 2 * KVH * HD * ctx + 2 * KVH * ctx * 2
    return {"context": ctx, "tgt": tgt, "us_per_layer": round(t, 2), "alg_bytes": alg, "gbs": round(alg / t / 1e3, 1),
            "frac_of_peak": round(alg / t / 1e3 / HBM_PEAK_GBS, 4), "cache_copies": copies}


def measure_cfg5(st):
    """the small-M verify GEMV, M in {4, 8, 16} on the 27B shapes
    (gate||up 5120->34816, down 17408->5120, qkv 5120->7168), activations N(0,1); weight
    copies cycled past the MALL. Reports HBM rate and MFMA rate (2 M K N flops)."""
    L, D = mi.lib(), Dev()
    rows = []
    for name, K, N in (("gate_up", 5120, 34816), ("down", 17408, 5120), ("qkv", 5120, 7168)):
        wb = K * N // 2 + (K // 64) * N * 2
        copies = max(3, -(-768 * 2**20 // wb))
        S = L.mi_gemv_pick_s(K, N)
        qw = [D.alloc(K // 8 * N * 4) for _ in range(copies)]
        sc = [D.alloc(K // 64 * N * 2) for _ in range(copies)]
        for c in range(copies):
            mi.check(L.mi_fill_u32(qw[c], K // 8 * N, 70 + c, st))
            mi.check(L.mi_fill_f16(sc[c], K // 64 * N, 170 + c, 0, 0.002, 0.02, st))
        x = D.alloc(16 * K * 2)
        mi.check(L.mi_fill_f16(x, 16 * K, 9, 1, 0.0, 1.0, st))
        part = D.alloc(S * 16 * N * 4)
        for M in (1, 4, 8, 16):
            fn = lambda i: mi.check(L.mi_gemv_w4a16(qw[i % copies], sc[i % copies], x, part, M, K, N, S, st))
            t = time_calls(st, fn, 60)
            alg = wb + 2 * M * K + 4 * M * N
            tf = 2 * M * K * N / t / 1e6
            rows.append({"linear": name, "K": K, "N": N, "M": M, "split_k": S, "us": round(t, 2),
                         "gbs": round(alg / t / 1e3, 1), "hbm_frac": round(alg / t / 1e3 / HBM_PEAK_GBS, 4),
                         "tflops": round(tf, 2), "mfma_frac_fp16": round(tf / 2500.0, 5)})
        D.free()
    return rows


def time_prefill(eng, T):
    """(ms, finite) of one T-token prefill from position 0 in one chunk (synthetic ids); the
    first call, which allocates the prefill scratch, is not timed. The synthetic 27B model's
    f16 residual leaves the f16 range somewhere in a 2048-token prompt (every prompt seed
    tried): the engine then fails the call after the work is done. The time does not depend on
    the values; `finite` says whether the last position's logits were."""
    ids = np.random.default_rng(7).integers(0, eng.desc.vocab_used, T).astype(np.uint32)

    def run():
        try:
            eng.prefill(ids, T)
            return True
        except mi.MiError as e:
            if "not finite" not in str(e):
                raise
            return False

    eng.reset(0, 0)
    run()
    eng.reset(0, 0)
    ev = Events(eng.stream)
    ev.start()
    finite = run()
    ms = ev.stop_ms()
    c = eng.ctrl()
    assert c[mi.CTRL_POS] == T and c[mi.CTRL_DEBUG] == 0, c[:20]
    return ms, finite


def measure_prefill(eng, T=2048):
    """The chunked prefill (the reference's Engine::prefill, north_star's small-M/prefill GEMM on
    the matrix cores): one T-token prompt from position 0 in one chunk on the 27B engine, and
    the int4 GEMM alone at T rows on layer 0's four linears (MFMA rate against the 2.5 PFLOP/s
    dense fp16 peak; 2 T K N flops per call)."""
    L, d, st = mi.lib(), eng.desc, eng.stream
    ms, finite = time_prefill(eng, T)
    out = {"workload": f"27B-shape prefill of a {T}-token prompt in one chunk (synthetic ids, random-init weights)",
           "ms": round(ms, 2), "tokens_per_s": round(T / ms * 1e3, 1), "logits_finite": finite}
    H, QH, KVH, HD, I = d.hidden, d.q_heads, d.kv_heads, d.head_dim, d.inter
    D = Dev()
    x = D.alloc(T * max(H, I, QH * HD) * 2)
    mi.check(L.mi_fill_f16(x, T * max(H, I, QH * HD), 5, 1, 0.0, 1.0, st))
    o = D.alloc(T * 2 * I * 4)
    gemms = []
    for name, (kq, ks), K, N in (("qkv", (mi.T_QKV_Q, mi.T_QKV_S), H, (QH + 2 * KVH) * HD),
                                 ("o", (mi.T_O_Q, mi.T_O_S), QH * HD, H),
                                 ("gate_up", (mi.T_GU_Q, mi.T_GU_S), H, 2 * I),
                                 ("down", (mi.T_DOWN_Q, mi.T_DOWN_S), I, H)):
        qp, sp = eng.tensor(kq, 0)[0], eng.tensor(ks, 0)[0]
        fn = lambda i: mi.check(L.mi_gemm_w4a16(qp, sp, x, o, T, K, N, st))
        t = time_calls(st, fn, 10, warm=2)
        tf = 2.0 * T * K * N / t / 1e6
        gemms.append({"linear": name, "T": T, "K": K, "N": N, "us": round(t, 1), "tflops": round(tf, 1),
                      "mfma_frac_fp16": round(tf / 2500.0, 4)})
    D.free()
    out["gemm_w4a16"] = gemms
    return out


def measure_bf16_step(args):
    """BASELINE configs[1]'s model with bf16 activations, the reference's own type (the f16 run
    is the headline, as BASELINE specifies): tokens/s of the captured step at seed 42, where the
    f16 activations of the same synthetic model leave the f16 range in the first step."""
    desc = mi.desc_27b(max_len=((args.context + 64 + 1 + 63) // 64) * 64, act_bf16=1)
    eng = mi.Engine(desc, seed=42)
    eng.capture(1)
    eng.reset(args.context, 1000)
    for _ in range(4):
        eng.replay(1)
    mi.check(mi.lib().mi_device_sync())
    ev = Events(eng.stream)
    ev.start()
    n = 32
    for _ in range(n):
        eng.replay(1)
    ms = ev.stop_ms() / n
    c = eng.ctrl()
    assert c[mi.CTRL_DEBUG] == 0, hex(c[mi.CTRL_DEBUG])
    eng.close()
    return {"workload": "BASELINE configs[1] with bf16 activations (seed 42: the f16 run of this seed leaves the "
                        "f16 range; logits finite here)", "ms_per_step": round(ms, 4),
            "tokens_per_s": round(1000.0 / ms, 2)}


def measure_cfg4(args, kv_int8=0):
    """a 40-layer MoE decoder (hidden 2048, 256 experts top 8 + shared,
    expert inter 512, attention 16 q / 2 kv of 256, vocab 151936 assumed) at context 4096:
    tokens/s of the captured step, and one step against the CPU oracle. kv_int8: the same
    model over the int8 rotated KV cache (the reference's --kv-cache int8)."""
    max_len = ((args.context + 64 + 1 + 63) // 64) * 64
    desc = mi.desc_moe_cfg4(max_len=max_len)
    desc.kv_int8 = kv_int8
    eng = mi.Engine(desc, seed=args.seed + 1)
    eng.capture(1)
    st = eng.stream
    out = {"workload": "BASELINE configs[3]: MoE decode step (40 layers, 256 experts top 8 + shared)"
                       + (", int8 rotated KV cache" if kv_int8 else "")}
    if not args.no_cpu:
        eng.reset(args.context, 1000)
        dt, cpu_logits, cpu_am, threads = cpu_oracle_step(eng, 1000, args.context)
        eng.reset(args.context, 1000)
        gpu_tok = int(eng.generate(1)[0])
        g = eng.logits(1)[0].astype(np.float64)
        w = cpu_logits.astype(np.float64)
        err = np.abs(g - w)
        out["parity"] = {"max_err_over_max_logit": float(err.max() / np.abs(w).max()),
                         "within_rel_2e-3": bool(np.all(err <= 2e-3 * np.abs(w) + 2e-3 * np.abs(w).max())),
                         "argmax_gpu": gpu_tok, "argmax_oracle": cpu_am}
        out["cpu_tokens_per_s"] = round(1.0 / dt, 4)
    eng.reset(args.context, 1000)
    for _ in range(4):
        eng.replay(1)
    mi.check(mi.lib().mi_device_sync())
    ev = Events(st)
    ev.start()
    n = 32
    for _ in range(n):
        eng.replay(1)
    ms = ev.stop_ms() / n
    c = eng.ctrl()
    assert c[mi.CTRL_DEBUG] == 0, hex(c[mi.CTRL_DEBUG])
    if not kv_int8:
        # the MoE model's chunked prefill (its expert FFN runs the decode expert kernels on 16-row
        # slices); after the decode timing, since it rewrites the cache's first T positions
        T = 2048
        pms, finite = time_prefill(eng, T)
        out["prefill"] = {"workload": f"prefill of a {T}-token prompt in one chunk (synthetic ids)",
                          "ms": round(pms, 2), "tokens_per_s": round(T / pms * 1e3, 1), "logits_finite": finite}
    eng.close()
    H, E, I, QH, KVH, HD, V = 2048, 256, 512, 16, 2, 256, 151936
    per_layer = 9 * (2 * I * H + I * H) * 17 // 32 + (E + 1 + 15) // 16 * 16 * H * 2 \
        + ((QH + 2 * KVH) * HD * H + QH * HD * H) * 17 // 32 \
        + 2 * KVH * (args.context + 1) * (HD + 2 if kv_int8 else HD * 2)
    alg = 40 * per_layer + H * V * 17 // 32
    out.update({"ms_per_step": round(ms, 4), "tokens_per_s": round(1000.0 / ms, 2), "alg_bytes_per_token": alg,
                "gbs": round(alg / ms / 1e6, 1)})
    return out


class CpuOracle:
    """The same model wired into the CPU oracle (the reference's scalar twins restated;
    OpenMP over columns in the GEMV twins, each column's order unchanged, so any thread count
    gives the same bits). Host copies of every weight are taken once."""

    def __init__(self, eng):
        import oracle as O
        self.O = O
        d = self.d = eng.desc
        H, I, HD, QH, KVH = d.hidden, d.inter, d.head_dim, d.q_heads, d.kv_heads
        S = [eng.linear_s(w) for w in range(5)]
        dims = [(H, (QH + 2 * KVH) * HD), (QH * HD, H), (H, 2 * I), (I, H)]
        keep = self.keep = []

        def h(kind, layer, dt):
            a = eng.to_host(kind, layer, dt)
            keep.append(a)
            return a.ctypes.data

        moe = d.experts > 0
        layers = (O.Layer * d.layers)()
        keep.append(layers)
        for li in range(d.layers):
            lins = [O.Linear(h(2 * w, li, np.uint32), h(2 * w + 1, li, np.uint16), K, N, S[w])
                    if not (moe and w >= 2) else O.Linear(None, None, K, N, 1)
                    for w, (K, N) in enumerate(dims)]
            Ly = layers[li]
            Ly.qkv, Ly.o, Ly.gate_up, Ly.down = lins
            if moe:
                Ly.router = h(mi.T_ROUTER, li, np.uint16)
                Ly.moe_gu = h(mi.T_MOE_GU, li, np.uint32)
                Ly.moe_dn = h(mi.T_MOE_DN, li, np.uint32)
            Ly.in_norm = h(mi.T_IN_NORM, li, np.float32)
            Ly.post_norm = h(mi.T_POST_NORM, li, np.float32)
            if d.qk_norm:
                Ly.q_norm = h(mi.T_Q_NORM, li, np.float32)
                Ly.k_norm = h(mi.T_K_NORM, li, np.float32)
        kv_t = np.int8 if d.kv_int8 else np.uint16
        self.kv_k = eng.to_host(mi.T_KV_K, 0, kv_t).copy()
        self.kv_v = eng.to_host(mi.T_KV_V, 0, kv_t).copy()
        if d.kv_int8:
            self.kv_ks = eng.to_host(mi.T_KV_KS, 0, np.uint16).copy()
            self.kv_vs = eng.to_host(mi.T_KV_VS, 0, np.uint16).copy()
        sh = O.attn_shape(QH, KVH, HD, rot_dim=d.rot_dim, eps=d.rms_eps)
        self.lm = (h(mi.T_LM_Q, 0, np.uint32), h(mi.T_LM_S, 0, np.uint16), H, d.vocab, S[4])
        self.model = O.DenseModel(d.layers, H, I, d.vocab, d.vocab_used, d.max_len, sh, d.rms_eps,
                                  C.cast(layers, C.c_void_p), h(mi.T_EMBED, 0, np.uint16),
                                  h(mi.T_FINAL_NORM, 0, np.float32),
                                  O.Linear(*self.lm),
                                  h(mi.T_ROPE, 0, np.float32), d.attn_tgt, H // 64)
        if moe:
            m = self.model
            m.experts, m.top_k, m.moe_inter = d.experts, d.top_k, d.moe_inter
            m.router_n, m.router_ksplit = (d.experts + 1 + 15) // 16 * 16, 16

    def step(self, tok, pos, layers=None, threads=None):
        """One decode step over the first `layers` layers (all by default) and the head.
        Returns (seconds, logits, argmax, threads used). The KV copies are the step's inputs
        (a step writes row `pos` into them, the same values on every call)."""
        O, d = self.O, self.d
        nl = d.layers if layers is None else layers
        full = O.lib().orc_threads()
        if threads:
            O.lib().orc_set_threads(threads)
        used = O.lib().orc_threads()
        logits = np.zeros(d.vocab, np.float32)
        t0 = time.perf_counter()
        if d.kv_int8:
            am = O.lib().orc_dense_step_kv8(O.ORC_F16, C.byref(self.model), tok, pos, O._p(self.kv_k),
                                            O._p(self.kv_v), O._p(self.kv_ks), O._p(self.kv_vs), O._p(logits), nl)
        else:
            am = O.lib().orc_dense_step(O.ORC_F16, C.byref(self.model), tok, pos, O._p(self.kv_k), O._p(self.kv_v),
                                        O._p(logits), nl)
        dt = time.perf_counter() - t0
        if threads:
            O.lib().orc_set_threads(full)
        return dt, logits, int(am), int(used)


    def head(self, threads=None):
        """Seconds of the step's head alone (the lm_head GEMV in the twin order over a unit x)."""
        O = self.O
        q, sc, K, N, S = self.lm
        xf = np.ones(K, np.float32)
        out = np.zeros(N, np.float32)
        full = O.lib().orc_threads()
        if threads:
            O.lib().orc_set_threads(threads)
        t0 = time.perf_counter()
        O.lib().orc_gemv_twin(0, q, sc, K, N, O._p(xf), 1, S, O._p(out))
        dt = time.perf_counter() - t0
        if threads:
            O.lib().orc_set_threads(full)
        return dt


def cpu_oracle_step(eng, tok, pos):
    """One full decode step of the same model through the CPU oracle on every host thread.
    Returns (seconds, logits, argmax, threads)."""
    return CpuOracle(eng).step(tok, pos)


def cpu_model():
    """The host CPU's model string and the threads this process may run on."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count()
    return name, avail, os.cpu_count()


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--attn-tgt", type=int, default=None,
                    help="attention blocks per kv head (the v2 grid's TGT); default: the model description's")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline and parity step")
    ap.add_argument("--no-other", action="store_true",
                    help="skip the secondary measurements of BASELINE configs 1, 3, 4 and 5")
    ap.add_argument("--eager", action="store_true",
                    help="enqueue each step kernel by kernel instead of replaying the captured graph "
                         "(no capture, no CPU step); with --steps 0 only the GEMV roofline sweep and "
                         "the stream-read probe run, which is the command the kernel profiles use")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="reduce two rocprofv3 --pmc output folders of `--only roofline` (FETCH_SIZE, WRITE_SIZE) "
                         "into profiles/gemv_w4a16_27b_*traffic.json")
    ap.add_argument("--only", choices=["cfg1", "cfg3", "cfg4", "cfg5", "prefill", "moe_prefill", "roofline",
                                       "lm8", "mtp"],
                    default=None,
                    help="run only that secondary measurement and print its JSON (the command the "
                         "attention and single-GEMV kernel profiles use)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (no sharding, no collectives); "
              "use --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.only == "prefill":
        eng = mi.Engine(mi.desc_27b(max_len=2112), seed=args.seed)
        print(json.dumps({"prefill": measure_prefill(eng)}), flush=True)
        eng.close()
        return
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.only == "roofline":
        # the GEMV roofline's launches alone (the command the GEMV kernel profiles use): the
        # step's fused launches per linear, then the plain sweep
        eng = mi.Engine(mi.desc_27b(max_len=((args.context + 64 + 1 + 63) // 64) * 64), seed=args.seed)
        eng.reset(args.context, 1000)
        roof, _ = step_gemv_roofline(eng)
        plain, _ = gemv_roofline(eng)
        eng.close()
        # the calibration kernels of the PMC passes: a 2 GiB fill and 2 GiB stream reads
        stream = stream_read_rate(None)
        print(json.dumps({"roofline": roof, "plain_sweep": plain, "stream_read_gbs": round(stream, 1)}), flush=True)
        return
    if args.only == "cfg4" and args.eager:
        # the configs[3] MoE decode step enqueued kernel by kernel (the MoE kernel profiles'
        # command): `--steps` steps at context `--context`
        eng = mi.Engine(mi.desc_moe_cfg4(max_len=((args.context + 64 + 1 + 63) // 64) * 64), seed=args.seed + 1)
        eng.reset(args.context, 1000)
        for _ in range(max(args.steps, 1)):
            eng.step_eager(1)
        mi.check(mi.lib().mi_device_sync())
        assert eng.ctrl()[mi.CTRL_DEBUG] == 0
        eng.close()
        print(json.dumps({"cfg4_eager_steps": args.steps}), flush=True)
        return
    if args.only == "cfg4":
        print(json.dumps({"cfg4_moe_step": measure_cfg4(args)}), flush=True)
        return
    if args.only == "lm8":
        print(json.dumps({"lm_head_int8": measure_lm_head_int8(None)}), flush=True)
        return
    if args.only == "mtp":
        print(json.dumps({"mtp": measure_mtp(args), "mtp_w16": measure_mtp(args, w16=True),
                          "mtp_moe": measure_mtp(args, moe=True)}), flush=True)
        return
    if args.only == "moe_prefill":
        # the configs[3] MoE model's chunked prefill of a 2048-token prompt, three timed calls
        eng = mi.Engine(mi.desc_moe_cfg4(max_len=2112), seed=args.seed + 1)
        ms = [time_prefill(eng, 2048)[0] for _ in range(3)]
        eng.close()
        print(json.dumps({"moe_prefill": {"workload": "configs[3] MoE model, prefill of a 2048-token prompt in one "
                                          "chunk (synthetic ids, random-init weights)",
                                          "ms": [round(m, 2) for m in ms],
                                          "tokens_per_s": round(2048 / min(ms) * 1e3, 1)}}), flush=True)
        return
    if args.only:
        fn = {"cfg1": lambda: measure_cfg1(None),
              "cfg3": lambda: [measure_cfg3(None, L, args.attn_tgt or 64) for L in (32768, 131072)],
              "cfg5": lambda: measure_cfg5(None)}[args.only]
        print(json.dumps({args.only: fn()}), flush=True)
        return

    max_len = ((args.context + args.warmup + args.steps + 1 + 63) // 64) * 64
    desc = mi.desc_27b(max_len=max_len)
    if args.attn_tgt:
        desc.attn_tgt = args.attn_tgt
    log(f"bench: building 27B-shape engine (max_len {max_len}) ...")
    t0 = time.time()
    eng = mi.Engine(desc, seed=args.seed)
    if not args.eager:
        eng.capture(1)
    log(f"bench: engine ready in {time.time() - t0:.1f} s; S per linear {[eng.linear_s(w) for w in range(5)]}")
    st = eng.stream
    tok0 = 1000

    parity = None
    cpu = None
    if not args.no_cpu and not args.eager:
        log("bench: CPU oracle step (one full 64-layer step on the host) ...")
        eng.reset(args.context, tok0)
        orc = CpuOracle(eng)
        dt, cpu_logits, cpu_am, threads = orc.step(tok0, args.context)
        # BASELINE.md's timing plan (median of >= 5 repetitions after a warm-up, which the full
        # step above is) on a bounded sample: the step's first 4 and first 8 layers (a partial
        # walk stops before the head) and the head alone, five times each; the layers cost the
        # same, so per layer = (t8 - t4) / 4 and the step = t4 + (layers - 4) per layer + the
        # head. 1 core: the same over 1 and 2 layers and the head, three times each.
        def med(fn, reps):
            return float(np.median([fn() for _ in range(reps)]))
        t4 = med(lambda: orc.step(tok0, args.context, layers=4)[0], 5)
        t8 = med(lambda: orc.step(tok0, args.context, layers=8)[0], 5)
        th = med(lambda: orc.head(), 5)
        per_layer_all = max(t8 - t4, 0.0) / 4
        step_all = t4 + (desc.layers - 4) * per_layer_all + th
        t1 = med(lambda: orc.step(tok0, args.context, layers=1, threads=1)[0], 3)
        t2 = med(lambda: orc.step(tok0, args.context, layers=2, threads=1)[0], 3)
        th1 = med(lambda: orc.head(threads=1), 3)
        per_layer = max(t2 - t1, 0.0)
        one_core_step = t1 + (desc.layers - 1) * per_layer + th1
        del orc
        eng.reset(args.context, tok0)
        gpu_tok = int(eng.generate(1)[0])
        g = eng.logits(1)[0].astype(np.float64)
        w = cpu_logits.astype(np.float64)
        err = np.abs(g - w)
        parity = {
            "max_abs_err": float(err.max()),
            "max_err_over_max_logit": float(err.max() / np.abs(w).max()),
            "within_rel_2e-3": bool(np.all(err <= 2e-3 * np.abs(w) + 2e-3 * np.abs(w).max())),
            "argmax_gpu": gpu_tok, "argmax_oracle": cpu_am,
        }
        cpu_name, cpu_avail, cpu_all = cpu_model()
        cpu = {"value": round(1.0 / step_all, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
               "sample": f"the decode step of the same 64-layer model at context {args.context} (oracle/oracle.cpp "
                         f"orc_dense_step, twin GEMV order, {threads} OpenMP threads): medians of 5 runs over the "
                         f"first 4 layers ({t4:.3f} s), the first 8 ({t8:.3f} s) and the head ({th:.3f} s), per "
                         f"layer {per_layer_all:.3f} s, so {step_all:.2f} s per step; the full 64-layer step of "
                         f"the parity check (the warm-up) took {dt:.2f} s",
               "full_step_s": round(dt, 3),
               "cpu_model": cpu_name, "threads_available": cpu_avail, "nproc": cpu_all,
               "one_core": {"value": round(1.0 / one_core_step, 5), "unit": "tokens/s", "cores": 1,
                            "sample": f"1 thread: medians of 3 runs over the first layer ({t1:.2f} s), the first 2 "
                                      f"({t2:.2f} s) and the head ({th1:.2f} s); per layer {per_layer:.2f} s, so the "
                                      f"64-layer step is {one_core_step:.1f} s (a full single-thread step is not run: "
                                      f"it would hold the GPU box for minutes)"}}
        log(f"bench: cpu step {dt:.2f} s on {threads} threads; parity {parity}")

    eng.reset(args.context, tok0)
    step = eng.step_eager if args.eager else eng.replay
    ms_per_step = tok_s = None
    if args.steps > 0:
        for _ in range(args.warmup):
            step(1)
        mi.check(mi.lib().mi_device_sync())
        ev = Events(st)
        tw = time.perf_counter()
        ev.start()
        for _ in range(args.steps):
            step(1)
        ms = ev.stop_ms()
        mi.check(mi.lib().mi_device_sync())
        wall = time.perf_counter() - tw
        ms_per_step = ms / args.steps
        c = eng.ctrl()
        assert c[mi.CTRL_POS] == args.context + args.warmup + args.steps, c[:20]
        assert c[mi.CTRL_DEBUG] == 0, hex(c[mi.CTRL_DEBUG])
        tok_s = 1000.0 / ms_per_step
        log(f"bench: {args.steps} steps in {ms:.2f} ms (events), {wall * 1e3:.2f} ms wall -> {tok_s:.1f} tok/s")

    verify = None
    if not args.eager and not args.no_other:
        verify = measure_verify_steps(eng, args.context, tok0)
        log(f"bench: verify steps {verify}")
    roof, alg_gemv = step_gemv_roofline(eng)
    plain, _ = gemv_roofline(eng)
    roof["plain_sweep"] = {k: plain[k] for k in ("achieved", "frac", "gemv_ms_per_step", "avg_launch_us")}
    roof["plain_sweep"]["note"] = "the same GEMVs as plain partials launches (no fused epilogue)"
    stream_gbs = stream_read_rate(st)
    kv_bytes = 2 * desc.layers * desc.kv_heads * (args.context + 1) * desc.head_dim * 2
    step_alg = alg_gemv + kv_bytes
    roof["traffic"] = profiled_traffic(eng, "gemv_w4a16_27b_step_traffic.json")
    roof["plain_sweep"]["traffic"] = profiled_traffic(eng)
    roof["stream_read_gbs"] = round(stream_gbs, 1)
    roof["frac_of_stream"] = round(roof["achieved"] / stream_gbs, 4)
    log(f"bench: gemv roofline {roof}")
    prefill = None
    if not args.eager and not args.no_other:
        prefill = measure_prefill(eng)
        log(f"bench: prefill {prefill}")
    eng.close()

    other = None
    if not args.eager and not args.no_other:
        log("bench: other configurations (cfg1 GEMV, cfg3 attention, cfg5 small-M, cfg4 MoE step) ...")
        other = {"cfg1_gemv": measure_cfg1(None)}
        log(f"bench: cfg1 {other['cfg1_gemv']}")
        other["cfg3_attention_int8_paged"] = [measure_cfg3(None, L) for L in (32768, 131072)]
        log(f"bench: cfg3 {other['cfg3_attention_int8_paged']}")
        other["cfg5_small_m_gemv"] = measure_cfg5(None)
        log(f"bench: cfg5 {other['cfg5_small_m_gemv']}")
        other["prefill_27b"] = prefill
        other["verify_steps_27b"] = verify
        other["bf16_27b_step"] = measure_bf16_step(args)
        log(f"bench: bf16 {other['bf16_27b_step']}")
        other["cfg4_moe_step"] = measure_cfg4(args)
        other["cfg4_moe_step_int8_kv"] = measure_cfg4(args, kv_int8=1)
        log(f"bench: cfg4 {other['cfg4_moe_step']}")
        other["lm_head_int8"] = measure_lm_head_int8(None)
        log(f"bench: int8 lm_head {other['lm_head_int8']}")
        other["mtp"] = measure_mtp(args)
        other["mtp_w16"] = measure_mtp(args, w16=True)
        other["mtp_moe"] = measure_mtp(args, moe=True)
        log(f"bench: mtp {other['mtp']}")

    out = {
        "metric": "batch-1 decode tokens/s (27B-shape W4A16); int4 GEMV HBM GB/s vs peak",
        "value": None if tok_s is None else round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None if ms_per_step is None else round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4a16 (int4 g64 weights, f16 activations, fp32 accumulate)",
        "data": "synthetic (random-init 27B-shape weights; fp16 KV pre-filled N(0,1))",
        "config": {"workload": "BASELINE configs[1]: dense 27B-shape decode step, batch 1, context 4096",
                   "launch": "eager" if args.eager else "hipGraph replay",
                   "layers": desc.layers, "hidden": desc.hidden, "q_heads": desc.q_heads,
                   "kv_heads": desc.kv_heads, "head_dim": desc.head_dim, "intermediate": desc.inter,
                   "vocab": desc.vocab, "context": args.context, "rope_theta": 1e6,
                   "attn_blocks_per_kv_head": desc.attn_tgt},
        "step_alg_bytes": step_alg,
        "step_hbm_gbs": None if ms_per_step is None else round(step_alg / (ms_per_step * 1e-3) / 1e9, 1),
        "roofline": roof,
        "cpu_baseline": cpu,
        "parity": parity,
        "other_configs": other,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
