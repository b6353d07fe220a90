"""Benchmark: fused q8 KV-cache decode attention at an 82,671-token context on one MI355X.

    python bench.py [--gpus 1] [--steps 256] [--warmup 16]

Workload (one "step" = one decode step of one full-attention layer): quantize-on-append of one new
bf16 K row and V row (N(0,1), group 64) into the layer's uint8 cache, then fused single-token
attention of 32 query heads over the 8 KV heads of that layer at n = 82,671 + appended rows -- one
launch of lq_q8_decode_append_attn (the append happens inside the attention kernel).
Ten distinct layer caches (the real model's 10 full-attention layers, 1.8 GB) rotate step by step
so the 256 MB last-level cache cannot hold the working set. Inputs are synthetic and resident in
HBM before the timed region starts.

Prints one JSON line: value = algorithmic HBM bytes per second over the timed steps (GB/s), the
roofline of the kernel each step launches (HIP events on the launch stream around the timed
steps; with --separate-append, around groups of back-to-back attention calls after them), and the
CPU baseline (the oracle's unfused
dequantize-to-bf16 + fp32 SDPA path, timed on the host cores).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "q8 decode-attn µs/call & HBM GB/s (% of 8 TB/s) at 82,671-token ctx"
PEAK_GBS = 8000.0
# The reference's fused kernel on an M4 GPU at three contexts (results/kv_decode_micro_fused.json,
# rows.<ctx>.fused_q8_ms; 48q/8kv -- the KV bytes, 2176 B per row over 8 KV heads, do not depend on
# the q-head count, so the GB/s carry over to 32q/8kv)
REF_M4_MS = {8192: 1.1922058201162145, 32768: 3.5013833199627697, 82671: 12.243627500138246}
HQ, HKV, D, GS = 32, 8, 128, 64
Q8_ROW = 2 * (D + 2 * 2 * (D // GS))  # K+V codes + bf16 scale/bias per token per KV head = 272
Q8_TOKEN = HKV * Q8_ROW               # 2176 B per token over 8 KV heads


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=256)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--ctx", type=int, default=82671)
    p.add_argument("--layers", type=int, default=10)
    p.add_argument("--roofline-calls", type=int, default=128,
                   help="plain attention calls timed in groups of 8 after the timed steps "
                        "(attn_us_per_call; the roofline with --separate-append)")
    p.add_argument("--settle-ms", type=float, default=500.0,
                   help="before the warm-up, run back-to-back attention calls over the rotating "
                        "caches for this long (GPU time, outside the timed region) so that a run "
                        "on a just-acquired GPU is timed at its settled clocks; 0 disables it")
    p.add_argument("--hot-calls", type=int, default=64,
                   help="after the timed region, plain attention calls on one layer's cache back to "
                        "back (single_cache: the reference micro-benchmark's way of timing; the "
                        "cache stays in the last-level cache), reported apart; 0 skips them")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU baseline sample: calls are repeated until this much time has passed")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--separate-append", action="store_true",
                   help="append with its own launch (lq_quantize_append_kv) before lq_decode_attn "
                        "instead of the fused step (lq_q8_decode_append_attn)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB 8 times (HBM counter calibration)")
    p.add_argument("--q-heads", type=int, default=32,
                   help="query heads over the 8 KV heads (decode, verify, q4, bf16, ragged): 32 is the "
                        "benchmarked 32q/8kv shape, 48 Laguna's own 48q/8kv (the dense kernel and a "
                        "merge launch for the 8-bit cache)")
    p.add_argument("--workload", default="decode",
                   choices=["decode", "q4", "bf16", "ragged", "verify", "lookup", "layers",
                            "prefill", "quantize"],
                   help="decode: the 8-bit decode step (default). q4 / bf16: decode attention over "
                        "a 4-bit / plain bf16 cache at the same context. ragged: 8 sequences of "
                        "default_rng(1) lengths in [42771, 82671]. verify: a 5-row causal verify "
                        "block over 65,536 cached rows plus its append. lookup: n-gram draft search "
                        "over 82,671 ids and greedy accept of 5 x 131,072 logits. layers: one decoded "
                        "token through the attention blocks of --layers full-attention layers. "
                        "prefill: a 2,048-row chunk appended and attended at --ctx rows. "
                        "quantize: bulk quantize-append of --ctx K and V rows (8 heads, one launch)")
    return p.parse_args()


def cpu_threads():
    """(worker threads, host cores) of the CPU baselines: every core this process may run on,
    capped at the OMP_NUM_THREADS share when that is set (the per-GPU CPU share of a box)."""
    host = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS", "")
    return (max(1, min(host, int(share))) if share.isdigit() else host), host


def cpu_attention(pool, q, k, v, n, scale, bits=8, causal=False, chunk=4096):
    """The reference's unfused path (dequantize to bf16, fp32 SDPA) on the host cores: one task
    per (KV head, chunk of keys) on ``pool`` -- the chunk dequantized by the oracle (bf16-rounded
    ``scale * code + bias``), fp32 scores and weights with BLAS, the chunk's (max, sum, weighted V)
    -- then the log-sum-exp merge per head. q fp32 [Hq, L, D]; k, v (codes [Hkv, cap, .], scale
    and bias bf16 bits [Hkv, cap, D / 64]) or fp32 [Hkv, cap, D] values (``bits`` None); causal:
    query row i at position n - L + i. Returns fp32 [Hq, L, D]."""
    import numpy as np

    from oracle import quantize as Q

    Hq, L, _ = q.shape
    Hkv = (k[0] if isinstance(k, tuple) else k).shape[0]
    G = Hq // Hkv
    row = n - L + np.arange(G * L) % L

    def task(t):
        h, a = t
        e = min(a + chunk, n)
        if bits is None:
            kk, vv = k[h, a:e], v[h, a:e]
        else:
            kk = Q.dequantize(k[0][h, a:e], k[1][h, a:e], k[2][h, a:e], GS, bits)
            vv = Q.dequantize(v[0][h, a:e], v[1][h, a:e], v[2][h, a:e], GS, bits)
        s = (q[h * G:(h + 1) * G].reshape(G * L, D) @ kk.T) * np.float32(scale)
        if causal and L > 1:
            s = np.where(np.arange(a, e)[None, :] <= row[:, None], s, np.float32(-np.inf))
        m = s.max(axis=-1)
        ms = np.where(np.isfinite(m), m, np.float32(0))
        p = np.exp(s - ms[:, None])
        return h, m, p.sum(axis=-1), p @ vv

    parts = list(pool.map(task, [(h, a) for h in range(Hkv) for a in range(0, n, chunk)]))
    out = np.empty((Hq, L, D), np.float32)
    for h in range(Hkv):
        mine = [x for x in parts if x[0] == h]
        m = np.stack([x[1] for x in mine])
        M = m.max(axis=0)
        w = np.where(np.isfinite(m), np.exp(m - M), 0).astype(np.float32)
        den = (w * np.stack([x[2] for x in mine])).sum(axis=0)
        acc = (w[..., None] * np.stack([x[3] for x in mine])).sum(axis=0)
        out[h * G:(h + 1) * G] = (acc / den[:, None]).reshape(G, L, D)
    return out


def time_cpu_attention(q, k, v, n, scale, seconds, bits=8, causal=False, min_calls=3):
    """Median wall time of :func:`cpu_attention` on all worker threads (one BLAS thread each),
    after one warm-up, repeated for about ``seconds``; returns (seconds per call, calls, threads,
    host cores)."""
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    threads, host = cpu_threads()
    with threadpool_limits(limits=1), ThreadPoolExecutor(threads) as pool:
        t, calls = _time_cpu(lambda: cpu_attention(pool, q, k, v, n, scale, bits, causal),
                             seconds, min_calls)
    return t, calls, threads, host


def cpu_baseline(kc, ks, kb, vc, vs, vb, q, n, seconds):
    """The reference's unfused path restated by the oracle, on all host cores
    (:func:`cpu_attention`): one decode step's attention over one layer at n keys."""
    t, calls, threads, host = time_cpu_attention(q.reshape(HQ, 1, D), (kc, ks, kb), (vc, vs, vb),
                                                 n, D ** -0.5, seconds)
    return {
        "value": round(Q8_TOKEN * n / t / 1e9, 3), "unit": "GB/s", "cores": threads,
        "host_cores": host, "blas_threads": 1, "kind": "port", "us_per_call": round(t * 1e6, 1),
        "sample": (f"median of {calls} calls (after 1 warm-up) of the unfused dequantize-to-bf16 + "
                   f"fp32 SDPA path at n={n} on one layer: (KV head, 4,096-key chunk) tasks on "
                   f"{threads} worker threads with one BLAS thread each ({host} host cores); "
                   f"CPU: {_cpu_model()}"),
    }


def copy_calibration(mib):
    """A plain device-to-device copy of `mib` MiB, 8 times: under rocprofv3 --pmc FETCH_SIZE (or
    WRITE_SIZE) it gives the counter's reading for a known number of HBM bytes, the factor that
    turns the counters read on the attention kernel into bytes."""
    import torch

    dev = torch.device("cuda", 0)
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    for _ in range(8):
        flush.fill_(0)  # evicts src/dst from the last-level cache between copies
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "copies": 8}), flush=True)


# ------------------------------------------------------------------------------------------------
# the other configurations: same JSON contract, one line each
# ------------------------------------------------------------------------------------------------

def _cpu_model():
    try:
        return [l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                if l.startswith("model name")][0]
    except Exception:
        return "unknown"


def _time_cpu(fn, seconds, min_calls=3):
    """Median wall time of fn() after one warm-up, repeated for about `seconds`."""
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_calls or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], len(times)


def _gpu_groups(stream, calls, group, fn):
    """Per-call ms of `calls` back-to-back fn(j) launches, one event pair per group of `group`."""
    import torch
    pairs = []
    for gi in range(max(1, calls // group)):
        e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        e[0].record(stream)
        for k in range(group):
            fn(gi * group + k)
        e[1].record(stream)
        pairs.append(e)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) / group for a, b in pairs]


def settle(stream, ms, fn, group=256):
    """Runs fn(j) back to back in groups of `group` launches until their GPU time (events on the
    launch stream) adds up to `ms`. A GPU that has just been acquired runs its first milliseconds
    of work below its settled clocks; this phase sits before the warm-up, outside the timed
    region. Returns what it did, for the JSON line."""
    import torch
    if ms <= 0:
        return {"ms": 0.0, "calls": 0}
    done, calls, t0 = 0.0, 0, time.perf_counter()
    while done < ms:
        e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        e[0].record(stream)
        for k in range(group):
            fn(calls + k)
        e[1].record(stream)
        e[1].synchronize()
        done += e[0].elapsed_time(e[1])
        calls += group
    return {"ms": round(done, 1), "calls": calls,
            "wall_ms": round((time.perf_counter() - t0) * 1e3, 1)}


def _result(metric, value, unit, hib, ms, args, dtype, config, extra):
    res = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": hib,
           "scaling": "weak", "vs_baseline": None, "dtype": dtype,
           "data": "synthetic (N(0,1) bf16 inputs; integer ids uniform)", "config": config}
    res.update(extra)
    print(json.dumps(res), flush=True)


def run_workload(args):
    import numpy as np
    import torch

    from lagunalab_amd import _lib

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    g = torch.Generator(device=dev).manual_seed(0)
    rng = np.random.default_rng(0)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)  # attention workspace, counters at 0
    scale = D ** -0.5
    do_cpu = not args.no_cpu_baseline and args.cpu_seconds > 0

    if args.workload in ("q4", "bf16"):
        # decode attention over 10 rotating layer caches (4-bit: 1152 B/token, bf16: 4096 B/token)
        n, nl = args.ctx, args.layers
        cap = (n + 255) // 256 * 256
        layers = []
        for _ in range(nl):
            lay = []
            for _kv in range(2):
                x = torch.randn((1, HKV, cap, D), device=dev, generator=g).to(torch.bfloat16)
                if args.workload == "bf16":
                    lay.append((x,))
                    continue
                codes = torch.empty((1, HKV, cap, D // 2), dtype=torch.uint8, device=dev)
                sc = torch.empty((1, HKV, cap, 2), dtype=torch.bfloat16, device=dev)
                bi = torch.empty_like(sc)
                _lib.check(lib.lq_quantize_append(x.data_ptr(), 1, HKV, cap, D, codes.data_ptr(),
                                                  sc.data_ptr(), bi.data_ptr(), cap, 0, 4, GS, sp),
                           "prefill quantize")
                del x
                lay.append((codes, sc, bi))
            layers.append(lay)
        qs = torch.randn((64, 1, HQ, 1, D), device=dev, generator=g).to(torch.bfloat16)
        out = torch.empty((1, HQ, 1, D), dtype=torch.bfloat16, device=dev)
        kind = _lib.LQ_KV_BF16 if args.workload == "bf16" else _lib.LQ_KV_Q4
        per_tok = HKV * (2 * D * 2 if kind == _lib.LQ_KV_BF16 else 2 * (D // 2 + 2 * 2 * (D // GS)))
        ptr = lambda t, i: t[i].data_ptr() if len(t) > i else None

        def call(j):
            (k, v) = layers[j % nl]
            st = lib.lq_decode_attn(kind, qs[j % 64].data_ptr(), k[0].data_ptr(), ptr(k, 1),
                                    ptr(k, 2), v[0].data_ptr(), ptr(v, 1), ptr(v, 2), 1, HQ, HKV,
                                    D, cap, n, None, scale, out.data_ptr(), ws.data_ptr(),
                                    ws.numel(), sp)
            if st:
                _lib.check(st, "lq_decode_attn")
        for j in range(args.warmup):
            call(j)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for j in range(args.steps):
            call(j)
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
        nbytes = per_tok * n + 2 * HQ * D * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        name = "4-bit" if kind == _lib.LQ_KV_Q4 else "plain bf16"
        extra = {"us_per_call": round(ms * 1e3, 2), "pct_of_hbm_peak": round(100 * gbs / PEAK_GBS, 2),
                 "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4), "traffic": None,
                              "kernel": f"lq_decode_attn ({name})", "bytes_per_call": nbytes}}
        if do_cpu:
            cv = lambda t: (t.cpu().numpy() if t.dtype == torch.uint8
                            else t.cpu().view(torch.int16).numpy().view(np.uint16))
            qn = qs[0, 0].float().cpu().numpy()  # [HQ, 1, D]
            if kind == _lib.LQ_KV_Q4:
                kh = tuple(cv(t)[0] for t in layers[0][0])
                vh = tuple(cv(t)[0] for t in layers[0][1])
                t, calls, threads, host = time_cpu_attention(qn, kh, vh, n, scale, args.cpu_seconds,
                                                             bits=4)
            else:
                kf = layers[0][0][0][0].float().cpu().numpy()
                vf = layers[0][1][0][0].float().cpu().numpy()
                t, calls, threads, host = time_cpu_attention(qn, kf, vf, n, scale, args.cpu_seconds,
                                                             bits=None)
            extra["cpu_baseline"] = {
                "value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads,
                "host_cores": host, "blas_threads": 1, "kind": "port",
                "us_per_call": round(t * 1e6, 1),
                "sample": f"median of {calls} calls of the oracle's "
                          f"{'dequantize + ' if kind == _lib.LQ_KV_Q4 else ''}fp32 SDPA at n={n}, "
                          f"one layer, (KV head, key chunk) tasks on {threads} threads; "
                          f"CPU: {_cpu_model()}"}
        _result(f"{name} decode-attn GB/s at {n}-token ctx", round(gbs, 2), "GB/s", True, ms, args,
                "u4" if kind == _lib.LQ_KV_Q4 else "bf16",
                {"workload": f"{name} KV decode attention, batch 1, {HQ}q/{HKV}kv heads, head_dim {D}, "
                             f"context {n}, {nl} rotating layer caches", "ctx": n, "layers": nl}, extra)
        return

    if args.workload == "ragged":
        lens = [int(x) for x in np.random.default_rng(1).integers(42771, 82672, size=8)]
        B, cap, nl = len(lens), 82944, 3
        layers = []
        for _ in range(nl):
            lay = []
            for _kv in range(2):
                codes = torch.randint(0, 256, (B, HKV, cap, D), dtype=torch.uint8, device=dev, generator=g)
                sc = (torch.rand((B, HKV, cap, 2), device=dev, generator=g) * 0.03).to(torch.bfloat16)
                bi = (torch.rand((B, HKV, cap, 2), device=dev, generator=g) * -3).to(torch.bfloat16)
                lay.append((codes, sc, bi))
            layers.append(lay)
        q = torch.randn((B, HQ, 1, D), device=dev, generator=g).to(torch.bfloat16)
        out = torch.empty((B, HQ, 1, D), dtype=torch.bfloat16, device=dev)
        import ctypes as C
        lens_arr = C.cast((C.c_int32 * B)(*lens), C.c_void_p)

        def call(j):
            (kc, ks, kb), (vc, vs, vb) = layers[j % nl]
            st = lib.lq_decode_attn(8, q.data_ptr(), kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
                                    vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), B, HQ, HKV, D,
                                    cap, 0, lens_arr, scale, out.data_ptr(), ws.data_ptr(),
                                    ws.numel(), sp)
            if st:
                _lib.check(st, "lq_decode_attn (ragged)")
        for j in range(args.warmup):
            call(j)
        torch.cuda.synchronize()
        per = _gpu_groups(stream, args.steps, 8, call)
        ms = sum(per) / len(per)
        nbytes = Q8_TOKEN * sum(lens) + 2 * B * HQ * D * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        extra = {"us_per_call": round(ms * 1e3, 2), "lens": lens,
                 "pct_of_hbm_peak": round(100 * gbs / PEAK_GBS, 2),
                 "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4), "traffic": None,
                              "kernel": "lq_decode_attn (8-bit, variable-length splits)",
                              "bytes_per_call": nbytes}}
        if do_cpu:  # one call per sequence, as the reference would have to run them
            cv = lambda t: t.numpy() if t.dtype == torch.uint8 else t.view(torch.int16).numpy().view(np.uint16)
            b0 = 4  # the shortest sequence keeps the sample bounded
            kh = tuple(cv(t[b0].cpu()) for t in layers[0][0])
            vh = tuple(cv(t[b0].cpu()) for t in layers[0][1])
            qn = q[b0].float().cpu().numpy()  # [HQ, 1, D]
            t, calls, threads, host = time_cpu_attention(qn, kh, vh, lens[b0], scale,
                                                         args.cpu_seconds, min_calls=2)
            extra["cpu_baseline"] = {
                "value": round(Q8_TOKEN * lens[b0] / t / 1e9, 3), "unit": "GB/s", "cores": threads,
                "host_cores": host, "blas_threads": 1, "kind": "port",
                "us_per_call": round(t * 1e6, 1),
                "sample": f"median of {calls} calls (dequantize + fp32 SDPA, {threads} threads) for "
                          f"one sequence of {lens[b0]} tokens (the reference runs one call per "
                          f"sequence); CPU: {_cpu_model()}"}
        _result("q8 ragged decode-attn GB/s, 8 sequences of 42,771-82,671 tokens", round(gbs, 2),
                "GB/s", True, ms, args, "u8",
                {"workload": f"ragged 8-bit decode attention, 8 sequences (sum {sum(lens)} tokens), "
                             f"{HQ}q/{HKV}kv heads, head_dim {D}, {nl} rotating caches",
                 "batch": B, "layers": nl}, extra)
        return

    if args.workload == "prefill":
        # A 2,048-row prefill chunk at the end of an 82,671-row context: quantize-append of its
        # K/V (rows 80,623 .. 82,670), then causal attention of its 32 x 2,048 query rows straight
        # off the 8-bit cache (q8_prefill_attention -> lq_q8_prefill_attn: no score matrix, no
        # dequantized copy). 4 rotating layer caches.
        from lagunalab_amd.q8_attn import q8_prefill_attention
        n, L, nl = args.ctx, 2048, 4
        if n < L:
            raise SystemExit(f"--ctx {n} must cover the {L}-row chunk")
        nc = n - L
        cap = (n + 255) // 256 * 256
        layers = []
        for _ in range(nl):
            lay = []
            for _kv in range(2):
                codes = torch.zeros((1, HKV, cap, D), dtype=torch.uint8, device=dev)
                sc = torch.zeros((1, HKV, cap, 2), dtype=torch.bfloat16, device=dev)
                bi = torch.zeros_like(sc)
                if nc:
                    x = torch.randn((1, HKV, nc, D), device=dev, generator=g).to(torch.bfloat16)
                    _lib.check(lib.lq_quantize_append(x.data_ptr(), 1, HKV, nc, D, codes.data_ptr(),
                                                      sc.data_ptr(), bi.data_ptr(), cap, 0, 8, GS,
                                                      sp), "prefill quantize")
                    del x
                lay.append((codes, sc, bi))
            layers.append(lay)
        qv = torch.randn((1, HQ, L, D), device=dev, generator=g).to(torch.bfloat16)
        kn = torch.randn((1, HKV, L, D), device=dev, generator=g).to(torch.bfloat16)
        vn = torch.randn((1, HKV, L, D), device=dev, generator=g).to(torch.bfloat16)

        def call(j):
            (kc, ks, kb), (vc, vs, vb) = layers[j % nl]
            _lib.check(lib.lq_quantize_append_kv(kn.data_ptr(), vn.data_ptr(), 1, HKV, L, D,
                                                 kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
                                                 vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), cap,
                                                 nc, 8, GS, sp), "chunk append")
            q8_prefill_attention(qv, layers[j % nl][0], layers[j % nl][1], n, scale)
        steps = max(1, min(args.steps, 32))
        for j in range(min(args.warmup, 4)):
            call(j)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for j in range(steps):
            call(j)
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / steps
        keys = L * nc + L * (L + 1) // 2  # keys seen, summed over the chunk's rows
        flops = 4 * D * HQ * keys
        tf = flops / (ms * 1e-3) / 1e12
        extra = {"ms_per_chunk": round(ms, 3), "timed_chunks": steps,
                 "rows_per_s": round(L / (ms * 1e-3), 1),
                 "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": 2500.0,
                              "unit": "TFLOP/s", "frac": round(tf / 2500.0, 4), "traffic": None,
                              "kernel": "lq_quantize_append_kv + q8_prefill_kernel "
                                        "(lq_q8_prefill_attn) per chunk",
                              "flops_per_chunk": flops}}
        if do_cpu:
            from oracle import attention as A
            cv = lambda t: t.cpu().numpy() if t.dtype == torch.uint8 else t.cpu().view(torch.int16).numpy().view(np.uint16)
            kh = tuple(cv(t) for t in layers[(steps - 1) % nl][0])
            vh = tuple(cv(t) for t in layers[(steps - 1) % nl][1])
            ns = 4  # the chunk's last rows: keys n-4 .. n-1 seen
            qn = qv[:, :, L - ns:].float().cpu().numpy()
            fn = lambda: A.unfused_attention(qn, kh, vh, n, scale, causal=True)
            t, calls = _time_cpu(fn, args.cpu_seconds, min_calls=2)
            fl = 4 * D * HQ * sum(n - ns + i + 1 for i in range(ns))
            extra["cpu_baseline"] = {
                "value": round(fl / t / 1e12, 5), "unit": "TFLOP/s", "cores": 1, "kind": "port",
                "sample": f"median of {calls} oracle calls (dequantize + causal fp64 SDPA) for the "
                          f"chunk's last {ns} rows over {n} keys; CPU: {_cpu_model()}"}
        args.steps, args.warmup = steps, min(args.warmup, 4)
        _result(f"q8 prefill attention TFLOP/s, {L}-row chunk at {n} keys", round(tf, 2),
                "TFLOP/s", True, ms, args, "u8",
                {"workload": f"append a {L}-row chunk + its causal attention over {n} rows, "
                             f"{HQ}q/{HKV}kv heads, head_dim {D}, 8-bit cache, {nl} rotating caches",
                 "q_len": L, "ctx": n, "layers": nl}, extra)
        return

    if args.workload == "verify":
        nc, L, nl = 65536, 5, 10
        cap = nc + 256
        layers = []
        for _ in range(nl):
            lay = []
            for _kv in range(2):
                x = torch.randn((1, HKV, nc, D), device=dev, generator=g).to(torch.bfloat16)
                codes = torch.zeros((1, HKV, cap, D), dtype=torch.uint8, device=dev)
                sc = torch.zeros((1, HKV, cap, 2), dtype=torch.bfloat16, device=dev)
                bi = torch.zeros_like(sc)
                _lib.check(lib.lq_quantize_append(x.data_ptr(), 1, HKV, nc, D, codes.data_ptr(),
                                                  sc.data_ptr(), bi.data_ptr(), cap, 0, 8, GS, sp),
                           "prefill quantize")
                del x
                lay.append((codes, sc, bi))
            layers.append(lay)
        qv = torch.randn((1, HQ, L, D), device=dev, generator=g).to(torch.bfloat16)
        kn = torch.randn((1, HKV, L, D), device=dev, generator=g).to(torch.bfloat16)
        vn = torch.randn((1, HKV, L, D), device=dev, generator=g).to(torch.bfloat16)
        out = torch.empty((1, HQ, L, D), dtype=torch.bfloat16, device=dev)

        def call(j):  # one fused verify step: append the 5 block rows at 65,536, then verify
            (kc, ks, kb), (vc, vs, vb) = layers[j % nl]
            if args.separate_append:
                st = lib.lq_quantize_append_kv(kn.data_ptr(), vn.data_ptr(), 1, HKV, L, D,
                                               kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
                                               vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), cap, nc,
                                               8, GS, sp)
                st |= lib.lq_q8_verify_attn(qv.data_ptr(), kc.data_ptr(), ks.data_ptr(),
                                            kb.data_ptr(), vc.data_ptr(), vs.data_ptr(), vb.data_ptr(),
                                            1, HQ, HKV, L, D, cap, nc + L, scale, out.data_ptr(),
                                            ws.data_ptr(), ws.numel(), sp)
            else:
                st = lib.lq_q8_verify_append_attn(qv.data_ptr(), kn.data_ptr(), vn.data_ptr(),
                                                  kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
                                                  vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), 1, HQ,
                                                  HKV, L, D, cap, nc, scale, out.data_ptr(),
                                                  ws.data_ptr(), ws.numel(), sp)
            if st:
                _lib.check(st, "verify step")
        for j in range(args.warmup):
            call(j)
        torch.cuda.synchronize()
        per = _gpu_groups(stream, args.steps, 8, call)
        ms = sum(per) / len(per)
        nbytes = Q8_TOKEN * (nc + L) + 2 * HQ * L * D * 2 + 2 * HKV * L * D * 2
        gbs = nbytes / (ms * 1e-3) / 1e9
        flops = 4 * (HQ // HKV) * L * D * HKV * (nc + L)
        extra = {"us_per_call": round(ms * 1e3, 2), "pct_of_hbm_peak": round(100 * gbs / PEAK_GBS, 2),
                 "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                 "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4), "traffic": None,
                              "kernel": ("lq_quantize_append_kv + lq_q8_verify_attn"
                                         if args.separate_append else
                                         "lq_q8_verify_append_attn") + " (causal, L=5)",
                              "bytes_per_call": nbytes}}
        if do_cpu:
            cv = lambda t: t.cpu().numpy() if t.dtype == torch.uint8 else t.cpu().view(torch.int16).numpy().view(np.uint16)
            kh = tuple(cv(t)[0] for t in layers[0][0])
            vh = tuple(cv(t)[0] for t in layers[0][1])
            qn = qv[0].float().cpu().numpy()  # [HQ, L, D]
            t, calls, threads, host = time_cpu_attention(qn, kh, vh, nc + L, scale,
                                                         args.cpu_seconds, causal=True,
                                                         min_calls=2)
            extra["cpu_baseline"] = {
                "value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads,
                "host_cores": host, "blas_threads": 1, "kind": "port",
                "us_per_call": round(t * 1e6, 1),
                "sample": f"median of {calls} calls (dequantize + causal fp32 SDPA, {threads} "
                          f"threads) at {nc + L} keys, L={L}; CPU: {_cpu_model()}"}
        _result("q8 verify-attn (q_len 5, causal) GB/s at 65,541 keys", round(gbs, 2), "GB/s",
                True, ms, args, "u8",
                {"workload": f"append 5 rows + causal verify attention, {HQ}q/{HKV}kv heads, "
                             f"head_dim {D}, {nc} cached rows, {nl} rotating caches",
                 "q_len": L, "ctx": nc + L, "layers": nl}, extra)
        return

    if args.workload == "layers":
        # One decoded token through the attention blocks of the model's full-attention layers
        # (laguna.py:94-111 per layer, with the layer's input RMSNorm and residual add), three
        # launches per layer: the q/k/v/gate projection with the input RMSNorm before it, the
        # fused decode step over the layer's 8-bit cache with the q/k RMSNorm + RoPE (YaRN,
        # partial rotary 0.5) in its prologue, o_proj with the softplus gate before it and the
        # residual add after.
        # Synthetic bf16 weights N(0, 0.02), caches of 82,671 quantized N(0,1) rows per layer.
        # Timed as one HIP graph replay per token (positions on the device); the eager step is
        # timed beside it.
        from lagunalab_amd.attention import Attention
        from lagunalab_amd.cache import DequantKVCache
        from lagunalab_amd.decoder import DecodeStack
        C, nl, n0 = 2048, args.layers, args.ctx
        rope = {"rope_type": "yarn", "rope_theta": 5e5, "factor": 32.0,
                "partial_rotary_factor": 0.5, "original_max_position_embeddings": 4096}
        w = lambda *sh: (0.02 * torch.randn(sh, device=dev, generator=g)).to(torch.bfloat16)
        blocks, caches, norms = [], [], []
        for _ in range(nl):
            blocks.append(Attention(w(HQ * D, C), w(HKV * D, C), w(HKV * D, C), w(C, HQ * D),
                                    w(HQ, C), 1 + w(D), 1 + w(D), HQ, HKV, rope))
            norms.append(1 + w(C))
            c = DequantKVCache(fused_decode=True)
            kx = torch.randn((1, HKV, n0, D), device=dev, generator=g).to(torch.bfloat16)
            vx = torch.randn((1, HKV, n0, D), device=dev, generator=g).to(torch.bfloat16)
            c.q.update_and_fetch(kx, vx)  # quantize the prefill rows (no dequantized copy)
            del kx, vx
            caches.append(c)
        stack = DecodeStack(blocks, norms, caches)
        n_eager = min(32, args.steps)
        xs = torch.randn((2 * args.warmup + n_eager + args.steps, 1, 1, C), device=dev,
                         generator=g).to(torch.bfloat16)
        # eager steps (host-issued launches)
        for j in range(args.warmup):
            stack.step(xs[j])
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for j in range(n_eager):
            stack.step(xs[args.warmup + j])
        t1.record(stream)
        torch.cuda.synchronize()
        eager_ms = t0.elapsed_time(t1) / n_eager
        # graph replays
        stack.capture(args.warmup + args.steps)
        base = args.warmup + n_eager
        for j in range(args.warmup):
            stack.replay(xs[base + j])
        torch.cuda.synchronize()
        t0.record(stream)
        for j in range(args.steps):
            stack.replay(xs[base + args.warmup + j])
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / args.steps
        n_mid = n0 + args.warmup + n_eager + args.warmup + args.steps // 2
        w_bytes = nl * 2 * (((HQ + 2 * HKV) * D + HQ) * C + C * HQ * D)  # q/k/v/gate + o_proj weights
        kv_bytes = nl * (Q8_TOKEN * n_mid + 2 * HKV * D * 2 + Q8_TOKEN + 2 * HQ * D * 2)
        nbytes = w_bytes + kv_bytes
        gbs = nbytes / (ms * 1e-3) / 1e9
        extra = {"us_per_token": round(ms * 1e3, 1), "tokens_per_s": round(1e3 / ms, 1),
                 "eager_us_per_token": round(eager_ms * 1e3, 1),
                 "pct_of_hbm_peak": round(100 * gbs / PEAK_GBS, 2),
                 "bytes_per_token": {"kv": kv_bytes, "weights": w_bytes},
                 "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4), "traffic": None,
                              "kernel": f"one HIP graph per token: {nl} x (lq_gemv_fused, "
                                        "lq_q8_decode_norm_append_attn, lq_gemv_fused)",
                              "bytes_per_call": nbytes}}
        _result(f"attention blocks of {nl} full-attention layers, us per decoded token at "
                f"{n0}-token ctx", round(ms * 1e3, 2), "us/token", False, ms, args, "u8",
                {"workload": f"decode token through {nl} full-attention blocks (hidden {C}, "
                             f"{HQ}q/{HKV}kv heads, head_dim {D}, YaRN RoPE 0.5, per-head gate, "
                             f"8-bit cache of {n0} rows each), one HIP graph per token",
                 "ctx": n0, "layers": nl, "hidden": C}, extra)
        return

    if args.workload == "quantize":
        # the prefill / growth path: K and V rows of all 8 heads quantized into the cache at once
        rows = args.ctx
        cap = (rows + 255) // 256 * 256
        k = torch.randn((1, HKV, rows, D), device=dev, generator=g).to(torch.bfloat16)
        v = torch.randn((1, HKV, rows, D), device=dev, generator=g).to(torch.bfloat16)

        def bufs():
            return (torch.zeros((1, HKV, cap, D), dtype=torch.uint8, device=dev),
                    torch.zeros((1, HKV, cap, D // GS), dtype=torch.bfloat16, device=dev),
                    torch.zeros((1, HKV, cap, D // GS), dtype=torch.bfloat16, device=dev))
        kq, vq = bufs(), bufs()

        def call(j):
            st = lib.lq_quantize_append_kv(k.data_ptr(), v.data_ptr(), 1, HKV, rows, D,
                                           kq[0].data_ptr(), kq[1].data_ptr(), kq[2].data_ptr(),
                                           vq[0].data_ptr(), vq[1].data_ptr(), vq[2].data_ptr(),
                                           cap, 0, 8, GS, sp)
            if st:
                _lib.check(st, "lq_quantize_append_kv")
        for j in range(args.warmup):
            call(j)
        torch.cuda.synchronize()
        per = _gpu_groups(stream, args.steps, 4, call)
        ms = sum(per) / len(per)
        vals = 2 * HKV * rows * D
        nbytes = vals * 3 + 2 * HKV * rows * (D // GS) * 4  # bf16 in, codes out, bf16 scale + bias
        gbs = nbytes / (ms * 1e-3) / 1e9
        extra = {"us_per_call": round(ms * 1e3, 2), "pct_of_hbm_peak": round(100 * gbs / PEAK_GBS, 2),
                 "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS,
                              "unit": "GB/s", "frac": round(gbs / PEAK_GBS, 4), "traffic": None,
                              "kernel": "lq_quantize_append_kv (8-bit, group 64)",
                              "bytes_per_call": nbytes}}
        if do_cpu:
            from oracle import quantize as OQ
            sample = 4096  # rows per head of K
            xs = k[0, :, :sample].float().cpu().numpy()
            t, calls = _time_cpu(lambda: OQ.quantize_packed(xs, GS, 8), min(20.0, args.cpu_seconds))
            sbytes = HKV * sample * D * 3 + HKV * sample * (D // GS) * 4
            extra["cpu_baseline"] = {
                "value": round(sbytes / t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                "us_per_call": round(t * 1e6, 1),
                "sample": f"median of {calls} calls of the NumPy quantizer on 8 heads x {sample} rows "
                          f"of K (one thread); CPU: {_cpu_model()}"}
        _result(f"bulk 8-bit quantize-append GB/s ({rows:,} K and V rows x 8 heads)", round(gbs, 2),
                "GB/s", True, ms, args, "u8",
                {"workload": f"quantize-append of {rows} K and V rows, {HKV} heads, head_dim {D}, "
                             f"group {GS}, one launch", "rows": rows}, extra)
        return

    if args.workload == "lookup":
        T, gram, nd = 82671, 3, 4
        h = rng.integers(0, 131072, size=T).astype(np.int32)
        for s0 in range(0, T - 600, 500):  # a copied 8-gram every ~500 tokens
            src = int(rng.integers(0, max(1, s0 - 8))) if s0 > 8 else 0
            h[s0:s0 + 8] = h[src:src + 8]
        h[-3:] = h[T // 2:T // 2 + 3]
        hist = torch.from_numpy(h).to(dev)
        logits = torch.randn((5, 131072), device=dev, generator=g)
        drafts = logits[:4].argmax(dim=1).to(torch.int32)  # all four drafts accepted
        nout = torch.empty(2 + nd, dtype=torch.int32, device=dev)
        aout = torch.empty(2 + 5, dtype=torch.int32, device=dev)
        nws = torch.empty(max(lib.lq_ngram_workspace_bytes(T), 256), dtype=torch.uint8, device=dev)
        aws = torch.empty(max(lib.lq_accept_workspace_bytes(5, 131072), 256), dtype=torch.uint8, device=dev)

        def ngram(j):
            st = lib.lq_ngram_propose(hist.data_ptr(), T, gram, nd, nout.data_ptr(), nws.data_ptr(),
                                      nws.numel(), sp)
            if st:
                _lib.check(st, "lq_ngram_propose")

        def accept(j):
            st = lib.lq_greedy_accept(logits.data_ptr(), 5, 131072, drafts.data_ptr(), 4,
                                      aout.data_ptr(), aws.data_ptr(), aws.numel(), sp)
            if st:
                _lib.check(st, "lq_greedy_accept")
        for j in range(args.warmup):
            ngram(j)
            accept(j)
        torch.cuda.synchronize()
        ng = _gpu_groups(stream, args.steps, 8, ngram)
        ac = _gpu_groups(stream, args.steps, 8, accept)
        ng_ms, ac_ms = sum(ng) / len(ng), sum(ac) / len(ac)
        extra = {"ngram_us_per_call": round(ng_ms * 1e3, 2), "accept_us_per_call": round(ac_ms * 1e3, 2),
                 "ngram_result": nout.tolist(), "accept_result": aout.tolist()[:2],
                 "roofline": {"bound": "hbm", "achieved": round((T * 4 + 5 * 131072 * 4) / ((ng_ms + ac_ms) * 1e-3) / 1e9, 1),
                              "peak": PEAK_GBS, "unit": "GB/s",
                              "frac": round((T * 4 + 5 * 131072 * 4) / ((ng_ms + ac_ms) * 1e-3) / 1e9 / PEAK_GBS, 5),
                              "traffic": None, "kernel": "lq_ngram_propose + lq_greedy_accept (latency-bound)",
                              "bytes_per_call": T * 4 + 5 * 131072 * 4}}
        if do_cpu:
            from oracle import lookup as O
            ids = h.tolist()
            idx = O.DictIndex(gram)
            idx.extend(ids)
            ln = logits.cpu().numpy()
            dr = drafts.cpu().numpy()
            t_dict, c1 = _time_cpu(lambda: idx.propose(nd), min(2.0, args.cpu_seconds))
            t_scan, c2 = _time_cpu(lambda: O.propose_scan(h, T, gram, nd), min(4.0, args.cpu_seconds))
            t_acc, c3 = _time_cpu(lambda: O.greedy_accept(ln, dr), min(4.0, args.cpu_seconds))
            extra["cpu_baseline"] = {
                "value": round((t_scan + t_acc) * 1e6, 1), "unit": "us/call", "cores": 1, "kind": "port",
                "dict_propose_us": round(t_dict * 1e6, 2), "scan_propose_us": round(t_scan * 1e6, 1),
                "accept_us": round(t_acc * 1e6, 1),
                "sample": f"medians of {c1}/{c2}/{c3} calls: the reference's dict NgramIndex.propose "
                          f"(amortised, index already built), the NumPy backward scan, np.argmax accept; "
                          f"CPU: {_cpu_model()}"}
        _result("n-gram draft search (82,671 ids, g=3, n=4) + greedy accept (5 x 131,072) us/call",
                round((ng_ms + ac_ms) * 1e3, 2), "us", False, ng_ms + ac_ms, args, "int32",
                {"workload": "prompt-lookup draft search + greedy accept", "history": T, "g": gram,
                 "n": nd, "vocab": 131072, "rows": 5}, extra)
        return


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported on this "
              "single-GPU build (the path would shard by KV head)", file=sys.stderr)
        sys.exit(2)

    import ctypes as C

    import numpy as np
    import torch

    from lagunalab_amd import _lib

    global HQ
    HQ = args.q_heads
    if HQ % HKV or not HKV <= HQ <= 16 * HKV:
        sys.exit(f"--q-heads must be a multiple of {HKV} in [{HKV}, {16 * HKV}]")
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.workload != "decode":
        run_workload(args)
        return

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    g = torch.Generator(device=dev).manual_seed(0)

    ctx, nl = args.ctx, args.layers
    total_steps = args.warmup + args.steps
    # Step i (warm-up steps first) appends at row ctx + i and attends over ctx + i + 1 rows: the
    # session's consecutive decode steps (n = ctx + 1, ctx + 2, ...), the layer caches rotating
    # step by step. Every cache holds ctx + total_steps quantized rows, so the rows below each
    # step's new row are valid whichever layer served the steps before.
    rows = ctx + total_steps
    cap = (rows + 255) // 256 * 256
    # ---- caches: N(0,1) bf16 rows quantized on the GPU (group 64, 8-bit)
    layers = []
    for _ in range(nl):
        lay = []
        for _kv in range(2):
            codes = torch.zeros((1, HKV, cap, D), dtype=torch.uint8, device=dev)
            sc = torch.zeros((1, HKV, cap, D // GS), dtype=torch.bfloat16, device=dev)
            bi = torch.zeros_like(sc)
            x = torch.randn((1, HKV, rows, D), device=dev, generator=g).to(torch.bfloat16)
            _lib.check(lib.lq_quantize_append(x.data_ptr(), 1, HKV, rows, D, codes.data_ptr(),
                                              sc.data_ptr(), bi.data_ptr(), cap, 0, 8, GS, sp),
                       "prefill quantize")
            del x
            lay.append((codes, sc, bi))
        layers.append(lay)
    qs = torch.randn((total_steps, 1, HQ, 1, D), device=dev, generator=g).to(torch.bfloat16)
    ks_new = torch.randn((total_steps, 1, HKV, 1, D), device=dev, generator=g).to(torch.bfloat16)
    vs_new = torch.randn((total_steps, 1, HKV, 1, D), device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty((1, HQ, 1, D), dtype=torch.bfloat16, device=dev)
    ws_bytes = lib.lq_decode_workspace_bytes(8, 1, HQ, HKV, D, rows, None)
    ws = torch.zeros(ws_bytes * 2, dtype=torch.uint8, device=dev)  # leading counters start at 0
    offsets = [ctx] * nl
    torch.cuda.synchronize()

    def attend_args(i, lay, n):
        (kc, ks, kb), (vc, vs, vb) = lay
        return (8, qs[i].data_ptr(), kc.data_ptr(), ks.data_ptr(), kb.data_ptr(), vc.data_ptr(),
                vs.data_ptr(), vb.data_ptr(), 1, HQ, HKV, D, cap, n, None, D ** -0.5,
                out.data_ptr(), ws.data_ptr(), ws.numel(), sp)

    def attend(i, lay, n):
        return lib.lq_decode_attn(*attend_args(i, lay, n))

    def step_launches(i):
        """Step i as the (entry point, arguments) of its launches: the fused step appends at row
        ctx + i of layer i % nl and attends over ctx + i + 1 rows. Built before any timing, so
        that the timed loop only issues the calls."""
        lay = layers[i % nl]
        (kc, ks, kb), (vc, vs, vb) = lay
        off = ctx + i
        if args.separate_append:
            return [(lib.lq_quantize_append_kv,
                     (ks_new[i].data_ptr(), vs_new[i].data_ptr(), 1, HKV, 1, D, kc.data_ptr(),
                      ks.data_ptr(), kb.data_ptr(), vc.data_ptr(), vs.data_ptr(), vb.data_ptr(),
                      cap, off, 8, GS, sp)),
                    (lib.lq_decode_attn, attend_args(i, lay, off + 1))]
        return [(lib.lq_q8_decode_append_attn,
                 (qs[i].data_ptr(), ks_new[i].data_ptr(), vs_new[i].data_ptr(), kc.data_ptr(),
                  ks.data_ptr(), kb.data_ptr(), vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), 1, HQ,
                  HKV, D, cap, off, None, D ** -0.5, out.data_ptr(), ws.data_ptr(), ws.numel(),
                  sp))]

    launches = [step_launches(i) for i in range(total_steps)]

    def run_steps(first, count):
        """Issues steps first .. first + count - 1; returns the OR of their status codes."""
        st = 0
        for i in range(first, first + count):
            for fn, a in launches[i]:
                st |= fn(*a)
        return st

    # ---- settle: plain attention calls (the same kernel without the append, n = ctx rows, which
    # every cache holds) over the rotating caches, then the warm-up steps
    settled = settle(stream, args.settle_ms,
                     lambda j: _lib.check(attend(j % total_steps, layers[j % nl], ctx), "settle"))
    _lib.check(run_steps(0, args.warmup), "warm-up step")
    torch.cuda.synchronize()

    # ---- timed region: K steps, bracketed by one pair of events on the launch stream
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    st = run_steps(args.warmup, args.steps)
    t_end.record(stream)
    torch.cuda.synchronize()
    _lib.check(st, "timed step")
    total_ms = t_start.elapsed_time(t_end)
    ns = [ctx + i + 1 for i in range(args.warmup, total_steps)]  # rows attended per timed step
    for i in range(total_steps):
        offsets[i % nl] = ctx + i + 1

    # ---- roofline of the dominant kernel. Fused steps: each timed step is exactly one launch of
    # lq_q8_decode_append_attn, so its average launch duration is the timed region's time / K
    # (events on the launch stream; this includes the short gap between consecutive launches).
    # Separate-append steps: groups of 8 back-to-back lq_decode_attn calls over the rotating
    # caches, one event pair per group, after the timed steps. Either way the plain attention
    # call is also timed that way and reported as attn_us_per_call.
    group = 8
    pairs, attn_n = [], []
    n_groups = args.roofline_calls // group if not args.separate_append else max(1, args.roofline_calls // group)
    for gi in range(n_groups):
        e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        e[0].record(stream)
        for k in range(group):
            j = gi * group + k
            li = j % nl
            _lib.check(attend(j % total_steps, layers[li], offsets[li]), "attention call")
            attn_n.append(offsets[li])
        e[1].record(stream)
        pairs.append(e)
    torch.cuda.synchronize()
    attn_ms = [a.elapsed_time(b) / group for a, b in pairs]  # empty with --roofline-calls 0

    # single cache ("hot"): the plain attention call repeated on layer 0's cache, outside the
    # timed region and reported apart from it
    single = None
    if nl > 1 and args.hot_calls > 0:
        n0 = offsets[0]
        for j in range(8):
            _lib.check(attend(j % total_steps, layers[0], n0), "single-cache warm-up call")
        e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        torch.cuda.synchronize()
        e[0].record(stream)
        for j in range(args.hot_calls):
            _lib.check(attend(j % total_steps, layers[0], n0), "single-cache call")
        e[1].record(stream)
        torch.cuda.synchronize()
        hot_ms = e[0].elapsed_time(e[1]) / args.hot_calls
        hot_bytes = Q8_TOKEN * n0 + 2 * HQ * D * 2
        single = {"us_per_call": round(hot_ms * 1e3, 2),
                  "gb_per_s": round(hot_bytes / (hot_ms * 1e-3) / 1e9, 1), "calls": args.hot_calls,
                  "rows": n0,
                  "label": f"lq_decode_attn on one layer's cache ({hot_bytes / 1e6:.1f} MB) call "
                           "after call, as the reference's micro-benchmark times it: the cache stays "
                           "in the 256 MB last-level cache between calls, so this is cache-assisted, "
                           "not the HBM rate of the headline"}

    # per step: K/V codes + scales/biases over n rows, the new bf16 K/V rows read (4096 B), the
    # appended q8 K/V rows written (2176 B), q read and out written (8192 B each)
    step_bytes = [Q8_TOKEN * n + 2 * HKV * D * 2 + Q8_TOKEN + 2 * HQ * D * 2 for n in ns]
    value = sum(step_bytes) / (total_ms * 1e-3) / 1e9
    attn_bytes = [Q8_TOKEN * n + 2 * HQ * D * 2 for n in attn_n]
    attn_avg_ms = sum(attn_ms) / len(attn_ms) if attn_ms else None
    attn_med_ms = sorted(attn_ms)[len(attn_ms) // 2] if attn_ms else None
    if args.separate_append:
        kernel = "lq_decode_attn (q8_attn_packed_kernel, split merge fused)"
        k_ms, k_bytes, k_calls = attn_avg_ms, sum(attn_bytes) / len(attn_bytes), len(attn_ms) * group
    else:
        if HQ // HKV <= 4 and ctx + 1 > 65536:
            kernel = ("lq_q8_decode_append_attn (q8_attn_packed_kernel: append + attention + split "
                      "merge)")
        elif HQ // HKV <= 8:
            kernel = ("lq_q8_decode_append_attn (q8_attn_dense_kernel: append + attention + split "
                      "merge)")
        else:
            kernel = ("lq_q8_decode_append_attn (q8_attn_dense_kernel: append + attention; "
                      "decode_merge_kernel)")
        k_ms, k_bytes, k_calls = total_ms / args.steps, sum(step_bytes) / len(step_bytes), args.steps
    achieved = k_bytes / (k_ms * 1e-3) / 1e9

    # HBM bytes per fused step: not measured in this run (hardware counters need a profiler run
    # of their own); read from the committed record of two rocprofv3 --pmc passes (FETCH_SIZE,
    # then WRITE_SIZE) of this same workload, scaled by a plain-copy calibration, and labelled so.
    traffic, traffic_src = None, None
    tf = ROOT / "profiles" / "q8_decode_traffic.json"
    if tf.exists() and HQ == 32 and not args.separate_append and ctx == 82671:
        try:
            traffic = json.loads(tf.read_text()).get("hbm_bytes_per_call")
            traffic_src = ("copied from profiles/q8_decode_traffic.json (rocprofv3 --pmc FETCH_SIZE "
                           "and WRITE_SIZE passes of this workload, scaled by a plain-copy "
                           "calibration), not measured in this run")
        except Exception:
            traffic = None

    # the metric names its context (the headline one is quoted at 82,671 cached rows); vs_baseline
    # only where the reference published a number for that context
    metric = METRIC if ctx == 82671 else METRIC.replace("82,671", f"{ctx:,}")
    if HQ != 32:
        metric = f"{metric}, {HQ}q/{HKV}kv"
    ref_gbs = ctx * Q8_TOKEN / (REF_M4_MS[ctx] * 1e-3) / 1e9 if ctx in REF_M4_MS and HKV == 8 else None
    res = {
        "metric": metric, "value": round(value, 2),
        "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": round(value / ref_gbs, 2) if ref_gbs else None,
        "dtype": "u8",
        "data": "synthetic (N(0,1) bf16 K/V/q, quantized on the GPU)",
        "config": {"workload": "q8 decode step (append 1 K/V row + fused attention, "
                               + ("separate append launch" if args.separate_append else "one launch")
                               + "), batch 1, "
                               f"{HQ}q/{HKV}kv heads, head_dim {D}, group {GS}, context {ctx}, "
                               f"{nl} rotating layer caches; step i attends over ctx + i + 1 rows",
                   "ctx": ctx, "batch": 1, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
                   "layers": nl, "cap": cap, "n_timed": [ns[0], ns[-1]]},
        "us_per_call": round(total_ms / args.steps * 1e3, 2),
        "attn_us_per_call": ({"mean": round(attn_avg_ms * 1e3, 2), "median": round(attn_med_ms * 1e3, 2)}
                             if attn_ms else None),
        "pct_of_hbm_peak": round(100 * value / PEAK_GBS, 2),
        "settle": settled,
        "single_cache": single,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_src, "kernel": kernel, "us_per_launch": round(k_ms * 1e3, 2),
                     "launches_timed": k_calls, "bytes_per_call": int(k_bytes)},
        "vs_baseline_ref": "reference fused q8 kernel on an M4 GPU: 12.24 ms/call = 14.69 GB/s",
    }
    if not args.no_cpu_baseline and args.cpu_seconds > 0:
        lay = layers[0]
        n0 = offsets[0]
        host = [t[0].cpu().numpy() if t.dtype == torch.uint8 else
                t[0].view(torch.int16).cpu().numpy().view(np.uint16) for kv in lay for t in kv]
        qn = qs[0, 0, :, 0].float().cpu().numpy()
        res["cpu_baseline"] = cpu_baseline(*host, qn, n0, args.cpu_seconds)
        res["cpu_baseline"]["value_vs_gpu"] = round(value / res["cpu_baseline"]["value"], 1)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
