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
roofline of the decode attention kernel (HIP events on the launch stream around groups of
back-to-back calls after the timed steps), and the CPU baseline (the oracle's unfused
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
REF_M4_GBS = 179892096 / 12.243627500138246e-3 / 1e9  # reference fused kernel on an M4 GPU (results/kv_decode_micro_fused.json)
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
                   help="attention calls timed for the roofline, in groups of 8, after the timed steps")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU baseline sample: calls are repeated until this much time has passed")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--separate-append", action="store_true",
                   help="append with its own launch (lq_quantize_append_kv) before lq_decode_attn "
                        "instead of the fused step (lq_q8_decode_append_attn)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB 8 times (HBM counter calibration)")
    return p.parse_args()


def cpu_baseline(kc, ks, kb, vc, vs, vb, q, n, seconds):
    """The reference's unfused path restated by the oracle: dequantize the cache to bf16, then
    fp32 SDPA (BLAS). The 8 KV heads run in a thread pool (NumPy releases the GIL)."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor

    from oracle import attention as A
    from oracle import quantize as Q

    threads = min(HKV, len(os.sched_getaffinity(0)))
    G = HQ // HKV

    def one_head(h):
        k = Q.dequantize(kc[h, :n], ks[h, :n], kb[h, :n])
        v = Q.dequantize(vc[h, :n], vs[h, :n], vb[h, :n])
        return A.sdpa(q[None, h * G:(h + 1) * G, None], k[None, None], v[None, None], D ** -0.5,
                      dtype=np.float32)

    times = []
    with ThreadPoolExecutor(threads) as ex:
        list(ex.map(one_head, range(HKV)))  # warm-up
        t_end = time.perf_counter() + seconds
        while len(times) < 3 or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            list(ex.map(one_head, range(HKV)))
            times.append(time.perf_counter() - t0)
    calls = len(times)
    t = sorted(times)[len(times) // 2]
    try:
        model = [l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name")][0]
    except Exception:
        model = "unknown"
    return {
        "value": round(Q8_TOKEN * n / t / 1e9, 3), "unit": "GB/s", "cores": threads,
        "kind": "port", "us_per_call": round(t * 1e6, 1),
        "sample": (f"median of {calls} calls (after 1 warm-up) of the unfused dequantize-to-bf16 + "
                   f"fp32 SDPA path at n={n} on one layer, 8 KV heads over {threads} threads; "
                   f"CPU: {model}"),
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

    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    g = torch.Generator(device=dev).manual_seed(0)

    ctx, nl = args.ctx, args.layers
    total_steps = args.warmup + args.steps
    grow = (total_steps + nl - 1) // nl
    cap = (ctx + 255) // 256 * 256
    if ctx + grow > cap:
        cap += 256
    # ---- caches: N(0,1) bf16 rows quantized on the GPU (group 64, 8-bit)
    layers = []
    for _ in range(nl):
        lay = []
        for _kv in range(2):
            codes = torch.zeros((1, HKV, cap, D), dtype=torch.uint8, device=dev)
            sc = torch.zeros((1, HKV, cap, D // GS), dtype=torch.bfloat16, device=dev)
            bi = torch.zeros_like(sc)
            x = torch.randn((1, HKV, ctx, D), device=dev, generator=g).to(torch.bfloat16)
            _lib.check(lib.lq_quantize_append(x.data_ptr(), 1, HKV, ctx, D, codes.data_ptr(),
                                              sc.data_ptr(), bi.data_ptr(), cap, 0, 8, GS, sp),
                       "prefill quantize")
            del x
            lay.append((codes, sc, bi))
        layers.append(lay)
    qs = torch.randn((total_steps, 1, HQ, 1, D), device=dev, generator=g).to(torch.bfloat16)
    ks_new = torch.randn((total_steps, 1, HKV, 1, D), device=dev, generator=g).to(torch.bfloat16)
    vs_new = torch.randn((total_steps, 1, HKV, 1, D), device=dev, generator=g).to(torch.bfloat16)
    out = torch.empty((1, HQ, 1, D), dtype=torch.bfloat16, device=dev)
    ws_bytes = lib.lq_decode_workspace_bytes(8, 1, HQ, HKV, D, ctx + grow, None)
    ws = torch.zeros(ws_bytes * 2, dtype=torch.uint8, device=dev)  # leading counters start at 0
    offsets = [ctx] * nl
    torch.cuda.synchronize()

    def append(i, lay, off):
        (kc, ks, kb), (vc, vs, vb) = lay
        return lib.lq_quantize_append_kv(ks_new[i].data_ptr(), vs_new[i].data_ptr(), 1, HKV, 1, D,
                                         kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
                                         vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), cap, off,
                                         8, GS, sp)

    def attend(i, lay, n):
        (kc, ks, kb), (vc, vs, vb) = lay
        return lib.lq_decode_attn(8, qs[i].data_ptr(), kc.data_ptr(), ks.data_ptr(),
                                  kb.data_ptr(), vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), 1,
                                  HQ, HKV, D, cap, n, None, D ** -0.5, out.data_ptr(),
                                  ws.data_ptr(), ws.numel(), sp)

    def fused_step(i, lay, off):
        (kc, ks, kb), (vc, vs, vb) = lay
        return lib.lq_q8_decode_append_attn(qs[i].data_ptr(), ks_new[i].data_ptr(),
                                            vs_new[i].data_ptr(), kc.data_ptr(), ks.data_ptr(),
                                            kb.data_ptr(), vc.data_ptr(), vs.data_ptr(),
                                            vb.data_ptr(), 1, HQ, HKV, D, cap, off, None,
                                            D ** -0.5, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                            sp)

    def step(i):
        li = i % nl
        off = offsets[li]
        if args.separate_append:
            st = append(i, layers[li], off)
            st |= attend(i, layers[li], off + 1)
        else:
            st = fused_step(i, layers[li], off)
        offsets[li] = off + 1
        if st:
            _lib.check(st, "bench step")
        return off + 1

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # ---- timed region: K steps, bracketed by one pair of events on the launch stream
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    ns = []
    torch.cuda.synchronize()
    t_start.record(stream)
    for j in range(args.steps):
        ns.append(step(args.warmup + j))
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)

    # ---- roofline of the attention kernel: groups of 8 back-to-back lq_decode_attn calls (one
    # kernel launch each) over the rotating caches, one event pair per group on the launch stream.
    # Per-call time = group time / 8, which includes the short gap between consecutive launches.
    group = 8
    pairs, attn_n = [], []
    for gi in range(max(1, args.roofline_calls // group)):
        e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        e[0].record(stream)
        for k in range(group):
            j = gi * group + k
            li = j % nl
            _lib.check(attend(j % total_steps, layers[li], offsets[li]), "roofline call")
            attn_n.append(offsets[li])
        e[1].record(stream)
        pairs.append(e)
    torch.cuda.synchronize()
    attn_ms = [a.elapsed_time(b) / group for a, b in pairs]

    # per step: K/V codes + scales/biases over n rows, the new bf16 K/V rows read (4096 B), the
    # appended q8 K/V rows written (2176 B), q read and out written (8192 B each)
    step_bytes = [Q8_TOKEN * n + 2 * HKV * D * 2 + Q8_TOKEN + 2 * HQ * D * 2 for n in ns]
    value = sum(step_bytes) / (total_ms * 1e-3) / 1e9
    attn_bytes = [Q8_TOKEN * n + 2 * HQ * D * 2 for n in attn_n]
    attn_avg_ms = sum(attn_ms) / len(attn_ms)
    attn_med_ms = sorted(attn_ms)[len(attn_ms) // 2]
    achieved = (sum(attn_bytes) / len(attn_bytes)) / (attn_avg_ms * 1e-3) / 1e9

    traffic = None
    tf = ROOT / "profiles" / "q8_decode_traffic.json"
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text()).get("hbm_bytes_per_call")
        except Exception:
            traffic = None

    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": round(value / REF_M4_GBS, 2), "dtype": "u8",
        "data": "synthetic (N(0,1) bf16 K/V/q, quantized on the GPU)",
        "config": {"workload": "q8 decode step (append 1 K/V row + fused attention, "
                               + ("separate append launch" if args.separate_append else "one launch")
                               + "), batch 1, "
                               f"{HQ}q/{HKV}kv heads, head_dim {D}, group {GS}, context {ctx}, "
                               f"{nl} rotating layer caches",
                   "ctx": ctx, "batch": 1, "q_heads": HQ, "kv_heads": HKV, "head_dim": D,
                   "layers": nl, "cap": cap},
        "us_per_call": round(total_ms / args.steps * 1e3, 2),
        "attn_us_per_call": {"mean": round(attn_avg_ms * 1e3, 2), "median": round(attn_med_ms * 1e3, 2)},
        "pct_of_hbm_peak": round(100 * value / PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "lq_decode_attn (q8_attn_packed_kernel, split merge fused)",
                     "calls_timed": len(attn_ms) * group,
                     "bytes_per_call": int(sum(attn_bytes) / len(attn_bytes))},
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
