#!/usr/bin/env python3
"""Benchmark of the KV-cache path on one MI355X: the headline metric and the other benchmark configs.

Default (the driver's line): benchmark config 3, the headline. A step is one
decode token through all 64 layers at Qwen2.5-32B attention shapes (40 query /
8 kv heads, head_dim 128, fp16 KV, context 32768 after the append, all 64
layers' caches resident in HBM, 8 GiB): per layer ONE launch of
friday_attn_decode_step = RoPE + KV append at position S-1 + split-K GQA decode
attention + log-sum-exp merge. The 64 launches are captured once into a HIP
graph (the reference captures its decode layers into a CUDA graph,
transformer.cpp:1465-1483) and replayed; layers run back to back, each one
after the previous one finished, as in a real decode step.

`value` = K/V bytes the attention must read per layer-step (2*S*Hkv*d*2 =
134,217,728 B) / measured time per layer-step, in GB/s. `roofline` is that of
the one kernel a layer-step launches (fa_decode_kernel, step variant): its
average duration = timed-region time / launches, from HIP events on the
stream the graph runs on. `cpu_baseline` times the reference's own CPU
attention (cpu_ops.cpp decodeAttention compiled from source into oracle/_ref)
on this host.

--config all additionally prints one JSON line per other benchmark config
(1: Qwen2.5-0.5B shapes; 2: 32 layers at 1k/4k/8k, cold and warm; 3 at 16k;
4: chunked prefill on MFMA with MFMA utilisation; 5: 16 paged sequences), the int8-KV step,
the RoPE + KV append rows (T = 1 and 512, fp16 and int8), the prefill launch against T
single-token decode launches (the reference's own comparison), and the matmuls either
side of attention;
--config short prints configs 1 and 2 only.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "friday-inference-engine_amd"))

METRIC = "decode-attn µs/layer-step + KV GB/s (% HBM peak) at 32k ctx, 40q/8kv d128"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 and bf16 MFMA
MALL_BYTES = 256 << 20         # Infinity Cache: a "cold" working set must exceed it

# HBM traffic of one step-kernel launch at the headline shape: a constant taken from the
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs recorded in the profile below (KiB per
# dispatch, scaled by the copy-kernel calibration FETCH_SIZE x 2.0, WRITE_SIZE x 1.0);
# it is not measured in this run.
HEADLINE_TRAFFIC_BYTES = 135877734
TRAFFIC_SOURCE = "constant from profiles/decode_step_cfg3_pmc.txt (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE; calibrated)"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Ctx:
    """HIP plumbing shared by the measurements."""

    def __init__(self):
        import friday_attn as fa

        self.fa = fa
        fa.load()
        if fa.Hip.device_count() < 1:
            raise SystemExit("no HIP device")
        self.bk = C.CDLL(os.path.join(ROOT, "bench_kit", "libfa_benchkit.so"))
        self.bk.fabk_fill_normal_f16.argtypes = [C.c_void_p, C.c_size_t, C.c_uint32, C.c_float, C.c_void_p]
        self.bk.fabk_fill_normal_bf16.argtypes = [C.c_void_p, C.c_size_t, C.c_uint32, C.c_float, C.c_void_p]
        self.stream = fa.Stream()
        if os.environ.get("FRIDAY_ATTN_LOCAL_MERGE") == "1":  # run the placement check before any capture
            fa.setDecodeForm(1, -1, -1)

    def fill(self, buf, n_half, seed, scale=1.0, bf16=False):
        f = self.bk.fabk_fill_normal_bf16 if bf16 else self.bk.fabk_fill_normal_f16
        f(buf.ptr, n_half, seed, scale, self.stream.s)

    def timed(self, fn, steps, warmup, stats=0):
        """Capture fn's launches into a graph; replay warmup + steps times; ms per replay.
        stats > 0: afterwards time that many further replays one by one (HIP events between
        consecutive replays) and return (ms per replay, {median, p10, p90} in ms)."""
        fa = self.fa
        graph = fa.Graph(self.stream, fn)
        ev = []
        try:
            for _ in range(warmup):
                graph.launch()
            self.stream.synchronize()
            t0, t1 = fa.Event(), fa.Event()
            ev += [t0, t1]
            t0.record(self.stream.s)
            for _ in range(steps):
                graph.launch()
            t1.record(self.stream.s)
            self.stream.synchronize()
            ms = t0.elapsed_ms(t1) / steps if steps else 0.0
            if not stats:
                return ms
            import numpy as np

            se = [fa.Event() for _ in range(stats + 1)]
            ev += se
            se[0].record(self.stream.s)
            for i in range(stats):
                graph.launch()
                se[i + 1].record(self.stream.s)
            self.stream.synchronize()
            d = np.array([se[i].elapsed_ms(se[i + 1]) for i in range(stats)])
            return ms, {"replays": stats, "median_ms": round(float(np.median(d)), 4),
                        "p10_ms": round(float(np.percentile(d, 10)), 4),
                        "p90_ms": round(float(np.percentile(d, 90)), 4)}
        finally:
            # the graph holds raw pointers into the caller's buffers, which are freed after
            # this returns: it must be gone first (and its launches complete)
            self.stream.synchronize()
            graph.destroy()
            for e in ev:
                e.destroy()


class DecodeLayers:
    """`sets` x `L` layer caches [S][Hkv*d] fp16 plus per-layer q/k/v/out and one workspace."""

    def __init__(self, cx, S, L, Hq, Hkv, d, sets=1, seed=0):
        import numpy as np

        fa = cx.fa
        self.cx, self.S, self.L, self.Hq, self.Hkv, self.d, self.sets = cx, S, L, Hq, Hkv, d, sets
        self.kv_dim = Hkv * d
        self.layer_bytes = S * self.kv_dim * 2
        n = sets * L
        self.k = fa.DeviceBuffer(n * self.layer_bytes)
        self.v = fa.DeviceBuffer(n * self.layer_bytes)
        cx.fill(self.k, n * S * self.kv_dim, 1 + seed)
        cx.fill(self.v, n * S * self.kv_dim, 2 + seed)
        rng = np.random.default_rng(seed)
        f16 = lambda shape: rng.standard_normal(shape, dtype=np.float32).astype(np.float16).view(np.uint16)
        self.q = fa.DeviceBuffer.from_array(f16((n, Hq * d)))
        self.kn = fa.DeviceBuffer.from_array(f16((n, self.kv_dim)))
        self.vn = fa.DeviceBuffer.from_array(f16((n, self.kv_dim)))
        self.out = fa.DeviceBuffer(n * Hq * d * 2)
        self.table = fa.DeviceBuffer(fa.rope_table_bytes(S, d))
        fa.rope_table_upload(self.table, S, d, 1e6)
        self.pos = fa.DeviceBuffer.from_array(np.array([S - 1], np.int32))
        self.ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, S))
        fa.decodeWorkspaceInit(self.ws, stream=cx.stream.s)
        cx.stream.synchronize()

    def ptrs(self, i):
        return (self.q.ptr + i * self.Hq * self.d * 2, self.kn.ptr + i * self.kv_dim * 2,
                self.vn.ptr + i * self.kv_dim * 2, self.k.ptr + i * self.layer_bytes,
                self.v.ptr + i * self.layer_bytes, self.out.ptr + i * self.Hq * self.d * 2)

    def step(self, s):
        """One decode step of layer set s: one launch per layer."""
        fa, cx = self.cx.fa, self.cx
        for l in range(self.L):
            q, kn, vn, kc, vc, out = self.ptrs(s * self.L + l)
            fa.decodeStep(q, kn, vn, kc, vc, out, self.pos, 0, self.S, self.Hq, self.Hkv, self.d, self.table, 1,
                          self.ws, cx.stream.s)

    def decode_only(self, s):
        fa, cx = self.cx.fa, self.cx
        for l in range(self.L):
            q, _, _, kc, vc, out = self.ptrs(s * self.L + l)
            fa.launchDecodeAttentionFused(q, kc, vc, out, 0, self.pos, self.S, self.Hq, self.Hkv, self.d, self.ws,
                                          cx.stream.s)

    def measure(self, steps, warmup, fn="step", stats=0):
        """ms per decode step; with several sets each replay walks all of them (cold caches).
        stats > 0: also the per-replay distribution (see Ctx.timed)."""
        f = getattr(self, fn)
        r = self.cx.timed(lambda: [f(s) for s in range(self.sets)], steps, warmup, stats)
        if stats:
            return r[0] / self.sets, r[1]
        return r / self.sets

    def check_layer0(self):
        import numpy as np

        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        from py_oracle import Oracle

        S, Hq, Hkv, d = self.S, self.Hq, self.Hkv, self.d
        q0 = self.q.download(Hq * d, np.uint16)
        k0 = self.k.download((S, self.kv_dim), np.uint16)
        v0 = self.v.download((S, self.kv_dim), np.uint16)
        got = self.out.download(Hq * d, np.uint16).view(np.float16).astype(np.float32)
        ref = Oracle().decode(q0, k0, v0, S, Hq, Hkv, d)
        err = np.abs(got - ref)
        ok = bool(np.all(err <= 2e-3 + 1e-2 * np.abs(ref)))
        log(f"[bench] layer 0 vs oracle: max_abs {err.max():.2e} {'PASS' if ok else 'FAIL'}")
        return {"layer0_vs_oracle_max_abs": float(err.max()), "pass": ok}

    def free(self):
        for b in (self.k, self.v, self.q, self.kn, self.vn, self.out, self.table, self.pos, self.ws):
            b.free()


# The GPU box gives one GPU's job a share of 16 logical CPUs, whatever os.cpu_count() reports.
CPU_SHARE = 16


def cpu_thread_counts(Hq):
    """The two thread counts the CPU baseline is timed at: min(logical CPUs, Hq) (the
    reference parallelises decode attention over query heads, cpu_ops.cpp:50) and the
    reference's default pool size, 2/3 of the logical CPUs (cpu_backend.cpp:45-50)."""
    ncpu = min(os.cpu_count() or 1, CPU_SHARE)
    return max(1, min(ncpu, Hq)), (ncpu * 2 // 3 if ncpu >= 3 else 1)


def cpu_baseline(S, Hq, Hkv, d, budget_s, threads=None):
    """Reference CPU decode attention (cpu_ops.cpp:45-83) on a bounded sample."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import py_oracle

    ncpu = os.cpu_count() or 1
    if threads is None:
        threads = cpu_thread_counts(Hq)[0]
    rng = np.random.default_rng(0)
    kv_dim = Hkv * d
    kc = rng.standard_normal((S, kv_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
    vc = rng.standard_normal((S, kv_dim), dtype=np.float32).astype(np.float16).astype(np.float32)
    q = rng.standard_normal(Hq * d, dtype=np.float32).astype(np.float16).astype(np.float32)
    if py_oracle.ref_available():
        ref = py_oracle.RefCpu()
        kind = "reference"
        run = lambda: ref.decode(q, kc, vc, S, Hq, Hkv, d, threads=threads)
        what = "oracle/_ref: the reference's cpu_ops.cpp decodeAttention compiled from source"
    else:
        orc = py_oracle.Oracle()
        kind, threads = "port", 1
        qh, kh, vh = (a.astype(np.float16) for a in (q, kc, vc))
        run = lambda: orc.decode(qh, kh, vh, S, Hq, Hkv, d)
        what = "oracle/fa_oracle.c restatement of cpu_ops.cpp decodeAttention (single thread)"
    run()  # warm the pool and the pages
    n, t0 = 0, time.perf_counter()
    while True:
        run()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 1000:
            break
    us = el / n * 1e6
    return {"value": round(us, 1), "unit": "us/layer-step", "cores": threads, "kind": kind,
            "kv_gbs_fp32": round(2 * S * kv_dim * 4 / (us * 1e-6) / 1e9, 2),
            "sample": f"{n} calls of one layer (ctx {S}, {Hq}q/{Hkv}kv d{d}, fp32 cache holding fp16 values), "
                      f"{el:.1f} s; {what}; host logical CPUs {ncpu}"}


def decode_form():
    """The decode placement / merge switches this process runs with (environment)."""
    return {k.lower().replace("friday_attn_", ""): os.environ.get(k, "0") for k in
            ("FRIDAY_ATTN_LOCAL_MERGE", "FRIDAY_ATTN_SPLIT_MAJOR", "FRIDAY_ATTN_KV_PAIR", "FRIDAY_ATTN_Q8_DEEP")}


def headline(cx, args):
    S, L, Hq, Hkv, d = args.ctx, args.layers, 40, 8, 128
    log(f"[bench] config 3: S={S} layers={L} {Hq}q/{Hkv}kv d{d}, {2 * L * S * Hkv * d * 2 / 2**30:.2f} GiB KV")
    dl = DecodeLayers(cx, S, L, Hq, Hkv, d)
    ms_step = dl.measure(args.steps, args.warmup, "step")
    step_stats = dl.measure(0, 0, "step", stats=args.stat_replays)[1] if args.stat_replays > 0 else None
    ms_dec = dl.measure(args.steps, args.warmup, "decode_only")
    check = None if args.no_check else dl.check_layer0()
    dl.free()
    us_layer = ms_step * 1e3 / L
    kv_bytes = 2 * S * Hkv * d * 2
    gbs = kv_bytes / (us_layer * 1e-6) / 1e9
    log(f"[bench] {ms_step:.3f} ms/step, {us_layer:.2f} us/layer-step ({gbs:.0f} GB/s), "
        f"decode-only launch {ms_dec * 1e3 / L:.2f} us")
    cpu = cpu_ref_default = None
    if not args.no_cpu:
        t_heads, t_default = cpu_thread_counts(Hq)
        log(f"[bench] timing the reference CPU attention ({t_heads} and {t_default} threads) ...")
        cpu = cpu_baseline(S, Hq, Hkv, d, args.cpu_seconds / 2, threads=t_heads)
        cpu_ref_default = cpu_baseline(S, Hq, Hkv, d, args.cpu_seconds / 2, threads=t_default)
    return {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: device-generated N(0,1) fp16 K/V caches, seeded N(0,1) q/k/v",
        "config": {"workload": f"benchmark config 3 (headline): decode step over {L} layers, one launch per layer "
                               f"(RoPE + KV append + split-K GQA attention + LSE merge), ctx {S} after the append, "
                               f"{Hq}q/{Hkv}kv d{d}, fp16 KV, batch 1, HIP graph replay",
                   "layers": L, "ctx": S, "num_heads": Hq, "num_kv_heads": Hkv, "head_dim": d},
        "us_per_layer_step": round(us_layer, 3),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "decode_form": decode_form(),
        "tokens_per_s": round(1e3 / ms_step, 2),
        "decode_only_launch_us": round(ms_dec * 1e3 / L, 3),
        "roofline": {"bound": "hbm", "kernel": "fa_decode_kernel (step variant: friday_attn_decode_step)",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": HEADLINE_TRAFFIC_BYTES,
                     "traffic_source": TRAFFIC_SOURCE,
                     "algorithmic_bytes_per_launch": kv_bytes, "launches_per_step": L},
        "step_stats": None if step_stats is None else {
            **step_stats, "us_per_layer_median": round(step_stats["median_ms"] * 1e3 / L, 3),
            "us_per_layer_p10": round(step_stats["p10_ms"] * 1e3 / L, 3),
            "us_per_layer_p90": round(step_stats["p90_ms"] * 1e3 / L, 3)},
        "cpu_baseline": cpu,
        "cpu_baseline_reference_default_threads": cpu_ref_default,
        "check": check,
    }


def decode_config(cx, name, S, L, Hq, Hkv, d, steps, warmup, cold):
    kv_bytes = 2 * S * Hkv * d * 2
    sets = 1
    if cold:  # rotate through enough layer sets that the working set exceeds the MALL 4x over
        sets = max(1, -(-4 * MALL_BYTES // (kv_bytes * L)))
    dl = DecodeLayers(cx, S, L, Hq, Hkv, d, sets=sets, seed=S)
    ms = dl.measure(steps, warmup, "step")
    dl.free()
    us = ms * 1e3 / L
    gbs = kv_bytes / (us * 1e-6) / 1e9
    return {"config": name, "ctx": S, "layers": L, "heads": f"{Hq}q/{Hkv}kv d{d}", "cache": "cold" if cold else "warm",
            "working_set_MiB": round(sets * L * kv_bytes / 2**20, 1), "us_per_layer_step": round(us, 3),
            "kv_GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "tokens_per_s": round(1e3 / ms, 1)}


def append_config(cx, T, steps, warmup):
    """RoPE + KV append (friday_attn_rope_store_kv, ropeStoreKvKernel semantics) at the
    headline shapes (40q/8kv, d128): T = 1 (a decode token) or T = 512 (a prefill chunk),
    one launch per layer over 64 layers' inputs and caches. Algorithmic bytes per token:
    read q, k, v and the RoPE table row ((Hq + 2 Hkv) d 2 + d/2 8), written q and k in
    place and the k and v cache rows ((Hq + 3 Hkv) d 2)."""
    import numpy as np

    fa = cx.fa
    Hq, Hkv, d, L, max_ctx = 40, 8, 128, 64, 8192
    kv_dim = Hkv * d
    q, k, v = (fa.DeviceBuffer(L * T * n * 2) for n in (Hq * d, kv_dim, kv_dim))
    for bb, n in ((q, Hq * d), (k, kv_dim), (v, kv_dim)):
        cx.fill(bb, L * T * n, 30 + n)
    kc, vc = fa.DeviceBuffer(L * max_ctx * kv_dim * 2), fa.DeviceBuffer(L * max_ctx * kv_dim * 2)
    table = fa.DeviceBuffer(fa.rope_table_bytes(max_ctx, d))
    fa.rope_table_upload(table, max_ctx, d, 1e6)
    pos = fa.DeviceBuffer.from_array(np.array([max_ctx - T - 1], np.int32))

    def run():
        for l in range(L):
            fa.ropeStoreKv(q.ptr + l * T * Hq * d * 2, k.ptr + l * T * kv_dim * 2, v.ptr + l * T * kv_dim * 2,
                           kc.ptr + l * max_ctx * kv_dim * 2, vc.ptr + l * max_ctx * kv_dim * 2, pos, 0, T, d, Hq, Hkv,
                           max_ctx, table, 1, cx.stream.s)

    ms = cx.timed(run, steps, warmup) / L
    for bb in (q, k, v, kc, vc, table, pos):
        bb.free()
    per_token = (Hq + 2 * Hkv) * d * 2 + d // 2 * 8 + (Hq + 3 * Hkv) * d * 2
    gbs = T * per_token / (ms * 1e-3) / 1e9
    return {"config": "RoPE + KV append (ropeStoreKvKernel)", "T": T, "heads": f"{Hq}q/{Hkv}kv d{d}",
            "us_per_layer": round(ms * 1e3, 3), "bytes_per_layer": T * per_token, "GBps": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def prefill_config(cx, p0, steps, warmup, q8=False, bf16=False):
    """benchmark config 4: 512-token causal chunk after p0 cached tokens, 40q/8kv d128, MFMA.
    q8: int8 caches with one fp16 scale per 32 values (random codes, scales of 0.01 scale).
    bf16: bf16 q, caches and output on the bf16 MFMA."""
    import numpy as np

    fa = cx.fa
    T, Hq, Hkv, d = 512, 40, 8, 128
    S = p0 + T
    esz = 1 if q8 else 2
    lb = S * Hkv * d * esz
    sb = S * Hkv * d // 32 * 2
    L = max(2, -(-2 * MALL_BYTES // (2 * (lb + (sb if q8 else 0)))))  # rotate caches beyond the MALL
    k, v = fa.DeviceBuffer(L * lb), fa.DeviceBuffer(L * lb)
    cx.fill(k, L * lb // 2, 5, bf16=bf16)  # int8: the fp16 fill's bytes serve as codes
    cx.fill(v, L * lb // 2, 6, bf16=bf16)
    ks = vs = None
    if q8:
        ks, vs = fa.DeviceBuffer(L * sb), fa.DeviceBuffer(L * sb)
        cx.fill(ks, L * sb // 2, 8, scale=0.01)
        cx.fill(vs, L * sb // 2, 9, scale=0.01)
    q, out = fa.DeviceBuffer(T * Hq * d * 2), fa.DeviceBuffer(T * Hq * d * 2)
    cx.fill(q, T * Hq * d, 7, bf16=bf16)
    pos = fa.DeviceBuffer.from_array(np.array([p0], np.int32))
    if bf16:
        ms = cx.timed(lambda: [fa.launchPrefillAttentionBf16(q, k.ptr + l * lb, v.ptr + l * lb, out, T, pos, Hq, Hkv, d,
                                                             cx.stream.s) for l in range(L)], steps, warmup) / L
    else:
        ms = cx.timed(lambda: [fa.launchPrefillAttention(q, k.ptr + l * lb, v.ptr + l * lb, out, T, pos, Hq, Hkv, d,
                                                         cx.stream.s, k_scale=ks.ptr + l * sb if q8 else None,
                                                         v_scale=vs.ptr + l * sb if q8 else None)
                                       for l in range(L)], steps, warmup) / L
    for b in (k, v, q, out, pos) + ((ks, vs) if q8 else ()):
        b.free()
    flops = 4.0 * d * Hq * (T * p0 + T * (T + 1) / 2)  # causal (unmasked) QK^T and PV flops
    tf = flops / (ms * 1e-3) / 1e12
    kind = " (int8 KV)" if q8 else (" (bf16)" if bf16 else "")
    return {"config": "4: chunked prefill" + kind, "T": T, "p0": p0, "heads": f"{Hq}q/{Hkv}kv d{d}",
            "us_per_chunk": round(ms * 1e3, 2), "gflop": round(flops / 1e9, 2), "tflops": round(tf, 1),
            "mfma_utilisation": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "tokens_per_s": round(T / (ms * 1e-3), 0)}


def prefill_vs_decode_config(cx, p0, steps, warmup):
    """The reference's own comparison (tests/kernels/test_prefill_attention.cu:89-107): one
    512-token chunk after p0 cached tokens, once as T single-token split decodes (row t
    attends p0 + t + 1 positions, its position read from device memory, the merge in a second
    kernel as launchDecodeAttentionSplit does) and once as one prefill launch; 40q/8kv d128,
    fp16 KV, one cache (warm, as in the reference bench). Both are graph replays."""
    import numpy as np

    fa = cx.fa
    T, Hq, Hkv, d = 512, 40, 8, 128
    S = p0 + T
    kv_dim = Hkv * d
    k, v = fa.DeviceBuffer(S * kv_dim * 2), fa.DeviceBuffer(S * kv_dim * 2)
    cx.fill(k, S * kv_dim, 5)
    cx.fill(v, S * kv_dim, 6)
    q, out = fa.DeviceBuffer(T * Hq * d * 2), fa.DeviceBuffer(T * Hq * d * 2)
    cx.fill(q, T * Hq * d, 7)
    pos0 = fa.DeviceBuffer.from_array(np.array([p0], np.int32))
    rows = fa.DeviceBuffer.from_array(np.arange(p0, p0 + T, dtype=np.int32))  # row t: *d_pos = p0 + t
    ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, S))
    qd = Hq * d * 2

    def per_token():
        for t in range(T):
            fa.launchDecodeAttentionSplit(q.ptr + t * qd, k, v, out.ptr + t * qd, 0, rows.ptr + 4 * t, S, Hq, Hkv, d,
                                          ws, cx.stream.s)

    ms_dec = cx.timed(per_token, steps, warmup)
    ms_pf = cx.timed(lambda: fa.launchPrefillAttention(q, k, v, out, T, pos0, Hq, Hkv, d, cx.stream.s), steps, warmup)
    for b in (k, v, q, out, pos0, rows, ws):
        b.free()
    return {"config": "4: prefill launch vs T single-token decode launches (test_prefill_attention.cu --bench)",
            "T": T, "p0": p0, "heads": f"{Hq}q/{Hkv}kv d{d}", "per_token_decode_us": round(ms_dec * 1e3, 1),
            "prefill_us": round(ms_pf * 1e3, 2), "prefill_speedup": round(ms_dec / ms_pf, 1)}


def append_q8_config(cx, T, steps, warmup):
    """int8 KV append (friday_attn_store_kv_q8, storeKvQ8Kernel semantics: already-rotated k and
    v quantised per 32 values) at the headline shapes (8 kv heads, d128): T = 1 or 512, one
    launch per layer over 64 layers. Algorithmic bytes per token: k and v read as fp16
    (2 kv_dim 2), int8 rows and fp16 scales written (2 kv_dim + 2 (kv_dim / 32) 2)."""
    import numpy as np

    fa = cx.fa
    Hkv, d, L, max_ctx = 8, 128, 64, 8192
    kv_dim = Hkv * d
    k, v = fa.DeviceBuffer(L * T * kv_dim * 2), fa.DeviceBuffer(L * T * kv_dim * 2)
    cx.fill(k, L * T * kv_dim, 40)
    cx.fill(v, L * T * kv_dim, 41)
    lb, sb = max_ctx * kv_dim, max_ctx * (kv_dim // 32) * 2
    k8, v8, ks, vs = fa.DeviceBuffer(L * lb), fa.DeviceBuffer(L * lb), fa.DeviceBuffer(L * sb), fa.DeviceBuffer(L * sb)
    pos = fa.DeviceBuffer.from_array(np.array([max_ctx - T - 1], np.int32))

    def run():
        for l in range(L):
            fa.storeKvQ8(k.ptr + l * T * kv_dim * 2, v.ptr + l * T * kv_dim * 2, k8.ptr + l * lb, ks.ptr + l * sb,
                         v8.ptr + l * lb, vs.ptr + l * sb, pos, 0, T, kv_dim, max_ctx, cx.stream.s)

    ms = cx.timed(run, steps, warmup) / L
    for bb in (k, v, k8, v8, ks, vs, pos):
        bb.free()
    per_token = 2 * kv_dim * 2 + 2 * kv_dim + 2 * (kv_dim // 32) * 2
    gbs = T * per_token / (ms * 1e-3) / 1e9
    return {"config": "int8 KV append (storeKvQ8Kernel)", "T": T, "heads": f"{Hkv}kv d{d}",
            "us_per_layer": round(ms * 1e3, 3), "bytes_per_layer": T * per_token, "GBps": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


# The reference's GEMM bench shapes (test_prefill_gemm.cu:40-42): kind code, K, N, what
GEMM_CASES = [(3, 4096, 14336, "8B ffn_gate Q4_K"), (5, 14336, 4096, "8B ffn_down Q6_K"),
              (1, 5120, 27648, "32B ffn_gate Q2_K"), (2, 27648, 5120, "32B ffn_down Q3_K")]
KQ_LAYOUT = {1: (84, 256, (80, 82)), 2: (110, 256, (108,)), 3: (144, 256, (0, 2)), 4: (176, 256, (0, 2)),
             5: (210, 256, (208,)), 6: (34, 32, (0,))}


def gemm_config(cx, kind, K, N, what, steps, warmup):
    """Prefill projection GEMM (friday_gemm_q8) at T = 512: random K-quant blocks with fp16
    scales in [1e-3, 1e-2], random int8 activations; fp16 MFMA utilisation and weight bytes."""
    import numpy as np

    fa = cx.fa
    T = 512
    bb, vals, offs = KQ_LAYOUT[kind]
    rng = np.random.default_rng(kind)
    W = rng.integers(0, 256, size=(N, K // vals, bb), dtype=np.uint8)
    for off in offs:
        W[:, :, off:off + 2] = rng.uniform(1e-3, 1e-2, size=(N, K // vals)).astype(np.float16).view(
            np.uint8).reshape(N, K // vals, 2)
    dW = fa.DeviceBuffer.from_array(W.reshape(N, -1))
    wbytes = W.nbytes
    del W
    xq, xd = fa.DeviceBuffer(T * K), fa.DeviceBuffer.from_array(np.full((T, K // 32), 0.01, np.float32))
    cx.fill(xq, T * K // 2, 13)
    Y = fa.DeviceBuffer(T * N * 2)
    fa.gemmQ8Reserve(T, K, N, cx.stream.s)  # K-split workspace, sized before capture (engine init)
    ms = cx.timed(lambda: fa.gemmQ8(kind, dW, xq, xd, T, K, N, Y, N, cx.stream.s), steps, warmup)
    for b in (dW, xq, xd, Y):
        b.free()
    flops = 2.0 * T * K * N
    tf = flops / (ms * 1e-3) / 1e12
    return {"config": "prefill projection GEMM", "what": what, "T": T, "K": K, "N": N, "us": round(ms * 1e3, 1),
            "tflops": round(tf, 1), "mfma_utilisation": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
            "weight_MB": round(wbytes / 1e6, 1)}


# Decode GEMVs (friday_gemv_q8): the attention O-projection of Qwen2.5-32B (transformer.cpp:
# 1057-1059) and the 8B ffn_down; kind code, K, N, what
GEMV_CASES = [(3, 5120, 5120, "32B attn_output Q4_K"), (5, 14336, 4096, "8B ffn_down Q6_K")]


def gemv_config(cx, kind, K, N, what, steps, warmup):
    """One int8-activation GEMV per layer over layer-distinct weights (rotated beyond the MALL):
    HBM bytes = the weight rows; us per layer and GB/s against the 8 TB/s peak."""
    import numpy as np

    fa = cx.fa
    bb, vals, offs = KQ_LAYOUT[kind]
    rng = np.random.default_rng(kind)
    W = rng.integers(0, 256, size=(N, K // vals, bb), dtype=np.uint8)
    for off in offs:
        W[:, :, off:off + 2] = rng.uniform(1e-3, 1e-2, size=(N, K // vals)).astype(np.float16).view(
            np.uint8).reshape(N, K // vals, 2)
    W = W.reshape(N, -1)
    wb = W.nbytes
    L = max(2, -(-2 * MALL_BYTES // wb))
    dW = fa.DeviceBuffer(L * wb)
    for l in range(L):
        dW.upload(W, l * wb)
    del W
    xq = fa.DeviceBuffer(K)
    cx.fill(xq, K // 2, 17)
    xd = fa.DeviceBuffer.from_array(np.full(K // 32, 0.01, np.float32))
    y = fa.DeviceBuffer(N * 2)
    ms = cx.timed(lambda: [fa.gemvQ8(kind, dW.ptr + l * wb, xq, xd, K, N, y, cx.stream.s) for l in range(L)],
                  steps, warmup) / L
    for b in (dW, xq, xd, y):
        b.free()
    gbs = wb / (ms * 1e-3) / 1e9
    return {"config": "decode GEMV (int8 activations)", "what": what, "K": K, "N": N, "layers": L,
            "us_per_layer": round(ms * 1e3, 2), "weight_MB": round(wb / 1e6, 2), "GBps": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def layer_block_config(cx, S, L, steps, warmup, fused=False):
    """The attention block of one decode layer at the headline shape, as gpuLayerFused runs it
    (transformer.cpp:1046-1059): decode step (RoPE + append + attention), quantizeQ8 of the
    output, O-projection gemvQ8 (Q4_K, 5120 x 5120) with the residual in place; 64 layers,
    one HIP graph. HBM bytes per layer = K/V of the context + the O-projection weights.
    fused: the quantisation runs in the decode step's merge epilogue (friday_attn_decode_step_quant)."""
    import numpy as np

    fa = cx.fa
    Hq, Hkv, d = 40, 8, 128
    H = Hq * d
    dl = DecodeLayers(cx, S, L, Hq, Hkv, d)
    bb, vals, offs = KQ_LAYOUT[3]
    rng = np.random.default_rng(3)
    W = rng.integers(0, 256, size=(H, H // vals, bb), dtype=np.uint8)
    for off in offs:
        W[:, :, off:off + 2] = rng.uniform(1e-3, 1e-2, size=(H, H // vals)).astype(np.float16).view(
            np.uint8).reshape(H, H // vals, 2)
    W = W.reshape(H, -1)
    wb = W.nbytes
    dW = fa.DeviceBuffer(L * wb)
    for l in range(L):
        dW.upload(W, l * wb)
    x = fa.DeviceBuffer(L * H * 2)
    cx.fill(x, L * H, 21)
    xq, xd = fa.DeviceBuffer(H), fa.DeviceBuffer(H // 32 * 4)

    def run():
        for l in range(L):
            q, kn, vn, kc, vc, out = dl.ptrs(l)
            if fused:
                fa.decodeStepQuant(q, kn, vn, kc, vc, out, xq, xd, dl.pos, 0, S, Hq, Hkv, d, dl.table, 1, dl.ws,
                                   cx.stream.s)
            else:
                fa.decodeStep(q, kn, vn, kc, vc, out, dl.pos, 0, S, Hq, Hkv, d, dl.table, 1, dl.ws, cx.stream.s)
                fa.quantizeQ8Rows(out, 1, H, xq, xd, cx.stream.s)
            xl = x.ptr + l * H * 2
            fa.gemvQ8(fa.Q4_K, dW.ptr + l * wb, xq, xd, H, H, xl, cx.stream.s, res=xl)

    ms = cx.timed(run, steps, warmup)
    dl.free()
    for b in (dW, x, xq, xd):
        b.free()
    us = ms * 1e3 / L
    hbm = 2 * S * Hkv * d * 2 + wb
    return {"config": "decode layer attention block" + (" (quantize fused into the step)" if fused else ""), "ctx": S, "layers": L, "heads": f"{Hq}q/{Hkv}kv d{d}",
            "o_proj": f"Q4_K {H}x{H}", "us_per_layer": round(us, 2), "hbm_MB_per_layer": round(hbm / 1e6, 1),
            "GBps": round(hbm / (us * 1e-6) / 1e9, 1), "hbm_frac": round(hbm / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def q8_config(cx, S, L, steps, warmup):
    """int8 KV (FRIDAY --kv q8) at the headline shape: one friday_attn_decode_step_q8 per layer."""
    import numpy as np

    fa = cx.fa
    Hq, Hkv, d = 40, 8, 128
    kv_dim = Hkv * d
    lb, sb = S * kv_dim, S * (kv_dim // 32) * 2  # int8 values and fp16 scales per layer
    k8, v8 = fa.DeviceBuffer(L * lb), fa.DeviceBuffer(L * lb)
    ks, vs = fa.DeviceBuffer(L * sb), fa.DeviceBuffer(L * sb)
    cx.fill(k8, L * lb // 2, 11)  # random bytes as int8 codes
    cx.fill(v8, L * lb // 2, 12)
    cx.fill(ks, L * sb // 2, 13, 0.02)
    cx.fill(vs, L * sb // 2, 14, 0.02)
    rng = np.random.default_rng(3)
    f16 = lambda shape: rng.standard_normal(shape, dtype=np.float32).astype(np.float16).view(np.uint16)
    q, kn, vn = (fa.DeviceBuffer.from_array(f16((L, n))) for n in (Hq * d, kv_dim, kv_dim))
    out = fa.DeviceBuffer(L * Hq * d * 2)
    table = fa.DeviceBuffer(fa.rope_table_bytes(S, d))
    fa.rope_table_upload(table, S, d, 1e6)
    pos = fa.DeviceBuffer.from_array(np.array([S - 1], np.int32))
    ws = fa.DeviceBuffer(fa.splitAttentionWorkspaceBytes(Hq, S))
    fa.decodeWorkspaceInit(ws, stream=cx.stream.s)
    cx.stream.synchronize()

    def step():
        for l in range(L):
            fa.decodeStepQ8(q.ptr + l * Hq * d * 2, kn.ptr + l * kv_dim * 2, vn.ptr + l * kv_dim * 2,
                            k8.ptr + l * lb, ks.ptr + l * sb, v8.ptr + l * lb, vs.ptr + l * sb,
                            out.ptr + l * Hq * d * 2, pos, 0, S, Hq, Hkv, d, table, 1, ws, cx.stream.s)

    ms = cx.timed(step, steps, warmup)
    for b in (k8, v8, ks, vs, q, kn, vn, out, table, pos, ws):
        b.free()
    us = ms * 1e3 / L
    nbytes = 2 * (lb + sb)
    return {"config": "3 with int8 KV (--kv q8)", "decode_form": decode_form(), "ctx": S, "layers": L, "heads": f"{Hq}q/{Hkv}kv d{d}",
            "us_per_layer_step": round(us, 3), "kv_bytes_per_layer": nbytes, "kv_GBps": round(nbytes / us / 1e3, 1),
            "hbm_frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "tokens_per_s": round(1e6 / (us * L), 2)}


def paged_config(cx, steps, warmup, L=8):
    """benchmark config 5: 16 sequences, S ~ U[256, 16k], 16-token pages in a permuted pool, one
    launch per layer; L layers (each its own pool, 3.7 GB together, beyond the Infinity Cache)
    in one graph replay, so the figure is per layer-step, as for the headline."""
    import numpy as np

    fa = cx.fa
    B, Hq, Hkv, d, P = 16, 40, 8, 128, 16
    kv_dim = Hkv * d
    rng = np.random.default_rng(5)
    lens = rng.integers(256, 16384 + 1, B).astype(np.int32)
    max_seq = 16384
    nblk = [(int(s) + P - 1) // P for s in lens]
    perm = rng.permutation(sum(nblk)).astype(np.int32)
    table = np.full((B, max_seq // P), -1, np.int32)
    at = 0
    for b in range(B):
        table[b, :nblk[b]] = perm[at:at + nblk[b]]
        at += nblk[b]
    pool_rows = sum(nblk) * P
    pool_b = pool_rows * kv_dim * 2
    kp, vp = fa.DeviceBuffer(L * pool_b), fa.DeviceBuffer(L * pool_b)
    cx.fill(kp, L * pool_rows * kv_dim, 8)
    cx.fill(vp, L * pool_rows * kv_dim, 9)
    bufs = [fa.DeviceBuffer.from_array(a) for a in (table, lens)]
    qb, kvb = B * Hq * d * 2, B * kv_dim * 2
    q = fa.DeviceBuffer(L * qb)
    kn, vn, out = fa.DeviceBuffer(L * kvb), fa.DeviceBuffer(L * kvb), fa.DeviceBuffer(L * qb)
    for bb, n in ((q, L * B * Hq * d), (kn, L * B * kv_dim), (vn, L * B * kv_dim)):
        cx.fill(bb, n, 10)
    rope = fa.DeviceBuffer(fa.rope_table_bytes(max_seq, d))
    fa.rope_table_upload(rope, max_seq, d, 1e6)
    ws = fa.DeviceBuffer(fa.pagedWorkspaceBytes(B, Hq, max_seq))
    fa.decodeWorkspaceInit(ws, stream=cx.stream.s)

    def run():
        for l in range(L):
            fa.pagedDecodeStep(q.ptr + l * qb, kn.ptr + l * kvb, vn.ptr + l * kvb, kp.ptr + l * pool_b,
                               vp.ptr + l * pool_b, out.ptr + l * qb, bufs[0], table.shape[1], bufs[1], B, max_seq,
                               Hq, Hkv, d, rope, 1, ws, cx.stream.s)

    ms = cx.timed(run, steps, warmup) / L
    for bb in (kp, vp, q, kn, vn, out, rope, ws, *bufs):
        bb.free()
    kv_bytes = float(lens.sum()) * kv_dim * 2 * 2
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    return {"config": "5: paged multi-sequence step", "sequences": B, "sum_ctx": int(lens.sum()), "layers": L,
            "pool_MiB_per_layer": round(2 * pool_b / 2**20, 1), "us_per_layer_step": round(ms * 1e3, 2),
            "kv_GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "tokens_per_s": round(B / (ms * 1e-3), 0)}


def probe_configs(cx, steps, warmup, L=64):
    """Read-pattern probes (bench_kit): the K/V access patterns of the decode kernels without
    their arithmetic, 256 workgroups per launch, one launch per layer over 64 layers of
    32768-row caches (cold: 8 GiB), timed like the headline (graph replays). They bound what a
    decode launch of that pattern can stream; the empty kernel gives the launch floor."""
    bk, fa = cx.bk, cx.fa
    bk.fabk_probe_count.restype = C.c_int
    bk.fabk_probe_name.restype = C.c_char_p
    bk.fabk_probe_name.argtypes = [C.c_int]
    bk.fabk_probe_row_bytes.argtypes = [C.c_int]
    bk.fabk_probe_launch.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
    S = 32768
    lb = S * 2048
    K, V, out = fa.DeviceBuffer(L * lb), fa.DeviceBuffer(L * lb), fa.DeviceBuffer(4096)
    recs = []
    try:
        for v in range(-1, bk.fabk_probe_count()):
            rowb = bk.fabk_probe_row_bytes(v)
            layer = S * rowb

            def run(v=v, layer=layer):
                for l in range(L):
                    if bk.fabk_probe_launch(v, C.c_void_p(K.ptr + l * layer), C.c_void_p(V.ptr + l * layer),
                                            C.c_void_p(out.ptr), cx.stream.s) != 0:
                        raise RuntimeError("probe launch failed")

            us = cx.timed(run, steps, warmup) * 1e3 / L
            rec = {"config": "probe: " + bk.fabk_probe_name(v).decode(), "us_per_launch": round(us, 3)}
            if rowb:
                gbs = 2 * layer / (us * 1e-6) / 1e9
                rec.update({"bytes_per_launch": 2 * layer, "GBps": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
            recs.append(rec)
            log(f"[bench] {rec}")
    finally:
        for b in (K, V, out):
            b.free()
    return recs


STAMP_NAMES = ("entry", "ctx_known", "q_ready", "stream_end", "combine_done", "partials_stored", "counted",
               "merged")


def stamps_config(cx, name, S, L, Hq, Hkv, d, steps, warmup):
    """Phase timestamps of the decode step kernel (the stamps build: libfriday_attn_stamps.so,
    the product kernels plus a 100 MHz real-time stamp per phase edge and workgroup). Replays
    the config's graph, then reads the stamps of the last launch (the last layer of the last
    replay) and reports, per phase, the spread over the workgroups in us after the earliest
    entry."""
    import numpy as np

    fa = cx.fa
    lib = fa.load()
    lib.friday_attn_debug_stamps.argtypes = [C.c_void_p]
    nwg_max = 1 << 14
    buf = fa.DeviceBuffer(nwg_max * 32 * 8)
    buf.upload(np.zeros(nwg_max * 32, np.uint64))
    if lib.friday_attn_debug_stamps(C.c_void_p(buf.ptr)) != 0:
        raise RuntimeError("friday_attn_debug_stamps failed")
    dl = DecodeLayers(cx, S, L, Hq, Hkv, d)
    ms = dl.measure(steps, warmup, "step")
    dl.free()
    lib.friday_attn_debug_stamps(None)
    st = buf.download((nwg_max, 32), np.uint64).astype(np.int64)
    buf.free()
    live = st[:, 0] > 0
    st = st[live]
    t0 = st[:, 0].min()
    phases = {}
    for k, nm in enumerate(STAMP_NAMES):
        has = st[:, k] > 0
        if has.any():
            v = (st[has, k] - t0) / 100.0
            phases[nm] = {"wgs": int(has.sum()), "min": round(float(v.min()), 2),
                          "median": round(float(np.median(v)), 2), "max": round(float(v.max()), 2)}
    tiles = []
    for i in range(16):
        has = st[:, 8 + i] > 0
        if has.any():
            tiles.append(round(float(np.median((st[has, 8 + i] - t0) / 100.0)), 2))
    info = st[:, 26]
    nsp, mk = (info >> 12) & 0xFFF, (info >> 24) - 1
    xcc = st[:, 24] & 0xF
    ends = np.where(st[:, 7] > 0, st[:, 7], np.where(st[:, 5] > 0, st[:, 5], st[:, 4]))
    span = (ends.max() - t0) / 100.0
    # per-workgroup durations of the phases (median over workgroups)
    dur = lambda a, b: round(float(np.median((st[:, b] - st[:, a])[(st[:, a] > 0) & (st[:, b] > 0)] / 100.0)), 2)
    rec = {"config": f"stamps: {name}", "ctx": S, "layers": L, "heads": f"{Hq}q/{Hkv}kv d{d}",
           "us_per_layer_step_stamps_build": round(ms * 1e3 / L, 3), "workgroups": int(live.sum()),
           "nsp": int(nsp.max()), "launch_span_us": round(span, 2), "phases_us_after_first_entry": phases,
           "wave0_tile_landed_median_us": tiles,
           "median_durations_us": {"entry_to_ctx": dur(0, 1), "ctx_to_first_tile": dur(1, 8),
                                   "entry_to_q_ready": dur(0, 2), "stream_end_to_combine": dur(3, 4),
                                   "combine_to_partials_stored": dur(4, 5), "partials_to_counted": dur(5, 6),
                                   "counted_to_merged": dur(6, 7)},
           "mergers": int((mk >= 0).sum())}
    # the XCDs each group's workgroups ran on (grid x = the groups, so group = linear id % groups)
    groups = Hkv * -(-(Hq // Hkv) // 16)
    lin = np.nonzero(live)[0]
    rec["xcds_per_group"] = [len(set(xcc[(lin % groups) == g].tolist())) for g in range(groups)]
    log(f"[bench] stamps {name}: span {span:.2f} us, {json.dumps(phases)}")
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--stat-replays", type=int, default=100,
                    help="further replays timed one by one for the median / p10 / p90 of a step")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--calibrate", action="store_true",
                    help="only copy 1 GiB three times with the bench-kit streaming copy (one 16-byte load and "
                         "store per element): rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of this run give the "
                         "counters' reading for a known 1 GiB read + 1 GiB write")
    ap.add_argument("--config", choices=("headline", "all", "others", "short", "prefill", "paged", "q8", "gemm", "layer", "append", "stamps", "probe"), default="headline",
                    help="headline: the driver's one line; all/others: also (only) the other benchmark configs; "
                         "short: configs 1 and 2 only")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): the KV-cache path is built and measured "
              f"on a single MI355X; how it would shard is a design note, not a run.", file=sys.stderr)
        sys.exit(2)

    if args.config == "stamps":  # the stamps build of the library, loaded instead of the product one
        os.environ["FRIDAY_ATTN_LIB"] = os.path.join(ROOT, "friday-inference-engine_amd", "lib",
                                                     "libfriday_attn_stamps.so")
    cx = Ctx()
    if args.calibrate:
        cx.bk.fabk_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        n = 1 << 30
        a, b = cx.fa.DeviceBuffer(n), cx.fa.DeviceBuffer(n)
        for _ in range(3):
            cx.bk.fabk_copy(a.ptr, b.ptr, n, cx.stream.s)
        cx.stream.synchronize()
        log(f"[bench] calibration: copied {n} bytes x3")
        return
    if args.config in ("headline", "all"):
        print(json.dumps(headline(cx, args)), flush=True)
    if args.config in ("all", "others", "short"):
        emit = lambda rec: print(json.dumps(rec), flush=True)
        emit(decode_config(cx, "1: Qwen2.5-0.5B layer", 513, 24, 14, 2, 64, args.steps, args.warmup, False))
        for S in (1024, 4096, 8192):
            for cold in (True, False):
                emit(decode_config(cx, "2: 32q/8kv x 32 layers", S, 32, 32, 8, 128, args.steps, args.warmup, cold))
    if args.config in ("all", "others"):
        emit(decode_config(cx, "3: 40q/8kv x 64 layers", 16384, 64, 40, 8, 128, args.steps, args.warmup, False))
        for p0 in (0, 1024, 2048, 4096, 7680):
            emit(prefill_config(cx, p0, args.steps, args.warmup))
        for p0 in (0, 7680):
            emit(prefill_config(cx, p0, args.steps, args.warmup, q8=True))
        for p0 in (0, 7680):
            emit(prefill_config(cx, p0, args.steps, args.warmup, bf16=True))
        emit(paged_config(cx, args.steps, args.warmup))
        for T in (1, 512):
            emit(append_config(cx, T, args.steps, args.warmup))
        for T in (1, 512):
            emit(append_q8_config(cx, T, args.steps, args.warmup))
        for p0 in (0, 7680):
            emit(prefill_vs_decode_config(cx, p0, args.steps, args.warmup))
        emit(q8_config(cx, 32768, 64, args.steps, args.warmup))
        for case in GEMM_CASES:
            emit(gemm_config(cx, *case, args.steps, args.warmup))
        for case in GEMV_CASES:
            emit(gemv_config(cx, *case, args.steps, args.warmup))
        emit(layer_block_config(cx, 32768, 64, args.steps, args.warmup))
        emit(layer_block_config(cx, 32768, 64, args.steps, args.warmup, fused=True))
    if args.config == "q8":
        print(json.dumps(q8_config(cx, 32768, 64, args.steps, args.warmup)), flush=True)
    if args.config == "append":
        for T in (1, 512):
            print(json.dumps(append_config(cx, T, args.steps, args.warmup)), flush=True)
        for T in (1, 512):
            print(json.dumps(append_q8_config(cx, T, args.steps, args.warmup)), flush=True)
    if args.config == "paged":
        print(json.dumps(paged_config(cx, args.steps, args.warmup)), flush=True)
    if args.config == "prefill":
        for p0 in (0, 1024, 2048, 4096, 7680):
            print(json.dumps(prefill_config(cx, p0, args.steps, args.warmup)), flush=True)
        for p0 in (0, 2048, 7680):
            print(json.dumps(prefill_config(cx, p0, args.steps, args.warmup, q8=True)), flush=True)
        for p0 in (0, 1024, 2048, 4096, 7680):
            print(json.dumps(prefill_config(cx, p0, args.steps, args.warmup, bf16=True)), flush=True)
        for p0 in (0, 7680):
            print(json.dumps(prefill_vs_decode_config(cx, p0, args.steps, args.warmup)), flush=True)
    if args.config == "layer":
        print(json.dumps(layer_block_config(cx, 32768, 64, args.steps, args.warmup)), flush=True)
        print(json.dumps(layer_block_config(cx, 32768, 64, args.steps, args.warmup, fused=True)), flush=True)
    if args.config == "probe":
        for rec in probe_configs(cx, args.steps, args.warmup):
            print(json.dumps(rec), flush=True)
    if args.config == "stamps":
        for rec in (stamps_config(cx, "3: 40q/8kv x 64 layers", 32768, 64, 40, 8, 128, args.steps, args.warmup),
                    stamps_config(cx, "2: 32q/8kv x 32 layers", 1024, 32, 32, 8, 128, args.steps, args.warmup),
                    stamps_config(cx, "ctx 16, 40q/8kv x 64 layers", 16, 64, 40, 8, 128, args.steps, args.warmup)):
            print(json.dumps(rec), flush=True)
    if args.config == "gemm":
        for case in GEMM_CASES:
            print(json.dumps(gemm_config(cx, *case, args.steps, args.warmup)), flush=True)
        for case in GEMV_CASES:
            print(json.dumps(gemv_config(cx, *case, args.steps, args.warmup)), flush=True)


if __name__ == "__main__":
    main()
