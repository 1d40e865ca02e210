"""Benchmark of the large-head-dim fused attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config N] [--head-dim D]

A "step" is one call of the hot path (atn_attention_fwd_ex, asynchronous,
on one HIP stream) over one batch of synthetic input already resident in
HBM.  The headline workload (`value`) is BASELINE config 2: fp32 SDPA,
batch 1, 4 heads, len_q = len_k = 64, head_dim 2048, Q/K/V iid N(0,1).

With no --config, the same line also carries `per_config`: configs 1, 3, 4
and 5, the config-2 head_dim sweep (512 / 4096 / 8192) and two fp32 shapes
beyond the single-launch window (the reference's own long test shape, on the
flash kernel, and a head_dim-2048 one, on the split-D pipeline), each timed
the same way, checked against the CPU oracle on sampled rows of the first, a
middle and the last head, and with its own CPU baseline.  --config N (and
--head-dim D) print one config's line only (for profiling).

Printed: ONE JSON line.  `value` is the algorithmic HBM throughput
(Q + K + V read once + O written once, bytes / second) of the whole job;
TFLOP/s use 4*B*H*Lq*Lk*D.  `roofline` times the dominant kernel with HIP
events on the stream it runs on; `cpu_baseline` times the CPU oracle (the
restatement of the reference's single-threaded attention_cpu,
final/attention.cu:228-283, and its RoPE / sinusoidal siblings) on a bounded
sample of the same workload.  The exit status is 1 when any sampled output
misses its tolerance (fp32: abs > 1e-4 AND rel > 1e-4; bf16: rel 2e-2).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for sub in ("accelerated-final-project_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
# fp32 work carried as three fp16 MFMA products (the hi + lo split)
F32_SPLIT_PEAK_TFLOPS = BF16_PEAK_TFLOPS / 3
MALL_FLUSH_MIB = 512  # > the 256 MiB MALL: a copy this large evicts it

# HBM traffic per launch of the dominant kernel, measured with rocprofv3
# FETCH_SIZE / WRITE_SIZE and scaled by a known-size device copy; keyed by
# (config, head_dim), with the profile that holds the counts.
MEASURED_TRAFFIC = {
    (2, 2048): ((11672 + 3080) * 1024, "profiles/fused_small_cfg2_traffic.md"),
    (3, 8192): ((23758 + 6224) * 1024, "profiles/fused_small_cfg3_kernel_trace.md"),
}

# (name, dtype, B, H, Lq, Lk, D, pe, sigma)
CONFIGS = {
    1: ("cfg1 fp32 SDPA (1,1,4,4,8)", "f32", 1, 1, 4, 4, 8, "none", 1.0),
    2: ("cfg2 fp32 SDPA (1,4,64,64,2048)", "f32", 1, 4, 64, 64, 2048, "none", 1.0),
    3: ("cfg3 bf16 SDPA cross (1,4,32,128,8192)", "bf16", 1, 4, 32, 128, 8192, "none", 1.0),
    4: ("cfg4 bf16 RoPE rotate-half (8,8,1024,1024,4096)", "bf16", 8, 8, 1024, 1024, 4096,
        "rope_half", 1.0),
    5: ("cfg5 bf16 sinusoidal cross (4,16,256,2048,1024)", "bf16", 4, 16, 256, 2048, 1024,
        "sinusoidal", 0.5),
}
SWEEP_D = (512, 4096, 8192)
# beyond the single-launch window, measured beside the configs: the
# reference's own long-sequence test shape (final/attention.cu:522; the flash
# kernel) in fp32 and in bf16, and a head_dim-2048 fp32 shape of the same
# length (the split-D pipeline)
LONG = {
    "ref_long_f32": ("fp32 SDPA, the reference's long test shape (4,32,512,512,128)", "f32", 4, 32,
                     512, 512, 128, "none", 1.0),
    "ref_long_bf16": ("bf16 SDPA at the reference's long test shape (4,32,512,512,128)", "bf16", 4,
                      32, 512, 512, 128, "none", 1.0),
    "long_f32_D2048": ("fp32 SDPA (1,4,512,512,2048)", "f32", 1, 4, 512, 512, 2048, "none", 1.0),
}

F32_ABS, F32_REL, BF16_REL = 1e-4, 1e-4, 2e-2
PATH_NAMES: dict = {}  # atn_attention_path_ex code -> kernel(s) per step, filled in main


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=0, choices=[0] + sorted(CONFIGS),
                    help="one config only (0 = headline config 2 plus every other config)")
    ap.add_argument("--head-dim", type=int, default=0, help="override D (config-2 sweep)")
    ap.add_argument("--shape", default="", metavar="B,H,LQ,LK,D",
                    help="time this shape instead (for profiling one kernel or path)")
    ap.add_argument("--dtype", default="f32", choices=["f32", "bf16"],
                    help="element type of --shape")
    ap.add_argument("--pe", default="none", choices=["none", "rope_half", "sinusoidal"],
                    help="positional encoding of --shape (sinusoidal inputs at sigma 0.5)")
    ap.add_argument("--no-flash", action="store_true",
                    help="keep calls off the flash kernel (atn_tuning.no_flash)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU-oracle sample time of the headline (0 = skip every CPU baseline)")
    ap.add_argument("--cpu-seconds-other", type=float, default=3.0,
                    help="CPU-oracle sample time of each per_config entry")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="also run 5 device-to-device copies of MIB MiB (the HIP runtime's "
                         "copy kernel), a known-size reference for rocprofv3 traffic counters")
    return ap.parse_args()


def host_info():
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    libc = platform.libc_ver()
    return {"cpu_model": model or platform.processor() or platform.machine(),
            "nproc_usable": usable, "cpu_count": os.cpu_count(),
            "glibc": f"{libc[0]} {libc[1]}".strip()}


def make_inputs(dtype, B, H, Lq, Lk, D, sigma, seed):
    """Seeded N(0, sigma) inputs generated on the host with numpy PCG64,
    uploaded once (they stay resident for every step).  Returns the device
    arrays and float32 host copies of exactly the values the kernel sees."""
    import hip_rt
    rng = np.random.default_rng(seed)
    dev, host = [], []
    for shape in ((B, H, Lq, D), (B, H, Lk, D), (B, H, Lk, D)):
        x = rng.standard_normal(shape, dtype=np.float32)
        if sigma != 1.0:
            x *= np.float32(sigma)
        if dtype == "f32":
            d = hip_rt.DeviceArray.from_numpy(x, "f32")
        else:
            bits = hip_rt.f32_to_bf16_bits(x)
            d = hip_rt.DeviceArray.from_numpy(bits, "bf16")
            x = hip_rt.bf16_bits_to_f32(bits)
        dev.append(d)
        host.append(x)
    return dev, host


def pe_desc(am, pe):
    if pe == "none":
        return None
    if pe == "rope_half":
        return am.make_pe("rope", pairing="half")
    if pe == "sinusoidal":
        return am.make_pe("sinusoidal")
    raise ValueError(pe)


def oracle_rows(cfg, host, bh, r0, r1, nthreads=1):
    """CPU oracle output rows [r0, r1) of head bh (flattened b*H + h) as
    float32 [r1 - r0, D].  Only that head's Q, K, V are handed over, so the
    positions (row index within the head) are those of the full tensors."""
    import oracle
    _, _, B, H, Lq, Lk, D, pe, _ = cfg
    b, h = divmod(bh, H)
    Q, K, V = (np.ascontiguousarray(t[b:b + 1, h:h + 1]) for t in host)
    rows = (r0, r1)
    if pe == "none":
        out = oracle.attention(Q, K, V, rows=rows, nthreads=nthreads)
    elif pe == "rope_half":
        c, s = oracle.rope_cache(max(Lq, Lk), D)
        out = oracle.attention_rope(Q, K, V, c, s, pairing="half", rows=rows, nthreads=nthreads)
    else:
        st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
        out = oracle.attention_sinusoidal(Q, K, V, st, ct, rows=rows, nthreads=nthreads)
    return out.reshape(Lq, D)[r0:r1]


def sampled_check(cfg, host, got_rows_fn):
    """Sampled-row parity: rows of the first, a middle and the last head --
    the first 4, 4 from the middle and the last 8 rows of each (the last row
    tile included) -- against the CPU oracle.  Returns a summary dict."""
    name, dtype, B, H, Lq, Lk, D, pe, _ = cfg
    BH = B * H
    heads = sorted({0, BH // 2, BH - 1})
    spans = sorted({(0, min(4, Lq)), (Lq // 2, min(Lq, Lq // 2 + 4)), (max(0, Lq - 8), Lq)})
    nfail, maxabs, num, den, nrows = 0, 0.0, 0.0, 0.0, 0
    worst_el = 0.0
    for bh in heads:
        for r0, r1 in spans:
            if r1 <= r0:
                continue
            ref = oracle_rows(cfg, host, bh, r0, r1, nthreads=8).astype(np.float64)
            got = got_rows_fn(bh, r0, r1).astype(np.float64)
            err = np.abs(got - ref)
            maxabs = max(maxabs, float(err.max()))
            nrows += r1 - r0
            if dtype == "f32":
                bad = (err > F32_ABS) & (err / (np.abs(ref) + 1e-8) > F32_REL)
            else:
                rms = float(np.sqrt(np.mean(ref * ref)))
                bad = (err > BF16_REL * np.abs(ref)) & (err > BF16_REL * rms)
                worst_el = max(worst_el, float((err / max(rms, 1e-30)).max()))
                num += float(np.sum(err * err))
                den += float(np.sum(ref * ref))
            nfail += int(bad.sum()) + int((~np.isfinite(got)).sum())
    out = {"rows_checked": nrows, "heads_checked": heads, "max_abs": maxabs, "fails": nfail}
    if dtype == "f32":
        out["bar"] = "abs > 1e-4 AND rel > 1e-4 fails (vs the fp32 oracle)"
        out["ok"] = nfail == 0
    else:
        nrel = (num ** 0.5) / max(den ** 0.5, 1e-30)
        out["normwise_rel"] = nrel
        out["bar"] = ("err > 2e-2*|ref| AND err > 2e-2*rms(ref) fails; normwise <= 2e-2 "
                      "(vs the fp32 oracle on the bf16-rounded inputs)")
        out["ok"] = nfail == 0 and nrel <= BF16_REL
    return out


def cpu_baseline(cfg, host, target_s):
    """Single-threaded CPU oracle on a bounded row sample of the workload;
    returns (value in GB/s of the same algorithmic bytes, sample text).
    Rows are taken head by head (the RoPE / sinusoidal oracles encode a
    head's K once per head, as the reference's CPU paths do)."""
    name, dtype, B, H, Lq, Lk, D, pe, _ = cfg
    rows_total = B * H * Lq
    es = 4 if dtype == "f32" else 2
    alg_bytes = (2 * B * H * Lq * D + 2 * B * H * Lk * D) * es

    def run_head_rows(bh, n):
        oracle_rows(cfg, host, bh, 0, n, nthreads=1)

    # cost of one head's first row (includes the per-head encoding of K)
    t0 = time.perf_counter()
    run_head_rows(0, 1)
    t1 = max(time.perf_counter() - t0, 1e-6)
    if t1 * Lq <= target_s:
        # whole heads, as many as fit the target (all of them if cheap)
        t0 = time.perf_counter()
        run_head_rows(0, Lq)
        th = max(time.perf_counter() - t0, 1e-6)
        nheads = int(max(1, min(B * H, target_s / th)))
        reps = 1
        t0 = time.perf_counter()
        for bh in range(nheads):
            run_head_rows(bh, Lq)
        el = time.perf_counter() - t0
        if nheads == B * H:
            reps = int(max(1, target_s / max(el, 1e-6)))
            if reps > 1:
                t0 = time.perf_counter()
                for _ in range(reps):
                    for bh in range(nheads):
                        run_head_rows(bh, Lq)
                el = time.perf_counter() - t0
        nrows = nheads * Lq
    else:
        # part of one head
        nrows = int(max(1, min(Lq, target_s / t1)))
        reps = 1
        t0 = time.perf_counter()
        run_head_rows(0, nrows)
        el = time.perf_counter() - t0
    frac = nrows / rows_total
    sec_per_job = el / reps / frac
    sample = (f"{nrows}/{rows_total} query rows x {reps} rep(s) of {name}, single thread; "
              f"{el:.2f} s measured, whole job = {sec_per_job * 1e3:.2f} ms"
              + (" (extrapolated linearly from the sample)" if frac < 1 else ""))
    return alg_bytes / sec_per_job / 1e9, sec_per_job * 1e3, sample


def run_config(am, hip_rt, cfg, steps, warmup, seed, cold):
    """Times one config: `steps` calls captured as one HIP graph and replayed
    (HIP events on the call's stream), and, with `cold`, the median single
    call between events of its own, with and without the 256 MiB MALL
    flushed before it (a 512 MiB device copy outside the events).  Returns
    the timing dict, the host inputs and a row reader of the final output."""
    name, dtype, B, H, Lq, Lk, D, pe, sigma = cfg
    (q, k, v), host = make_inputs(dtype, B, H, Lq, Lk, D, sigma, seed)
    out = hip_rt.DeviceArray((B, H, Lq, D), dtype)
    desc = pe_desc(am, pe)
    dcode = am.ATN_DTYPE_F32 if dtype == "f32" else am.ATN_DTYPE_BF16
    # a caller workspace is zero-filled once before its first use
    ws = hip_rt.DeviceArray((max(am.workspace_bytes(dcode, B, H, Lq, Lk, D, desc), 4) // 4,),
                            "f32", fill=0)
    stream = hip_rt.Stream()
    if desc is not None:
        st = am.lib().atn_prepare_pe_ex(desc, D, max(Lq, Lk))
        if st != 0:
            raise am.AtnError(st, "atn_prepare_pe_ex")

    def step():
        am.attention_ex(q, k, v, out, pe=desc, workspace=ws, stream=stream)

    for _ in range(warmup):
        step()
    hip_rt.synchronize()

    e0, e1 = hip_rt.Event(), hip_rt.Event()
    # eager: one Python-driven call per step (host-bound for small shapes)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    e1.synchronize()
    eager_ms = e0.elapsed_ms(e1) / steps

    def timed_graph(fn, extra=0):
        g = hip_rt.Graph(stream, fn)
        g.launch()  # warm replay
        stream.synchronize()
        hip_rt.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        g.launch()
        e1.record(stream)
        e1.synchronize()
        wall = time.perf_counter() - t0
        ms = e0.elapsed_ms(e1)
        trials = [ms]
        for _ in range(extra):  # further replays, after the timed region
            e0.record(stream)
            g.launch()
            e1.record(stream)
            e1.synchronize()
            trials.append(e0.elapsed_ms(e1))
        g.destroy()
        return ms, wall, trials

    # timed region: the K steps captured once as a HIP graph and replayed,
    # so the GPU runs them back to back with no host work in between; four
    # more replays give the median of five trials beside it
    ev_ms, wall, trials = timed_graph(lambda: [step() for _ in range(steps)], extra=4)
    st = am.lib().atn_sync_status_ex(ws.ptr, B, H, stream.handle)
    if st != 0:
        raise am.AtnError(st, f"device status after the timed region ({name})")
    res = {"ms_per_step": ev_ms / steps, "eager_ms": eager_ms, "wall_s": wall,
           "median5_ms_per_step": sorted(trials)[len(trials) // 2] / steps,
           "path": am.path(dcode, B, H, Lq, Lk, D, desc)}
    if cold:
        n = MALL_FLUSH_MIB << 20
        src = hip_rt.DeviceArray((n // 4,), "f32", fill=0)
        dst = hip_rt.DeviceArray((n // 4,), "f32")

        def bracketed(flush):
            # median over `steps` calls, each between two events of its own;
            # with `flush`, a MALL-sized device copy runs before each call,
            # outside its events (a difference of whole-run timings would
            # carry the copies' own spread, larger than a short kernel)
            evs = [(hip_rt.Event(), hip_rt.Event()) for _ in range(steps)]
            for b, e in evs:
                if flush:
                    hip_rt.copy_d2d_async(dst, src, n, stream)
                b.record(stream)
                step()
                e.record(stream)
            evs[-1][1].synchronize()
            t = sorted(b.elapsed_ms(e) for b, e in evs)
            for b, e in evs:
                b.destroy()
                e.destroy()
            return t[len(t) // 2]

        res["bracketed_ms_per_step"] = bracketed(False)
        res["cold_ms_per_step"] = bracketed(True)
        st = am.lib().atn_sync_status_ex(ws.ptr, B, H, stream.handle)
        if st != 0:
            raise am.AtnError(st, f"device status after the cold run ({name})")
        src.free()
        dst.free()
    if pe == "none":
        # the synchronous drop-in (the reference's host entry point: launch,
        # then wait for the device), host wall clock per call, median
        fn = am.attention_forward_optimized if dtype == "f32" else am.attention_forward_bf16
        for _ in range(3):
            fn(q, k, v, out)
        ts = []
        for _ in range(max(steps, 20)):
            t0 = time.perf_counter()
            fn(q, k, v, out)
            ts.append(time.perf_counter() - t0)
        res["dropin_sync_ms"] = sorted(ts)[len(ts) // 2] * 1e3
    hip_rt.synchronize()
    bits = out.numpy()

    def rows_fn(bh, r0, r1):
        return bits.reshape(B * H, Lq, D)[bh, r0:r1]

    stream.destroy()
    for t in (q, k, v, out, ws):
        t.free()
    return res, host, rows_fn


def cold_kernel(cfg, res):
    """Kernel-only time of one call with the MALL flushed: the cold
    event-bracketed median minus the events' own overhead, which is the
    bracketed median without the flush less the graph-replayed step time.
    Returns (ms, HBM fraction), or None without cold timings."""
    if "cold_ms_per_step" not in res:
        return None
    name, dtype, B, H, Lq, Lk, D, pe, _ = cfg
    es = 4 if dtype == "f32" else 2
    alg_bytes = (2 * B * H * Lq * D + 2 * B * H * Lk * D) * es
    overhead = max(0.0, res["bracketed_ms_per_step"] - res["ms_per_step"])
    ms = max(res["cold_ms_per_step"] - overhead, 1e-6)
    return ms, alg_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS


def summarize(cfg, res):
    name, dtype, B, H, Lq, Lk, D, pe, _ = cfg
    es = 4 if dtype == "f32" else 2
    alg_bytes = (2 * B * H * Lq * D + 2 * B * H * Lk * D) * es
    flops = 4 * B * H * Lq * Lk * D
    ms = res["ms_per_step"]
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    # fp32 work runs on fp16 matrix cores as three products of hi + lo parts
    # per fp32 product: its matrix ceiling is the fp16 rate / 3 (ridge 104
    # FLOP/B), above fp32 MFMA's 157.3 TFLOP/s
    mpeak = BF16_PEAK_TFLOPS if dtype == "bf16" else F32_SPLIT_PEAK_TFLOPS
    bound = "hbm" if flops / alg_bytes < mpeak * 1e12 / (HBM_PEAK_GBS * 1e9) else "mfma"
    if bound == "hbm":
        frac = gbs / HBM_PEAK_GBS
    else:
        frac = tflops / mpeak
    return alg_bytes, flops, gbs, tflops, bound, frac


def main():
    a = parse()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the hot path is per-GPU; heads "
              "shard across GPUs with no exchange); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import attn_mi355x as am
    import hip_rt

    am.lib()
    if hip_rt.device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    head_cfg_id = a.config or 2
    cfg = list(CONFIGS[head_cfg_id])
    if a.no_flash:
        am.set_tuning(no_flash=True)
    if a.shape:
        b_, h_, lq_, lk_, d_ = (int(x) for x in a.shape.split(","))
        lbl = "fp32" if a.dtype == "f32" else "bf16"
        enc = {"none": "", "rope_half": " RoPE rotate-half", "sinusoidal": " sinusoidal"}[a.pe]
        cfg = [f"{lbl} SDPA{enc} ({b_},{h_},{lq_},{lk_},{d_})", a.dtype, b_, h_, lq_, lk_, d_,
               a.pe, 0.5 if a.pe == "sinusoidal" else 1.0]
        head_cfg_id = 0
    if a.head_dim:
        cfg[6] = a.head_dim
        cfg[0] = cfg[0].split(" (")[0] + f" ({cfg[2]},{cfg[3]},{cfg[4]},{cfg[5]},{cfg[6]})"
    cfg = tuple(cfg)
    name, dtype, B, H, Lq, Lk, D, pe, sigma = cfg
    print(f"[bench] {name} steps={a.steps} warmup={a.warmup} device={hip_rt.device_name(0)}",
          file=sys.stderr, flush=True)

    res, host, rows_fn = run_config(am, hip_rt, cfg, a.steps, a.warmup, a.seed,
                                    cold=1 <= head_cfg_id <= 3)
    if a.calib_copy > 0:
        n = a.calib_copy << 20
        src, dst = hip_rt.DeviceArray((n // 4,), "f32", fill=0), hip_rt.DeviceArray((n // 4,), "f32")
        for _ in range(5):
            hip_rt.copy_d2d(dst, src, n)
        hip_rt.synchronize()
        print(f"[bench] calibration: 5 device copies of {a.calib_copy} MiB", file=sys.stderr)
    check = sampled_check(cfg, host, rows_fn)
    alg_bytes, flops, gbs, tflops, bound, frac = summarize(cfg, res)
    ms = res["ms_per_step"]

    traffic, traffic_src = MEASURED_TRAFFIC.get((head_cfg_id, D), (None, None))
    if bound == "hbm":
        roof = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(frac, 4), "traffic": traffic}
    else:
        peak = BF16_PEAK_TFLOPS if dtype == "bf16" else F32_SPLIT_PEAK_TFLOPS
        roof = {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(frac, 4), "traffic": traffic}
        if dtype == "f32":
            roof["peak_note"] = ("fp32 work as three fp16 MFMA products (hi + lo parts): the "
                                 "fp16 dense rate 2500 / 3; fp32 MFMA's own peak is "
                                 f"{FP32_PEAK_TFLOPS} TFLOP/s")
    path = res["path"]
    PATH_NAMES.update({
        am.ATN_PATH_FUSED_SMALL: "k_fused_small (one launch per step)",
        am.ATN_PATH_SPLIT_D: "split-D pipeline (QK^T partials + softmax + PV per step)",
        am.ATN_PATH_FLASH: "k_flash (one launch per step)",
        am.ATN_PATH_GEMM: ("GEMM path (encode, QK^T GEMM with exp epilogue, PV GEMM per step; "
                           "whole-step figure, per-kernel split in profiles/)"),
    })
    roof["kernel"] = PATH_NAMES.get(path, "unknown")
    roof["timing"] = "HIP events around one graph replay of all timed steps, on its stream"
    ck = cold_kernel(cfg, res)
    if ck is not None:
        # the warm figure above runs on inputs the 256 MiB MALL holds between
        # graph replays; this one is a single call after a MALL flush
        roof["cold"] = {"ms": round(ck[0], 6), "achieved": round(ck[1] * HBM_PEAK_GBS, 2),
                        "frac": round(ck[1], 4),
                        "method": "median single call after a 512 MiB device copy, minus the "
                                  "events' own overhead (bracketed median without the copy "
                                  "less the graph-replayed step time); an upper bound, since "
                                  "events after a flush cost more than without one (rocprofv3 "
                                  "per-dispatch durations of the same calls: profiles/)"}
    if traffic is not None:
        roof["traffic_note"] = ("bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE scaled by "
                                f"a known-size device copy ({traffic_src})")

    hinfo = host_info()
    cpu = None
    if a.cpu_seconds > 0:
        v_cpu, job_ms, sample = cpu_baseline(cfg, host, a.cpu_seconds)
        cpu = {"value": round(v_cpu, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "job_ms": round(job_ms, 3), "sample": sample, "host": hinfo}
    del host

    all_ok = check["ok"]
    per_config = None
    if a.config == 0 and not a.shape:
        per_config = {}
        others = [(f"cfg2_D{d}", 2, d) for d in SWEEP_D] + [(f"cfg{c}", c, 0) for c in (1, 3, 4, 5)]
        others += [(k, 0, 0) for k in LONG]
        for key, cid, dov in others:
            c = list(CONFIGS[cid] if cid else LONG[key])
            if dov:
                c[6] = dov
                c[0] = c[0].split(" (")[0] + f" ({c[2]},{c[3]},{c[4]},{c[5]},{c[6]})"
            c = tuple(c)
            print(f"[bench] per_config {key}: {c[0]}", file=sys.stderr, flush=True)
            r, h, rf = run_config(am, hip_rt, c, a.steps, a.warmup, a.seed, cold=1 <= cid <= 3)
            chk = sampled_check(c, h, rf)
            ab, fl, g, tf, bd, fr = summarize(c, r)
            ent = {"workload": c[0], "dtype": c[1], "pe": c[7], "ms_per_step": round(r["ms_per_step"], 6),
                   "ms_per_step_median5": round(r["median5_ms_per_step"], 6),
                   "tflops": round(tf, 3), "gbs": round(g, 2), "roofline_bound": bd,
                   "roofline_frac": round(fr, 4), "alg_bytes": ab, "flops": fl,
                   "path": PATH_NAMES.get(r["path"], "unknown"), "check": chk}
            if "cold_ms_per_step" in r:
                ent["cold_ms_per_step"] = round(r["cold_ms_per_step"], 6)
                ent["bracketed_ms_per_step"] = round(r["bracketed_ms_per_step"], 6)
                ck = cold_kernel(c, r)
                ent["cold_kernel_ms"] = round(ck[0], 6)
                ent["roofline_frac_cold"] = round(ck[1], 4)
            if "dropin_sync_ms" in r:
                ent["dropin_sync_ms"] = round(r["dropin_sync_ms"], 6)
            if a.cpu_seconds > 0:
                v_cpu, job_ms, sample = cpu_baseline(c, h, a.cpu_seconds_other)
                ent["cpu_baseline"] = {"value": round(v_cpu, 4), "unit": "GB/s", "cores": 1,
                                       "kind": "port", "job_ms": round(job_ms, 3),
                                       "sample": sample,
                                       "gpu_speedup": round(job_ms / r["ms_per_step"], 1)}
            per_config[key] = ent
            all_ok = all_ok and chk["ok"]
            del h

    cfg_out = {"workload": name, "batch": B, "heads": H, "len_q": Lq, "len_k": Lk,
               "head_dim": D, "pe": pe, "alg_bytes": alg_bytes, "flops": flops,
               "check": check}
    if "cold_ms_per_step" in res:
        cfg_out["cold_ms_per_step"] = round(res["cold_ms_per_step"], 6)
        cfg_out["bracketed_ms_per_step"] = round(res["bracketed_ms_per_step"], 6)
        cfg_out["cold_note"] = (f"median of single calls between events of their own, each after a "
                                f"{MALL_FLUSH_MIB} MiB device copy (MALL flushed); "
                                "bracketed_ms_per_step is the same without the copies, so the "
                                "events' own overhead shows against ms_per_step")
    if "dropin_sync_ms" in res:
        cfg_out["dropin_sync_ms"] = round(res["dropin_sync_ms"], 6)
        cfg_out["dropin_note"] = ("median host wall clock of one synchronous drop-in call "
                                  "(attention_forward_optimized / attention_forward_bf16: "
                                  "launch, then wait for the device)")
    line = {
        "metric": "attention ms + TFLOPS + HBM GB/s (% roofline) at hdim 512-8192, 1 GPU",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 6),
        "ms_per_step_median5": round(res["median5_ms_per_step"], 6),
        "ms_per_step_eager_python": round(res["eager_ms"], 6),
        "tflops": round(tflops, 4),
        "pct_hbm_roofline": round(100 * gbs / HBM_PEAK_GBS, 2),
        "wall_s": round(res["wall_s"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if dtype == "f32" else "bf16 storage, f32 math",
        "data": "synthetic N(0,%g), numpy PCG64 seed %d, resident in HBM" % (sigma, a.seed),
        "config": cfg_out,
        "roofline": roof,
        "cpu_baseline": cpu,
        "host": hinfo,
        "parity_ok": all_ok,
    }
    if per_config is not None:
        line["per_config"] = per_config
    print(json.dumps(line), flush=True)
    if not all_ok:
        print("bench.py: a sampled output missed its tolerance (see check / per_config.*.check)",
              file=sys.stderr)
        sys.exit(1)


if __name__ == "__main__":
    main()
