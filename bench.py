"""Benchmark of the large-head-dim fused attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--head-dim D]

A "step" is one call of the hot path (atn_attention_fwd_ex, asynchronous,
on one HIP stream) over one batch of synthetic input already resident in
HBM.  The default workload is BASELINE config 2: fp32 SDPA, batch 1, 4
heads, len_q = len_k = 64, head_dim 2048, Q/K/V iid N(0,1).  --config 3/4/5
and --head-dim select the other BASELINE shapes for profiling; the default
line is config 2.

Printed: ONE JSON line.  `value` is the algorithmic HBM throughput
(Q + K + V read once + O written once, bytes / second) of the whole job;
TFLOP/s use 4*B*H*Lq*Lk*D.  `roofline` times the dominant kernel with HIP
events on the stream it runs on; `cpu_baseline` times the CPU oracle (the
restatement of the reference's single-threaded attention_cpu,
final/attention.cu:228-283) on a bounded sample of the same workload.
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

# HBM traffic per launch of the dominant kernel, measured with rocprofv3
# FETCH_SIZE / WRITE_SIZE and scaled by a known-size device copy
# (profiles/fused_small_cfg2_traffic.md).  Keyed by (config, head_dim).
MEASURED_TRAFFIC_BYTES = {
    (2, 2048): (14845 + 3081) * 1024,
}
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3

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


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--head-dim", type=int, default=0, help="override D (config-2 sweep)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target CPU-oracle sample time (0 = skip)")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="also run 5 device-to-device copies of MIB MiB (the HIP runtime's "
                         "copy kernel), a known-size reference for rocprofv3 traffic counters")
    return ap.parse_args()


def make_inputs(dtype, B, H, Lq, Lk, D, sigma, seed):
    """Seeded N(0, sigma) inputs generated on the host with numpy PCG64,
    uploaded once (they stay resident for every step)."""
    import hip_rt
    rng = np.random.default_rng(seed)
    dev, host = [], []
    for shape in ((B, H, Lq, D), (B, H, Lk, D), (B, H, Lk, D)):
        x = rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)
        d = hip_rt.DeviceArray.from_numpy(x, dtype)
        dev.append(d)
        host.append(x if dtype == "f32" else hip_rt.bf16_bits_to_f32(hip_rt.f32_to_bf16_bits(x)))
    return dev, host


def pe_desc(am, pe):
    if pe == "none":
        return None
    if pe == "rope_half":
        return am.make_pe("rope", pairing="half")
    if pe == "sinusoidal":
        return am.make_pe("sinusoidal")
    raise ValueError(pe)


def cpu_baseline(cfg, host, target_s):
    """Single-threaded CPU oracle on a bounded row sample of the workload;
    returns (value in GB/s of the same algorithmic bytes, sample text)."""
    import oracle
    name, dtype, B, H, Lq, Lk, D, pe, _ = cfg
    Q, K, V = host
    rows_total = B * H * Lq
    es = 4 if dtype == "f32" else 2

    def run(rows):
        if pe == "none":
            return oracle.attention(Q, K, V, rows=rows)
        if pe == "rope_half":
            c, s = oracle.rope_cache(max(Lq, Lk), D)
            return oracle.attention_rope(Q, K, V, c, s, pairing="half", rows=rows)
        st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
        return oracle.attention_sinusoidal(Q, K, V, st, ct, rows=rows)

    # per-row cost estimate from one row, then a sample of whole rows
    t0 = time.perf_counter()
    run((0, 1))
    t1 = max(time.perf_counter() - t0, 1e-6)
    nrows = int(max(1, min(rows_total, target_s / t1)))
    reps = 1
    t0 = time.perf_counter()
    run((0, nrows))
    el = time.perf_counter() - t0
    if nrows == rows_total:
        # whole workload is cheap: repeat it until the target time
        reps = int(max(1, target_s / max(el, 1e-6)))
        t0 = time.perf_counter()
        for _ in range(reps):
            run((0, nrows))
        el = time.perf_counter() - t0
    frac = nrows / rows_total
    alg_bytes = (2 * B * H * Lq * D + 2 * B * H * Lk * D) * es
    sec_per_job = el / reps / frac
    sample = (f"{nrows}/{rows_total} query rows x {reps} rep(s) of {name}, single thread; "
              f"{el:.2f} s measured, whole job = {sec_per_job * 1e3:.2f} ms"
              + (" (extrapolated linearly)" if frac < 1 else ""))
    return alg_bytes / sec_per_job / 1e9, sample


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
    cfg = list(CONFIGS[a.config])
    if a.head_dim:
        cfg[6] = a.head_dim
        cfg[0] = cfg[0].split(" (")[0] + f" ({cfg[2]},{cfg[3]},{cfg[4]},{cfg[5]},{cfg[6]})"
    name, dtype, B, H, Lq, Lk, D, pe, sigma = cfg
    print(f"[bench] {name} steps={a.steps} warmup={a.warmup} device={hip_rt.device_name(0)}",
          file=sys.stderr, flush=True)

    (q, k, v), host = make_inputs(dtype, B, H, Lq, Lk, D, sigma, a.seed)
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

    for _ in range(a.warmup):
        step()
    hip_rt.synchronize()

    # eager: one Python-driven call per step (host-bound for small shapes)
    e0, e1 = hip_rt.Event(), hip_rt.Event()
    e0.record(stream)
    for _ in range(a.steps):
        step()
    e1.record(stream)
    e1.synchronize()
    eager_ms = e0.elapsed_ms(e1) / a.steps

    # timed region: the K steps captured once as a HIP graph and replayed,
    # so the GPU runs them back to back with no host work in between
    graph = hip_rt.Graph(stream, lambda: [step() for _ in range(a.steps)])
    graph.launch()  # warm replay
    stream.synchronize()
    hip_rt.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    graph.launch()
    e1.record(stream)
    e1.synchronize()
    hip_rt.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = e0.elapsed_ms(e1)
    graph.destroy()
    st = am.lib().atn_sync_status_ex(ws.ptr, B, H, stream.handle)
    if st != 0:
        raise am.AtnError(st, "device status after the timed region")
    path = am.path(dcode, B, H, Lq, Lk, D, desc)
    if a.calib_copy > 0:
        n = a.calib_copy << 20
        src, dst = hip_rt.DeviceArray((n // 4,), "f32", fill=0), hip_rt.DeviceArray((n // 4,), "f32")
        for _ in range(5):
            hip_rt.copy_d2d(dst, src, n)
        hip_rt.synchronize()
        print(f"[bench] calibration: 5 device copies of {a.calib_copy} MiB", file=sys.stderr)

    es = 4 if dtype == "f32" else 2
    alg_bytes = (2 * B * H * Lq * D + 2 * B * H * Lk * D) * es
    flops = 4 * B * H * Lq * Lk * D
    ms = ev_ms / a.steps
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12

    # sanity: the last output against the oracle on a few rows
    import oracle
    ref_rows = (0, min(4, B * H * Lq))
    got = out.numpy().reshape(-1, D)[ref_rows[0]:ref_rows[1]]
    if pe == "none":
        ref = oracle.attention(*host, rows=ref_rows)
    elif pe == "rope_half":
        c, s = oracle.rope_cache(max(Lq, Lk), D)
        ref = oracle.attention_rope(*host, c, s, pairing="half", rows=ref_rows)
    else:
        st_, ct_ = oracle.sinusoidal_table(max(Lq, Lk), D)
        ref = oracle.attention_sinusoidal(*host, st_, ct_, rows=ref_rows)
    ref = ref.reshape(-1, D)[ref_rows[0]:ref_rows[1]]
    err = float(np.max(np.abs(got - ref)))

    bound = "hbm" if flops / alg_bytes < (312 if dtype == "bf16" else 19.7) else "mfma"
    traffic = MEASURED_TRAFFIC_BYTES.get((a.config, D))
    if bound == "hbm":
        roof = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic}
    else:
        peak = BF16_PEAK_TFLOPS if dtype == "bf16" else FP32_PEAK_TFLOPS
        roof = {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak, "unit": "TFLOP/s",
                "frac": round(tflops / peak, 4), "traffic": traffic}
    roof["kernel"] = {
        am.ATN_PATH_FUSED_SMALL: "k_fused_small (one launch per step)",
        am.ATN_PATH_SPLIT_D: "split-D pipeline (k_qk_partial + k_softmax + k_pv per step)",
        am.ATN_PATH_GEMM: ("GEMM path (encode, QK^T GEMM with exp epilogue, k_rowscale, PV GEMM "
                           "per step; whole-step figure, per-kernel split in profiles/)"),
    }.get(path, "unknown")
    roof["timing"] = "HIP events around one graph replay of all timed steps, on its stream"
    if traffic is not None:
        roof["traffic_note"] = ("bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE scaled by "
                                "a known-size device copy (profiles/fused_small_cfg2_traffic.md); "
                                "measured for this build's kernel")

    cpu = None
    if a.cpu_seconds > 0:
        v_cpu, sample = cpu_baseline(cfg, host, a.cpu_seconds)
        cpu = {"value": round(v_cpu, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": sample, "host": platform.processor() or platform.machine()}

    line = {
        "metric": "attention ms + TFLOPS + HBM GB/s (% roofline) at hdim 512-8192, 1 GPU",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 6),
        "ms_per_step_eager_python": round(eager_ms, 6),
        "tflops": round(tflops, 4),
        "pct_hbm_roofline": round(100 * gbs / HBM_PEAK_GBS, 2),
        "wall_s": round(wall, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if dtype == "f32" else "bf16 storage, f32 math",
        "data": "synthetic N(0,%g), numpy PCG64 seed %d, resident in HBM" % (sigma, a.seed),
        "config": {"workload": name, "batch": B, "heads": H, "len_q": Lq, "len_k": Lk,
                   "head_dim": D, "pe": pe, "alg_bytes": alg_bytes, "flops": flops,
                   "check_max_abs_vs_oracle": err},
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
