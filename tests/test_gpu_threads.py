"""Host threads calling the library at once, each on a stream of its own with
the library's per-stream workspace: the plan caches, the per-stream
workspaces and the positional-encoding tables are shared host state, and
the encoding tables grow (to more positions) while kernels of other threads
that read the smaller tables are still queued.  ctypes releases the GIL
around each foreign call, so the calls overlap in the library's host code.

The shapes take the GEMM path (bf16, with and without encodings), the
flash kernel (bf16 and fp32) and the split-D pipeline (fp32 past head_d
256): none waits on other workgroups, so kernels of the other threads
holding CUs only delay them.  (The single-launch kernel's exchange needs its whole grid resident;
its concurrency contract is covered in test_gpu_fused.py.)
"""
import threading

import numpy as np
import pytest

import helpers as H
import oracle

pytestmark = pytest.mark.gpu

CASES = [  # (dtype, pe, (B, H, Lq, Lk, D), expected path)
    ("bf16", "sinusoidal", (1, 2, 256, 384, 256), "gemm"),
    ("bf16", "rope_half", (1, 2, 128, 640, 128), "flash"),
    ("f32", "none", (1, 2, 100, 300, 64), "flash"),
    ("f32", "none", (1, 2, 100, 300, 520), "split_d"),
    ("bf16", "sinusoidal", (1, 1, 129, 1040, 512), "gemm"),
]


def _desc(am, pe):
    return {"none": None, "rope_half": am.make_pe("rope", pairing="half"),
            "sinusoidal": am.make_pe("sinusoidal")}[pe]


def _ref(pe, Q, K, V):
    Lq, Lk, D = Q.shape[2], K.shape[2], Q.shape[3]
    if pe == "none":
        return oracle.attention(Q, K, V, nthreads=16)
    if pe == "sinusoidal":
        st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
        return oracle.attention_sinusoidal(Q, K, V, st, ct, nthreads=16)
    c, s = oracle.rope_cache(max(Lq, Lk), D)
    return oracle.attention_rope(Q, K, V, c, s, pairing="half", nthreads=16)


def test_threads_share_library_state(am, dev):
    import hip_rt
    print("[case] four host threads, four streams, library workspaces", flush=True)
    paths = {"gemm": am.ATN_PATH_GEMM, "split_d": am.ATN_PATH_SPLIT_D, "flash": am.ATN_PATH_FLASH}
    jobs = []
    for i, (dt, pe, shape, want) in enumerate(CASES):
        B, Hh, Lq, Lk, D = shape
        desc = _desc(am, pe)
        code = 1 if dt == "bf16" else 0
        assert am.path(code, B, Hh, Lq, Lk, D, desc) == paths[want], (shape, pe)
        sigma = 0.5 if pe == "sinusoidal" else 1.0
        ins, host = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 300 + i, dt, sigma)
        jobs.append(dict(dt=dt, pe=pe, shape=shape, desc=desc, ins=ins, host=host,
                         out=H.empty((B, Hh, Lq, D), dt), stream=hip_rt.Stream()))
    errors = []
    start = threading.Barrier(len(jobs))

    def run(job):
        try:
            start.wait()
            for _ in range(10):
                am.attention_ex(*job["ins"], job["out"], pe=job["desc"], stream=job["stream"])
        except Exception as e:  # reported on the main thread
            errors.append(repr(e))

    threads = [threading.Thread(target=run, args=(j,)) for j in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a calling thread did not return"
    assert not errors, errors
    for job in jobs:
        job["stream"].synchronize()
        B, Hh = job["shape"][:2]
        assert am.sync_status(None, B, Hh, job["stream"]) == 0
        ref = _ref(job["pe"], *job["host"])
        got = job["out"].numpy()
        if job["dt"] == "f32":
            n, mabs, _ = H.check_f32(got, ref)
            assert n == 0, f"{job['shape']}: {n} mismatches, max abs {mabs}"
        else:
            n, nrel, mabs = H.check_bf16(got, ref)
            assert n == 0, f"{job['shape']} {job['pe']}: normwise rel {nrel}, max abs {mabs}"
        job["stream"].destroy()
