"""Context numbers: this library next to PyTorch-ROCm on the same MI355X.

    python accelerated-final-project_amd/torch_compare.py [--iters 100] [--json out.json]
        [--shapes cfg2,"ref hdim=512"] [--save DIR]
    python accelerated-final-project_amd/torch_compare.py --gemm-ceiling [--json out.json]

The reference's PyTorch harness (final/benchmark_pytorch_wrapper.cu:25-130)
times F.scaled_dot_product_attention ("optimized") and matmul -> softmax ->
matmul ("naive") on its four head-dim shapes, 10 warm-up and 100 timed
calls between CUDA events.  This does the same on the MI355X for those four
shapes and the BASELINE configurations, and puts this library's
atn_attention_fwd_ex beside them: all three run on the same device tensors
and on torch's current stream, timed by the same events.  For the RoPE
(rotate-half) and sinusoidal configurations the torch side encodes Q and K
with elementwise ops from tables built the way the reference builds its
caches (final/rope.cu:20-40, final/sinusoidal.cu:838-855), then attends.

--gemm-ceiling instead times torch.bmm (hipBLASLt / rocBLAS) in bf16 on the
two contractions of BASELINE configs 4 and 5 (Q K^T and P V per head,
contiguous operands, bf16 out): plain library GEMMs with no encoding and no
softmax, the floor under any two-GEMM attention of those shapes on this
device.

The printed max |difference| against torch SDPA is context only; parity is
established against the CPU oracle by the test suite (--save writes each
shape's inputs and this library's output as .npy files, which
tests/test_gpu_torch_harness.py checks against the oracle).

One HIP runtime.  This process hands torch's device pointers and stream to
the library, which is only sound if both use the same HIP runtime.  torch's
bundled libamdhip64 and /opt/rocm's carry the same SONAME
(libamdhip64.so.7), so once torch is imported the loader binds the library
to torch's copy; hip_runtimes_mapped() reads /proc/self/maps to confirm that
exactly one libamdhip64 is mapped, the run stops otherwise, and the path is
printed and recorded in the JSON output.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

# (name, dtype, B, H, Lq, Lk, D, pe); the first four are the reference
# harness's shapes (fp32, no encoding), then BASELINE configs 1-5
SHAPES = [
    ("ref hdim=512", "f32", 1, 4, 64, 64, 512, "none"),
    ("ref hdim=2048", "f32", 1, 4, 64, 64, 2048, "none"),
    ("ref hdim=4096", "f32", 1, 2, 32, 32, 4096, "none"),
    ("ref hdim=8192", "f32", 1, 1, 16, 16, 8192, "none"),
    ("cfg1", "f32", 1, 1, 4, 4, 8, "none"),
    ("cfg2", "f32", 1, 4, 64, 64, 2048, "none"),
    ("cfg3", "bf16", 1, 4, 32, 128, 8192, "none"),
    ("cfg4 rope-half", "bf16", 8, 8, 1024, 1024, 4096, "rope_half"),
    ("cfg5 sinusoidal", "bf16", 4, 16, 256, 2048, 1024, "sinusoidal"),
    # the encodings inside the single-launch kernel at configs 2 and 3
    ("cfg2 rope-half", "f32", 1, 4, 64, 64, 2048, "rope_half"),
    ("cfg2 sinusoidal", "f32", 1, 4, 64, 64, 2048, "sinusoidal"),
    ("cfg3 rope-half", "bf16", 1, 4, 32, 128, 8192, "rope_half"),
    # fp32 beyond the single-launch window: the reference's own long-sequence
    # test shape (final/attention.cu:522, the flash kernel) and a large-head
    # one (the split-D pipeline); names without commas (--shapes splits on them)
    ("ref llama 4x32x512x128", "f32", 4, 32, 512, 512, 128, "none"),
    ("f32 long 1x4x512x512x2048", "f32", 1, 4, 512, 512, 2048, "none"),
    # bf16 at head_dim <= 128 beyond the single-launch window (the flash
    # kernel; torch's SDPA runs its own flash kernel here)
    ("bf16 llama 4x32x512x128", "bf16", 4, 32, 512, 512, 128, "none"),
    ("bf16 rope-half 4x32x512x128", "bf16", 4, 32, 512, 512, 128, "rope_half"),
    ("bf16 long 1x8x4096x4096x128", "bf16", 1, 8, 4096, 4096, 128, "none"),
    ("bf16 long 1x32x2048x2048x64", "bf16", 1, 32, 2048, 2048, 64, "none"),
    ("bf16 rope-half long 1x8x4096x4096x128", "bf16", 1, 8, 4096, 4096, 128, "rope_half"),
]


def hip_runtimes_mapped() -> list[str]:
    """Distinct libamdhip64 files mapped into this process."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64" in os.path.basename(parts[-1]):
                paths.add(parts[-1])
    return sorted(paths)


def tables(torch, pe, npos, D, dev):
    """fp32 encoding tables [npos][D/2] with the reference's expressions."""
    pos = torch.arange(npos, dtype=torch.float32, device=dev)[:, None]
    i = torch.arange(D // 2, dtype=torch.float32, device=dev)[None, :]
    freq = 1.0 / torch.pow(torch.tensor(10000.0, device=dev), (2.0 * i) / D)
    ang = pos * freq
    return torch.cos(ang), torch.sin(ang)


def torch_encode(torch, x, pe, cos, sin):
    """Encoded copy of x [B,H,L,D] (fp32 math, cast back to x's dtype)."""
    L, D = x.shape[2], x.shape[3]
    xf = x.float()
    if pe == "rope_half":
        c, s = cos[:L], sin[:L]
        x1, x2 = xf[..., : D // 2], xf[..., D // 2:]
        y = torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)
    else:  # sinusoidal: even dims + sin, odd dims + cos
        pe_t = torch.stack([sin[:L], cos[:L]], dim=-1).reshape(L, D)
        y = xf + pe_t
    return y.to(x.dtype)


# (name, batch of heads, M, K, N) of C[b] = A[b] B[b]: Q K^T and P V of
# BASELINE configs 4 (B=8 H=8 L=1024 D=4096) and 5 (B=4 H=16 Lq=256 Lk=2048
# D=1024)
GEMMS = [
    ("cfg4 QK^T", 64, 1024, 4096, 1024),
    ("cfg4 PV", 64, 1024, 1024, 4096),
    ("cfg5 QK^T", 64, 256, 1024, 2048),
    ("cfg5 PV", 64, 256, 2048, 1024),
]


def write_json(path, rows):
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    with open(path, "w") as f:
        json.dump(rows, f, indent=1)


def gemm_ceiling(torch, dev, timed):
    """bf16 torch.bmm on the config-4/5 contractions (contiguous operands)."""
    rows = []
    g = torch.Generator(device=dev).manual_seed(0)
    for name, b, m, k, n in GEMMS:
        A = torch.randn(b, m, k, device=dev, generator=g).to(torch.bfloat16)
        Bm = torch.randn(b, k, n, device=dev, generator=g).to(torch.bfloat16).contiguous()
        C = torch.empty(b, m, n, device=dev, dtype=torch.bfloat16)
        ms = timed(lambda: torch.bmm(A, Bm, out=C))
        flops = 2 * b * m * k * n
        nbytes = 2 * (b * m * k + b * k * n + b * m * n)
        rows.append({"gemm": name, "batch": b, "M": m, "K": k, "N": n, "ms": ms,
                     "tflops": flops / ms / 1e9, "gbs": nbytes / ms / 1e6})
        print(f"{name:10s} bmm bf16 [{b}x{m}x{k}] x [{b}x{k}x{n}]  {ms * 1e3:9.1f} us  "
              f"{flops / ms / 1e9:8.1f} TFLOP/s  {nbytes / ms / 1e6:8.1f} GB/s", flush=True)
        del A, Bm, C
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--json", default="")
    ap.add_argument("--shapes", default="",
                    help="comma-separated shape names to run (default: all)")
    ap.add_argument("--save", default="",
                    help="directory for each shape's inputs and this library's output (.npy)")
    ap.add_argument("--gemm-ceiling", action="store_true",
                    help="time torch.bmm on the config-4/5 contractions instead")
    a = ap.parse_args()
    wanted = [w.strip() for w in a.shapes.split(",") if w.strip()]
    shapes = [sh for sh in SHAPES if not wanted or sh[0] in wanted]
    if wanted and len(shapes) != len(wanted):
        print(f"torch_compare.py: unknown shape in {wanted}", file=sys.stderr)
        sys.exit(2)

    import torch
    import torch.nn.functional as F

    import attn_mi355x as am

    if not torch.cuda.is_available():
        print("torch_compare.py: no GPU visible to torch", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    lib = am.lib()
    runtimes = hip_runtimes_mapped()
    if len(runtimes) != 1:
        print(f"torch_compare.py: {len(runtimes)} HIP runtimes mapped ({runtimes}); torch's "
              "device pointers cannot be handed to the library", file=sys.stderr)
        sys.exit(1)
    print(f"GPU: {torch.cuda.get_device_name(0)}  torch {torch.__version__}  "
          f"HIP {torch.version.hip}  runtime {runtimes[0]}", flush=True)

    def timed(fn):
        for _ in range(a.warmup):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(a.iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / a.iters

    if a.gemm_ceiling:
        rows = gemm_ceiling(torch, dev, timed)
        if a.json:
            write_json(a.json, rows)
        return

    rows = []
    g = torch.Generator(device=dev).manual_seed(0)
    for idx, (name, dt, B, H, Lq, Lk, D, pe) in enumerate(shapes):
        tdt = torch.float32 if dt == "f32" else torch.bfloat16
        sigma = 0.5 if pe == "sinusoidal" else 1.0
        Q = (torch.randn(B, H, Lq, D, device=dev, generator=g) * sigma).to(tdt)
        K = (torch.randn(B, H, Lk, D, device=dev, generator=g) * sigma).to(tdt)
        V = (torch.randn(B, H, Lk, D, device=dev, generator=g) * sigma).to(tdt)
        out = torch.empty_like(Q)
        desc = None
        if pe == "rope_half":
            desc = am.make_pe("rope", pairing="half")
        elif pe == "sinusoidal":
            desc = am.make_pe("sinusoidal")
        dcode = am.ATN_DTYPE_F32 if dt == "f32" else am.ATN_DTYPE_BF16
        nbytes = lib.atn_attention_workspace_bytes(dcode, B, H, Lq, Lk, D,
                                                   ctypes.byref(desc) if desc else None)
        ws = torch.zeros(max(nbytes, 4) // 4 + 1, dtype=torch.float32, device=dev)
        if desc is not None:
            st = lib.atn_prepare_pe_ex(ctypes.byref(desc), D, max(Lq, Lk))
            if st != am.ATN_OK:
                raise am.AtnError(st, "atn_prepare_pe_ex")

        def ours():
            st = lib.atn_attention_fwd_ex(
                dcode, ctypes.c_void_p(Q.data_ptr()), ctypes.c_void_p(K.data_ptr()),
                ctypes.c_void_p(V.data_ptr()), ctypes.c_void_p(out.data_ptr()), B, H, Lq, Lk, D,
                ctypes.byref(desc) if desc else None, ctypes.c_void_p(ws.data_ptr()),
                ws.numel() * 4, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if st != am.ATN_OK:
                raise am.AtnError(st, "atn_attention_fwd_ex")

        if pe == "none":
            def enc():
                return Q, K
        else:
            cos, sin = tables(torch, pe, max(Lq, Lk), D, dev)

            def enc():
                return torch_encode(torch, Q, pe, cos, sin), torch_encode(torch, K, pe, cos, sin)

        def sdpa():
            q, k = enc()
            return F.scaled_dot_product_attention(q, k, V)

        scale = 1.0 / (D ** 0.5)

        def naive():
            q, k = enc()
            s = torch.matmul(q, k.transpose(-2, -1).contiguous()) * scale
            return torch.matmul(F.softmax(s, dim=-1), V)

        t_ours = timed(ours)
        t_sdpa = timed(sdpa)
        t_naive = timed(naive)
        ours()
        ref = sdpa()
        torch.cuda.synchronize()
        diff = float((out.float() - ref.float()).abs().max())
        flops = 4 * B * H * Lq * Lk * D
        alg_bytes = (2 * B * H * Lq * D + 2 * B * H * Lk * D) * (4 if dt == "f32" else 2)
        row = {"shape": name, "hip_runtime": runtimes[0], "dtype": dt, "B": B, "H": H, "Lq": Lq,
               "Lk": Lk, "D": D, "pe": pe,
               "ours_ms": t_ours, "torch_sdpa_ms": t_sdpa, "torch_naive_ms": t_naive,
               "ours_tflops": flops / t_ours / 1e9, "ours_gbs": alg_bytes / t_ours / 1e6,
               "speedup_vs_sdpa": t_sdpa / t_ours, "max_abs_diff_vs_sdpa": diff}
        if a.save:
            import numpy as np
            os.makedirs(a.save, exist_ok=True)
            for tag, t in (("Q", Q), ("K", K), ("V", V), ("out", out)):
                np.save(os.path.join(a.save, f"{idx}_{tag}.npy"), t.float().cpu().numpy())
            row["saved"] = f"{idx}_{{Q,K,V,out}}.npy"
        rows.append(row)
        print(f"{name:16s} {dt:4s} ours {t_ours:9.4f} ms  sdpa {t_sdpa:9.4f} ms  "
              f"naive {t_naive:9.4f} ms  x{t_sdpa / t_ours:6.2f} vs sdpa  "
              f"{row['ours_tflops']:8.2f} TFLOP/s  max|d| {diff:.2e}", flush=True)
        del Q, K, V, out, ws
        torch.cuda.empty_cache()
    if a.json:
        write_json(a.json, rows)


if __name__ == "__main__":
    main()
