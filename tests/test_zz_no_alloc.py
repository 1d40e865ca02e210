"""The allocation-free entry point (atn_attention_fwd_noalloc_ex) on the GPU.

Its kernels are the ones atn_attention_fwd_ex runs, with scratch in the
library's per-device static array instead of a workspace, so its outputs must
equal atn_attention_fwd_ex's bit for bit.  Each case makes two calls in a
row -- the second with a smaller input -- so the second call runs on the
array the first one left behind.  Calls beyond the array's 64 MiB and
encodings whose tables were never prepared are refused with their status
codes, with nothing launched.
"""
import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def _pair(am, shape, dtype, pe, seed):
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    sigma = 0.5 if pe is not None and pe.kind == am.ATN_PE_SINUSOIDAL else 1.0
    (q, k, v), _ = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed, dtype, sigma)
    dcode = 0 if dtype == "f32" else 1
    ws = hip_rt.DeviceArray((am.workspace_bytes(dcode, *shape, pe) // 4,), "f32", fill=0)
    ref = H.empty((B, Hh, Lq, D), dtype)
    am.attention_ex(q, k, v, ref, pe=pe, workspace=ws)
    got = H.empty((B, Hh, Lq, D), dtype)
    am.attention_noalloc_ex(q, k, v, got, pe=pe)
    hip_rt.synchronize()
    assert am.sync_status(ws, B, Hh) == 0 and am.sync_status() == 0
    a, b = ref.bits(), got.bits()
    assert np.isfinite(ref.numpy()).all()
    assert np.array_equal(a, b), f"{shape} {dtype}: allocation-free result differs from _ex"


@pytest.mark.parametrize("first,second,dtype,pe", [
    ((1, 4, 64, 64, 2048), (1, 2, 32, 32, 512), "f32", None),          # single-launch kernel
    ((1, 4, 32, 128, 8192), (1, 1, 16, 100, 1024), "bf16", None),      # single-launch, bf16
    ((1, 2, 256, 512, 256), (1, 1, 128, 256, 128), "bf16", "rope_half"),  # GEMM path
    ((1, 2, 300, 200, 36), (1, 1, 70, 90, 20), "f32", None),           # split-D pipeline
    ((2, 2, 256, 512, 128), (1, 2, 128, 128, 128), "bf16", "sinusoidal"),  # GEMM path
], ids=["fused-f32", "fused-bf16", "gemm-rope", "splitd", "gemm-sin"])
def test_noalloc_matches_ex_two_calls(am, dev, first, second, dtype, pe):
    desc = None
    if pe == "rope_half":
        desc = am.make_pe("rope", pairing="half")
    elif pe == "sinusoidal":
        desc = am.make_pe("sinusoidal")
    if desc is not None:
        D = first[4]
        assert am.lib().atn_prepare_pe_ex(desc, D, max(first[2], first[3])) == 0
        assert am.lib().atn_prepare_pe_ex(desc, second[4], max(second[2], second[3])) == 0
    for i, shp in enumerate((first, second)):
        print(f"[case] noalloc {dtype} {shp} pe={pe} call {i}", flush=True)
        _pair(am, shp, dtype, desc, 900 + i)


def test_noalloc_refuses_what_it_cannot_do(am, dev):
    import hip_rt
    print("[case] noalloc refusals", flush=True)
    L_ = am.lib()
    # config 4 needs far more than 64 MiB of scratch (E alone is 128 MiB):
    # refused before anything is launched
    B, Hh, L, D = 8, 8, 1024, 4096
    desc = am.make_pe("rope", pairing="half")
    assert L_.atn_prepare_pe_ex(desc, D, L) == 0
    q, k, v, o = (hip_rt.DeviceArray((B, Hh, L, D), "bf16") for _ in range(4))
    st = L_.atn_attention_fwd_noalloc_ex(1, q.ptr, k.ptr, v.ptr, o.ptr, B, Hh, L, L, D, desc, None)
    assert st == am.ATN_ERR_SCRATCH_LIMIT, st
    # an encoding base whose tables were never built
    odd = am.make_pe("rope", pairing="half", base=1234.5)
    st = L_.atn_attention_fwd_noalloc_ex(1, q.ptr, k.ptr, v.ptr, o.ptr, 1, 1, 64, 64, 256, odd,
                                         None)
    assert st == am.ATN_ERR_NOT_PREPARED, st
    hip_rt.synchronize()
    assert am.sync_status() == 0
    for t in (q, k, v, o):
        t.free()
