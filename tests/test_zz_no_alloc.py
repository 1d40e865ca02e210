"""The allocation-free entry point (atn_attention_fwd_noalloc_ex) on the GPU.

Its kernels are the ones atn_attention_fwd_ex runs, with scratch in the
library's per-device static array instead of a workspace, so its outputs must
equal atn_attention_fwd_ex's bit for bit.  Each case makes two calls in a
row -- the second with a smaller input -- so the second call runs on the
array the first one left behind.  Larger shapes run in chunks that fit the
array's 64 MiB; a shape whose smallest chunk does not fit, and encodings
whose tables were never prepared, are refused with their status codes, with
nothing launched.
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
    ((1, 2, 256, 512, 256), (1, 1, 128, 256, 256), "bf16", "rope_half"),  # GEMM path
    ((1, 2, 300, 200, 260), (1, 1, 70, 90, 22), "f32", None),          # split-D pipeline
    ((1, 2, 300, 200, 36), (1, 1, 70, 90, 20), "f32", None),           # flash kernel
    ((1, 2, 300, 200, 128), (1, 1, 70, 90, 64), "bf16", "rope_half"),  # flash kernel, bf16
    ((1, 4, 1024, 2048, 128), (1, 2, 16, 1000, 64), "bf16", None),      # flash, key splits
    ((2, 2, 256, 512, 256), (1, 2, 128, 128, 256), "bf16", "sinusoidal"),  # GEMM path
], ids=["fused-f32", "fused-bf16", "gemm-rope", "splitd", "flash", "flash-bf16", "flash-split",
        "gemm-sin"])
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


def test_noalloc_chunks_large_shapes(am, dev, tuner):
    """A shape whose scratch exceeds the 64 MiB array (E alone is 128 MiB
    here; held on the GEMM path, since the flash kernel that bf16 at head_d
    256 takes by default needs none) runs in chunks of heads that fit it,
    with the same bits as the unchunked atn_attention_fwd_ex."""
    tuner.set(no_flash=True)
    shape = (4, 8, 1024, 2048, 256)
    print(f"[case] noalloc chunked {shape}", flush=True)
    _pair(am, shape, "bf16", None, 950)


def test_noalloc_refuses_what_it_cannot_do(am, dev, tuner):
    import hip_rt
    print("[case] noalloc refusals", flush=True)
    L_ = am.lib()
    # one query row against 32 Mi keys on the GEMM path (the flash kernel,
    # which bf16 at head_d 8 takes by default, needs no scratch): even a
    # one-row chunk needs 64 MiB of scores -- refused before anything is
    # launched
    tuner.set(no_flash=True)
    Lk = 1 << 25
    q, o = hip_rt.DeviceArray((1, 1, 1, 8), "bf16"), hip_rt.DeviceArray((1, 1, 1, 8), "bf16")
    k, v = hip_rt.DeviceArray((1, 1, Lk, 8), "bf16"), hip_rt.DeviceArray((1, 1, Lk, 8), "bf16")
    st = L_.atn_attention_fwd_noalloc_ex(1, q.ptr, k.ptr, v.ptr, o.ptr, 1, 1, 1, Lk, 8, None,
                                         None)
    assert st == am.ATN_ERR_SCRATCH_LIMIT, st
    tuner.clear()
    # an encoding base whose tables were never built
    odd = am.make_pe("rope", pairing="half", base=1234.5)
    qs, os_ = (hip_rt.DeviceArray((1, 1, 64, 256), "bf16") for _ in range(2))
    st = L_.atn_attention_fwd_noalloc_ex(1, qs.ptr, qs.ptr, qs.ptr, os_.ptr, 1, 1, 64, 64, 256,
                                         odd, None)
    assert st == am.ATN_ERR_NOT_PREPARED, st
    hip_rt.synchronize()
    assert am.sync_status() == 0
    for t in (q, o, k, v, qs, os_):
        t.free()
