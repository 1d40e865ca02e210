"""Bounded scratch: calls too large for their scratch run in chunks.

The cap is the caller's workspace size, or (library workspace) 1 GiB,
lowered here through atn_tuning.workspace_cap_mib so that moderate shapes split:
first into chunks of heads, and when one head is still too large, into
chunks of query rows (K and V whole; the query side's encoding tables start
at the chunk's first position).  Chunked results must match the oracle and,
on the GEMM path, the unchunked call bit for bit (every output row is
computed the same way whatever the chunking).
"""
import numpy as np
import pytest

import helpers as H
import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _scratch_paths(tuner):
    """The flash kernel needs no scratch: these tests hold calls on the
    paths that do (the GEMM path, the split-D pipeline)."""
    tuner.set(no_flash=True)


def _desc(am, pe):
    return {"none": None, "rope_half": am.make_pe("rope", pairing="half"),
            "rope_inter": am.make_pe("rope"), "sinusoidal": am.make_pe("sinusoidal")}[pe]


def _ref(pe, Q, K, V, Lq, Lk, D):
    if pe == "none":
        return oracle.attention(Q, K, V, nthreads=16)
    if pe == "sinusoidal":
        st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
        return oracle.attention_sinusoidal(Q, K, V, st, ct, nthreads=16)
    c, s = oracle.rope_cache(max(Lq, Lk), D)
    return oracle.attention_rope(Q, K, V, c, s, nthreads=16,
                                 pairing="half" if pe == "rope_half" else "interleaved")


@pytest.mark.parametrize("shape,dtype,pe,cap_mib", [
    ((2, 3, 300, 520, 128), "bf16", "none", 1),        # GEMM path, head and row chunks
    ((1, 2, 700, 300, 256), "bf16", "rope_half", 1),   # row chunks with Q positions offset
    ((1, 2, 500, 260, 64), "bf16", "sinusoidal", 1),
    ((1, 3, 260, 300, 36), "f32", "none", 1),          # split-D pipeline (flash off)
    ((1, 2, 200, 150, 64), "f32", "rope_inter", 1),
], ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_chunked_library_workspace(am, dev, tuner, shape, dtype, pe, cap_mib):
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] chunked {dtype} {shape} {pe} cap {cap_mib} MiB", flush=True)
    desc = _desc(am, pe)
    sigma = 0.5 if pe == "sinusoidal" else 1.0
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 1200 + Lq, dtype, sigma)
    full = H.empty(Q.shape, dtype)
    am.attention_ex(q, k, v, full, pe=desc)
    hip_rt.synchronize()
    tuner.set(workspace_cap_mib=cap_mib)
    dcode = 0 if dtype == "f32" else 1
    assert am.workspace_bytes(dcode, B, Hh, Lq, Lk, D, desc) <= cap_mib << 20
    s = hip_rt.Stream()  # a fresh stream: its library workspace starts within the cap
    out = H.empty(Q.shape, dtype)
    am.attention_ex(q, k, v, out, pe=desc, stream=s)
    s.synchronize()
    assert am.sync_status(None, B, Hh, s) == 0
    ref = _ref(pe, Q, K, V, Lq, Lk, D)
    if dtype == "f32":
        n, mabs, _ = H.check_f32(out.numpy(), ref)
        assert n == 0, mabs
    else:
        n, nrel, mabs = H.check_bf16(out.numpy(), ref)
        assert n == 0, (nrel, mabs)
        if am.path(dcode, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM:
            assert np.array_equal(out.bits(), full.bits()), "chunked GEMM result differs"
    s.destroy()


def test_chunked_caller_workspace(am, dev):
    """A caller workspace smaller than the shape's full need (but at least
    what the chunks need) splits the call instead of failing."""
    import hip_rt
    B, Hh, Lq, Lk, D = 2, 4, 512, 1024, 128
    print("[case] chunked caller workspace", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 1301, "bf16")
    full = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, full)
    hip_rt.synchronize()
    ws = hip_rt.DeviceArray(((3 << 20) // 4,), "f32", fill=0)  # 3 MiB: E alone is 8 MiB
    out = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, out, workspace=ws)
    hip_rt.synchronize()
    assert am.sync_status(ws, B, Hh) == 0
    assert np.array_equal(out.bits(), full.bits())
    tiny = hip_rt.DeviceArray((40960 // 4 + 16,), "f32", fill=0)  # the sync region only
    with pytest.raises(am.AtnError) as e:
        am.attention_ex(q, k, v, out, workspace=tiny)
    assert e.value.status == am.ATN_ERR_WORKSPACE


def test_growing_shapes_keep_library_memory_bounded(am, dev):
    """A growing sequence of shapes on one stream: the library workspace
    grows at least twofold at a time and a superseded workspace that no
    capture used is freed at once, so the library ends up holding less than
    twice the largest need (not the sum of every size)."""
    import hip_rt
    s = hip_rt.Stream()
    base = am.retained_bytes()
    largest = 0
    print("[case] growing shapes, library memory", flush=True)
    for Lk in range(256, 4097, 256):  # bf16 long-sequence path: E grows with Lk
        B, Hh, Lq, D = 1, 4, 512, 128
        (q, k, v), _ = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 1400 + Lk, "bf16")
        out = H.empty((B, Hh, Lq, D), "bf16")
        am.attention_ex(q, k, v, out, stream=s)
        largest = max(largest, am.workspace_bytes(1, B, Hh, Lq, Lk, D))
    s.synchronize()
    assert am.sync_status(None, 1, 1, s) == 0
    held = am.retained_bytes() - base
    assert 0 < held < 2 * largest, (held, largest)
    s.destroy()


def test_captured_workspace_is_kept_until_release(am, dev):
    """A workspace that captured work used is kept when a larger shape
    supersedes it (a graph may still replay it): the library holds it until
    atn_release_ex, which frees it."""
    import hip_rt
    s = hip_rt.Stream()
    B, Hh, Lq, Lk, D = 1, 4, 512, 512, 128
    print("[case] captured workspace kept until release", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 1501, "bf16")
    out = H.empty((B, Hh, Lq, D), "bf16")
    am.attention_ex(q, k, v, out, stream=s)  # allocates the stream's workspace
    s.synchronize()
    g = hip_rt.Graph(s, lambda: am.attention_ex(q, k, v, out, stream=s))
    g.launch()
    s.synchronize()
    g.destroy()
    before = am.retained_bytes()
    # a key length whose need exceeds any workspace the earlier tests grew (a
    # new stream may reuse a destroyed stream's handle, and its workspace)
    big = 64 * Lk
    (q2, k2, v2), _ = H.device_inputs((B, Hh, Lq, D), (B, Hh, big, D), 1502, "bf16")
    am.attention_ex(q2, k2, v2, out, stream=s)  # grows: the captured workspace is kept
    s.synchronize()
    grown = am.retained_bytes()
    assert grown > before  # the new workspace, and the old one kept
    am.release()
    assert am.retained_bytes() < grown  # the old one freed
    am.attention_ex(q, k, v, out, stream=s)  # the stream's current workspace still serves
    s.synchronize()
    assert am.sync_status(None, 1, 1, s) == 0
    n, nrel, mabs = H.check_bf16(out.numpy(), oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, (nrel, mabs)
    s.destroy()
