"""GPU tests of the single-launch split-D kernel (len_q <= 64, len_k <= 128).

Besides parity with the CPU oracle (the drop-in tests in
test_gpu_parity.py route these shapes here too), this kernel keeps state in
its workspace: per-row-group epoch words that tag the exchanged scores, and
a status word.  These tests check that many calls in a row on one workspace
keep working and give bit-identical results (fixed summation order), that
every row-group size and both exchange forms agree with the oracle, that
caller workspaces on two streams do not interfere, that captured HIP graphs
replay correctly, and that no call reports a device-side wait timeout.
"""
import numpy as np
import pytest

import helpers as H
import oracle

pytestmark = pytest.mark.gpu


def _ws(am, dcode, B, Hh, Lq, Lk, D, pe=None):
    import hip_rt
    n = am.workspace_bytes(dcode, B, Hh, Lq, Lk, D, pe)
    return hip_rt.DeviceArray((n // 4,), "f32", fill=0)


@pytest.mark.parametrize("shape", [(1, 4, 64, 64, 2048), (1, 4, 64, 64, 512),
                                   (1, 4, 64, 64, 8192), (1, 2, 32, 32, 4096),
                                   (1, 1, 16, 16, 8192), (2, 8, 64, 64, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_fused_path_selected_and_repeatable(am, dev, shape):
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] fused repeat f32 {shape}", flush=True)
    assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_FUSED_SMALL
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 5 + D)
    ws = _ws(am, 0, B, Hh, Lq, Lk, D)
    out = H.empty(Q.shape)
    first = None
    for it in range(25):
        am.attention_ex(q, k, v, out, workspace=ws)
        if it in (0, 24):
            hip_rt.synchronize()
            got = out.bits()
            if first is None:
                first = got
            else:
                assert np.array_equal(first, got), "results differ between calls"
    assert am.sync_status(ws, B, Hh) == 0
    ref = oracle.attention(Q, K, V, nthreads=16)
    n, mabs, mrel = H.check_f32(first, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"


def test_fused_config3_bf16_repeat(am, dev):
    """BASELINE config 3 (bf16 cross-attention 32 -> 128, D = 8192)."""
    import hip_rt
    B, Hh, Lq, Lk, D = 1, 4, 32, 128, 8192
    print("[case] fused repeat bf16 cfg3", flush=True)
    assert am.path(1, B, Hh, Lq, Lk, D) == am.ATN_PATH_FUSED_SMALL
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 33, "bf16")
    out = H.empty(Q.shape, "bf16")
    for _ in range(10):
        am.attention_ex(q, k, v, out)
    hip_rt.synchronize()
    assert am.sync_status() == 0
    ref = oracle.attention(Q, K, V, nthreads=16)
    n, nrel, mabs = H.check_bf16(out.numpy(), ref)
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"
    # the bf16 result is the fp32 result rounded once: far inside 2e-2
    assert nrel < 4e-3, nrel


def test_fused_two_streams_two_workspaces(am, dev):
    import hip_rt
    B, Hh, Lq, Lk, D = 1, 4, 64, 64, 1024
    print("[case] fused two streams", flush=True)
    s1, s2 = hip_rt.Stream(), hip_rt.Stream()
    ins1, host1 = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 71)
    ins2, host2 = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 72)
    w1, w2 = _ws(am, 0, B, Hh, Lq, Lk, D), _ws(am, 0, B, Hh, Lq, Lk, D)
    o1, o2 = H.empty((B, Hh, Lq, D)), H.empty((B, Hh, Lq, D))
    for _ in range(20):
        am.attention_ex(*ins1, o1, workspace=w1, stream=s1)
        am.attention_ex(*ins2, o2, workspace=w2, stream=s2)
    s1.synchronize()
    s2.synchronize()
    assert am.sync_status(w1, B, Hh, s1) == 0 and am.sync_status(w2, B, Hh, s2) == 0
    for o, h in ((o1, host1), (o2, host2)):
        n, mabs, _ = H.check_f32(o.numpy(), oracle.attention(*h, nthreads=16))
        assert n == 0, mabs
    s1.destroy()
    s2.destroy()


@pytest.mark.parametrize("pe", ["rope_half", "rope_inter", "sinusoidal"])
def test_fused_with_encodings_bf16(am, dev, pe):
    """Positional encodings applied at load inside the single-launch kernel."""
    import hip_rt
    B, Hh, Lq, Lk, D = 1, 4, 48, 96, 2048
    print(f"[case] fused bf16 {pe}", flush=True)
    sigma = 0.5 if pe == "sinusoidal" else 1.0
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 81, "bf16", sigma)
    desc = {"rope_half": am.make_pe("rope", pairing="half"),
            "rope_inter": am.make_pe("rope"),
            "sinusoidal": am.make_pe("sinusoidal")}[pe]
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_FUSED_SMALL
    out = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    assert am.sync_status() == 0
    if pe == "sinusoidal":
        st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
        ref = oracle.attention_sinusoidal(Q, K, V, st, ct, nthreads=16)
    else:
        c, s = oracle.rope_cache(max(Lq, Lk), D)
        ref = oracle.attention_rope(Q, K, V, c, s, pairing="half" if pe == "rope_half"
                                    else "interleaved", nthreads=16)
    n, nrel, mabs = H.check_bf16(out.numpy(), ref)
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


# Encodings on the single-launch kernel.  With the library's compact tables
# each thread encodes its rows a batch at a time (the angle and partner loads
# of a batch issued together, rows clamped into the sequence); the caller's
# duplicated tables and a rotate-half width whose half is not a multiple of 4
# take the row-at-a-time form; a side without an encoding is stored as
# loaded.
_FUSED_PE = {
    "rope_half": dict(kind="rope", pairing="half"),
    "rope_inter": dict(kind="rope"),
    "rope_inter_r64": dict(kind="rope", rotary_dim=64),
    "rope_half_r96": dict(kind="rope", pairing="half", rotary_dim=96),
    "rope_half_r52": dict(kind="rope", pairing="half", rotary_dim=52),
    "sinusoidal": dict(kind="sinusoidal"),
    "rope_q_only": dict(kind="rope", pairing="half", apply_k=False),
    "rope_k_only": dict(kind="rope", apply_q=False),
    "sin_k_only": dict(kind="sinusoidal", apply_q=False),
    "rope_caller": dict(kind="rope", caller=True),
    "sin_caller": dict(kind="sinusoidal", caller=True),
}


@pytest.mark.parametrize("mode", list(_FUSED_PE))
@pytest.mark.parametrize("shape,dtype", [((1, 2, 37, 100, 512), "f32"),
                                         ((1, 3, 20, 128, 256), "bf16"),
                                         ((1, 2, 48, 96, 1024), "f32")],
                         ids=["f32-ragged", "bf16", "f32-d1024"])
def test_fused_encodings(am, dev, shape, dtype, mode):
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    kw = dict(_FUSED_PE[mode])
    caller = kw.pop("caller", False)
    print(f"[case] fused encodings {dtype} {shape} {mode}", flush=True)
    n = max(Lq, Lk)
    sin = kw["kind"] == "sinusoidal"
    r = kw.get("rotary_dim", 0) or D
    tabs = oracle.sinusoidal_table(n, D) if sin else oracle.rope_cache(n, r)
    held = []
    if caller:
        held = [H.upload(t) for t in tabs]
        kw.update(table_a=held[0], table_b=held[1])
    desc = am.make_pe(**kw)
    dcode = 0 if dtype == "f32" else 1
    assert am.path(dcode, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_FUSED_SMALL
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 61 + r, dtype,
                                           0.5 if sin else 1.0)
    out = H.empty(Q.shape, dtype)
    am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    assert am.sync_status() == 0
    if sin:
        ref = oracle.attention_sinusoidal(Q, K, V, *tabs, add_q=kw.get("apply_q", True),
                                          add_k=kw.get("apply_k", True), nthreads=16)
    else:
        ref = oracle.attention_rope(Q, K, V, *tabs, rotary_dim=r,
                                    pairing=kw.get("pairing", "interleaved"),
                                    rotate_q=kw.get("apply_q", True),
                                    rotate_k=kw.get("apply_k", True), nthreads=16)
    if dtype == "f32":
        bad, mabs, _ = H.check_f32(out.numpy(), ref)
        assert bad == 0, mabs
    else:
        bad, nrel, mabs = H.check_bf16(out.numpy(), ref)
        assert bad == 0, (nrel, mabs)
    for x in (q, k, v, out, *held):
        x.free()


@pytest.mark.parametrize("xcd", ["0", "1", ""], ids=["device", "xcd", "default"])
@pytest.mark.parametrize("shape", [(1, 4, 64, 64, 2048), (1, 2, 130, 70, 256)],
                         ids=lambda s: "x".join(map(str, s)))
def test_graph_replays_match_eager(am, dev, tuner, shape, xcd):
    """Captured HIP graph of three calls, replayed four times with eager work
    and synchronizations in between; every replay must equal the eager
    result bit for bit (the single-launch kernel keeps its barrier epochs in
    device memory, so replayed arguments stay valid)."""
    import hip_rt
    if xcd:
        tuner.set(fused_xcd={"0": "device", "1": "xcd"}[xcd])
    B, Hh, Lq, Lk, D = shape
    print(f"[case] graph replay {shape} xcd={xcd or 'default'}", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 91)
    ws = _ws(am, 0, B, Hh, Lq, Lk, D)
    st = hip_rt.Stream()
    eager = H.empty(Q.shape)
    am.attention_ex(q, k, v, eager, workspace=ws, stream=st)
    st.synchronize()
    ref = eager.bits()
    outs = [H.empty(Q.shape) for _ in range(3)]
    g = hip_rt.Graph(st, lambda: [am.attention_ex(q, k, v, o, workspace=ws, stream=st)
                                  for o in outs])
    for rep in range(4):
        for o in outs:
            o.fill_nan()
        hip_rt.synchronize()
        g.launch()
        st.synchronize()
        for o in outs:
            assert np.array_equal(o.bits(), ref), f"replay {rep} differs from eager"
        am.attention_ex(q, k, v, eager, workspace=ws, stream=st)  # eager work between replays
        st.synchronize()
        assert np.array_equal(eager.bits(), ref)
    g.destroy()
    assert am.sync_status(ws, B, Hh, st) == 0
    n, mabs, _ = H.check_f32(ref, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, mabs
    st.destroy()


@pytest.mark.parametrize("rows,exchange,xcd", [("16", "gather", "0"), ("16", "rsag", "0"),
                                               ("32", "rsag", "0"), ("64", "rsag", "0"),
                                               ("16", "gather", "1"), ("16", "rsag", "1"),
                                               ("32", "rsag", "1"), ("64", "rsag", "1"),
                                               ("32", "gather", "1"), ("", "", "")],
                         ids=lambda v: v or "default")
@pytest.mark.parametrize("shape,dtype,pe", [((1, 4, 64, 64, 2048), "f32", None),
                                            ((1, 3, 40, 72, 1024), "f32", None),
                                            ((1, 2, 48, 96, 1024), "bf16", "rope_half")],
                         ids=["cfg2", "ragged", "bf16rope"])
def test_fused_row_groups_and_exchanges(am, dev, tuner, rows, exchange, xcd, shape, dtype, pe):
    """Every row-group size and both exchange forms (one gather; reduce-scatter
    + all-gather), each at device scope (xcd 0) and inside one XCD's L2 (xcd
    1; the ragged shape's 9 row groups leave XCDs with different counts and
    idle workgroups), forced through the planner's tuning overrides, give the
    oracle's result, and repeated calls on one workspace are bit-identical."""
    import hip_rt
    if rows:
        tuner.set(fused_rows=int(rows), fused_exchange=exchange,
                  fused_xcd={"0": "device", "1": "xcd"}[xcd])
    B, Hh, Lq, Lk, D = shape
    print(f"[case] fused rows={rows or 'default'} exchange={exchange or 'default'} "
          f"xcd={xcd or 'default'} {dtype} {shape} pe={pe}", flush=True)
    dcode = 0 if dtype == "f32" else 1
    desc = am.make_pe("rope", pairing="half") if pe else None
    assert am.path(dcode, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_FUSED_SMALL
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 101 + D, dtype)
    ws = _ws(am, dcode, B, Hh, Lq, Lk, D, desc)
    out = H.empty(Q.shape, dtype)
    first = None
    for it in range(6):
        am.attention_ex(q, k, v, out, pe=desc, workspace=ws)
        if it in (0, 5):
            hip_rt.synchronize()
            got = out.bits()
            if first is None:
                first = got
            elif not np.array_equal(first, got):
                word = int(ws.bits().ravel()[:1].view(np.uint32)[0])
                st = am.sync_status(ws, B, Hh)
                f32 = (first if dtype == "f32" else hip_rt.bf16_bits_to_f32(first)).reshape(-1, D)
                g32 = (got if dtype == "f32" else hip_rt.bf16_bits_to_f32(got)).reshape(-1, D)
                diff = np.abs(np.nan_to_num(f32, nan=1e9) - np.nan_to_num(g32, nan=1e9))
                rows_d = np.where(diff.max(1) > 0)[0]
                raise AssertionError(
                    f"results differ between calls: status {st} (word {word:#x}), NaNs first "
                    f"{np.isnan(f32).sum()} "
                    f"last {np.isnan(g32).sum()}, {len(rows_d)} rows differ {rows_d[:12].tolist()}, "
                    f"max diff {diff.max():.3g}")
    assert am.sync_status(ws, B, Hh) == 0
    if pe:
        c, s = oracle.rope_cache(max(Lq, Lk), D)
        ref = oracle.attention_rope(Q, K, V, c, s, pairing="half", nthreads=16)
        n, nrel, mabs = H.check_bf16(out.numpy(), ref)
        assert n == 0, f"normwise rel {nrel}, max abs {mabs}"
    else:
        n, mabs, mrel = H.check_f32(out.numpy(), oracle.attention(Q, K, V, nthreads=16))
        assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"


# (shape, forced plan): each of the two layouts of the exchange's sync words.
# Device scope: a group's done words one per 128-byte line (n <= 64 slices
# and at most 32 row groups), or packed (more slices, or more groups).
# XL: a group's arrival counters one per line (at most 32 row groups), or
# packed.
_LAYOUTS = [
    ((1, 4, 64, 64, 2048), dict(fused_rows=16, fused_exchange="rsag",
                                fused_xcd="device")),  # device, spread
    ((1, 1, 16, 16, 8192), dict(fused_rows=16, fused_dc=64, fused_exchange="rsag",
                                fused_xcd="device")),  # 128 slices
    ((1, 36, 64, 128, 448), dict(fused_rows=64, fused_exchange="rsag",
                                 fused_xcd="device")),  # device, 36 groups
    ((1, 4, 64, 64, 2048), dict(fused_rows=16, fused_exchange="gather",
                                fused_xcd="xcd")),  # XL, spread
    ((1, 36, 64, 128, 448), dict(fused_rows=64, fused_exchange="rsag",
                                 fused_xcd="xcd")),  # XL, 36 groups
]


def test_fused_sync_word_layouts_share_a_workspace(am, dev, tuner):
    """The exchange's sync words are laid out one per cache line or packed,
    depending on the plan; calls of every layout, alternating on one
    workspace (sized for the largest), each give the oracle's result three
    times over, and no wait times out: a word one layout leaves behind never
    passes for another layout's (done words carry call tags; every call adds
    exactly its units to each counter it uses)."""
    import hip_rt
    cases = []
    for shape, env in _LAYOUTS:
        B, Hh, Lq, Lk, D = shape
        ins, host = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 701 + D + Hh)
        ref = oracle.attention(*host, nthreads=16)
        cases.append((shape, env, ins, ref))
    need = 0
    for shape, env, _, _ in cases:
        tuner.set(**env)
        need = max(need, am.workspace_bytes(0, *shape))
        tuner.clear()
    ws = hip_rt.DeviceArray((need // 4,), "f32", fill=0)
    for rnd in range(3):
        for shape, env, (q, k_, v), ref in cases:
            print(f"[case] sync word layout round {rnd} {shape} {env}", flush=True)
            tuner.set(**env)
            B, Hh, Lq, Lk, D = shape
            assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_FUSED_SMALL
            out = H.empty((B, Hh, Lq, D))
            am.attention_ex(q, k_, v, out, workspace=ws)
            hip_rt.synchronize()
            assert am.sync_status(ws, B, Hh) == 0
            n, mabs, mrel = H.check_f32(out.numpy(), ref)
            assert n == 0, f"{shape} {env}: {n} mismatches, max abs {mabs}, max rel {mrel}"
            tuner.clear()


@pytest.mark.parametrize("rows,exchange", [("64", "rsag"), ("", "")], ids=["rows64-rsag", "default"])
def test_fused_uneven_slices(am, dev, tuner, rows, exchange):
    """36 heads with 7 D-slices each: with 64-row groups and slices of 64 the
    reduce-scatter owns 1171 entries per workgroup, so a thread reduces
    several entries (4-byte words); by default the planner makes its own
    choice."""
    import hip_rt
    if rows:
        tuner.set(fused_rows=int(rows), fused_exchange=exchange, fused_dc=64)
    B, Hh, Lq, Lk, D = 1, 36, 64, 128, 448
    print(f"[case] fused uneven slices rows={rows or 'default'}", flush=True)
    assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_FUSED_SMALL
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 131)
    ws = _ws(am, 0, B, Hh, Lq, Lk, D)
    out = H.empty(Q.shape)
    for _ in range(3):
        am.attention_ex(q, k, v, out, workspace=ws)
    hip_rt.synchronize()
    assert am.sync_status(ws, B, Hh) == 0
    n, mabs, mrel = H.check_f32(out.numpy(), oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"


@pytest.mark.parametrize("shape,dtype", [((1, 1, 16, 16, 8192), "f32"), ((1, 2, 32, 32, 4096), "f32"),
                                         ((1, 1, 64, 64, 2048), "f32"), ((2, 4, 64, 64, 2048), "f32"),
                                         ((1, 8, 64, 64, 1024), "f32"), ((1, 1, 32, 128, 8192), "bf16"),
                                         ((1, 3, 48, 100, 3072), "bf16")],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else v)
def test_fused_planner_shapes(am, dev, shape, dtype):
    """Shapes on which the planner's time estimate takes wide slices with few
    workgroups (down to 32 for one head), several workgroups per CU, or the
    whole padded head of 48 rows: the oracle's result on each."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] fused planner shape {shape} {dtype}", flush=True)
    dcode = 0 if dtype == "f32" else 1
    assert am.path(dcode, B, Hh, Lq, Lk, D) == am.ATN_PATH_FUSED_SMALL
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 401 + D, dtype)
    ws = _ws(am, dcode, B, Hh, Lq, Lk, D)
    out = H.empty(Q.shape, dtype)
    am.attention_ex(q, k, v, out, workspace=ws)
    hip_rt.synchronize()
    assert am.sync_status(ws, B, Hh) == 0
    ref = oracle.attention(Q, K, V, nthreads=16)
    if dtype == "f32":
        n, mabs, mrel = H.check_f32(out.numpy(), ref)
        assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"
    else:
        n, nrel, mabs = H.check_bf16(out.numpy(), ref)
        assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


def test_fused_forced_plan_fits_default_workspace(am, dev, tuner):
    """A plan forced to narrow slices (16-row groups, 32-dim slices, 1024
    workgroups, several per CU) runs in the workspace the size query reported
    without overrides, and gives the oracle's result."""
    import hip_rt
    B, Hh, Lq, Lk, D = 1, 4, 64, 64, 2048
    print("[case] fused forced narrow plan in the default workspace", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 613)
    ws = _ws(am, 0, B, Hh, Lq, Lk, D)
    tuner.set(fused_rows=16, fused_dc=32, fused_exchange="rsag")
    out = H.empty(Q.shape)
    am.attention_ex(q, k, v, out, workspace=ws)
    hip_rt.synchronize()
    assert am.sync_status(ws, B, Hh) == 0
    n, mabs, mrel = H.check_f32(out.numpy(), oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"


@pytest.mark.parametrize("shape,dtype,pe", [((1, 1, 32, 128, 8192), "bf16", "rope_half"),
                                            ((1, 2, 32, 32, 4096), "f32", "sinusoidal"),
                                            ((1, 1, 16, 16, 8192), "f32", "rope_inter"),
                                            ((1, 1, 64, 64, 2048), "bf16", "sinusoidal")],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else v)
def test_fused_planner_shapes_with_encoding(am, dev, shape, dtype, pe):
    """The few-workgroup, wide-slice plans with the positional encoding
    applied to Q and K at load: the oracle's result."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] fused planner shape {shape} {dtype} {pe}", flush=True)
    dcode = 0 if dtype == "f32" else 1
    desc = {"rope_half": am.make_pe("rope", pairing="half"), "rope_inter": am.make_pe("rope"),
            "sinusoidal": am.make_pe("sinusoidal")}[pe]
    assert am.path(dcode, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_FUSED_SMALL
    sigma = 0.5 if pe == "sinusoidal" else 1.0
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 523 + D, dtype, sigma)
    ws = _ws(am, dcode, B, Hh, Lq, Lk, D, desc)
    out = H.empty(Q.shape, dtype)
    am.attention_ex(q, k, v, out, pe=desc, workspace=ws)
    hip_rt.synchronize()
    assert am.sync_status(ws, B, Hh) == 0
    if pe == "sinusoidal":
        st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
        ref = oracle.attention_sinusoidal(Q, K, V, st, ct, nthreads=16)
    else:
        c, s_ = oracle.rope_cache(max(Lq, Lk), D)
        ref = oracle.attention_rope(Q, K, V, c, s_, nthreads=16,
                                    pairing="half" if pe == "rope_half" else "interleaved")
    if dtype == "f32":
        n, mabs, mrel = H.check_f32(out.numpy(), ref)
        assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"
    else:
        n, nrel, mabs = H.check_bf16(out.numpy(), ref)
        assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


def test_fused_exchange_scopes_share_one_workspace(am, dev, tuner):
    """One workspace, calls alternating between device-scope and XCD-local
    plans of different shapes (different slice counts per row group, so the
    XCD-local counters are shared by plans of different sizes) and both
    exchange forms: every call keeps the oracle's result, bit for bit from
    call to call, and no wait times out."""
    import hip_rt
    shapes = [(1, 4, 64, 64, 2048), (1, 8, 32, 64, 1024), (1, 3, 40, 72, 1024)]
    cases = []
    for i, shp in enumerate(shapes):
        B, Hh, Lq, Lk, D = shp
        (q, k, v), host = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 700 + i)
        cases.append((shp, (q, k, v), oracle.attention(*host, nthreads=16)))
    nbytes = max(am.workspace_bytes(0, *shp) for shp in shapes)
    ws = hip_rt.DeviceArray((nbytes // 4,), "f32", fill=0)
    first = {}
    plans = [("1", "gather", "16"), ("0", "gather", "16"), ("1", "rsag", "32"),
             ("0", "rsag", "16"), ("1", "rsag", "16"), ("1", "gather", "32")]
    for rnd in range(3):
        for xcd, ex, rows in plans:
            tuner.set(fused_xcd={"0": "device", "1": "xcd"}[xcd], fused_exchange=ex,
                      fused_rows=int(rows))
            for shp, ins, ref in cases:
                print(f"[case] shared workspace round {rnd} xcd={xcd} {ex} rows={rows} {shp}",
                      flush=True)
                out = H.empty(ref.shape)
                am.attention_ex(*ins, out, workspace=ws)
                hip_rt.synchronize()
                got = out.bits()
                n, mabs, mrel = H.check_f32(got, ref)
                assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"
                key = (xcd, ex, rows, shp)
                if key in first:
                    assert np.array_equal(first[key], got)
                else:
                    first[key] = got
    assert am.sync_status(ws, 1, 1) == 0


@pytest.mark.parametrize("xcd,exchange", [("0", "gather"), ("0", "rsag"), ("1", "gather"),
                                          ("1", "rsag")])
def test_fail_closed_then_recovers(am, dev, tuner, xcd, exchange):
    """The fail-closed path, forced from the host: the workspace's status word
    is preset (as a timed-out call would leave it), so every workgroup of the
    next call takes the fail-closed exit -- no wait is entered, every
    workgroup ends normally.  That call's outputs are NaN and
    atn_sync_status_ex reports ATN_ERR_DEVICE_TIMEOUT once (clearing the word
    and moving the epochs on); the call after it gives the oracle's result,
    on device-scope and XCD-local plans, one gather and reduce-scatter."""
    import hip_rt
    tuner.set(fused_xcd={"0": "device", "1": "xcd"}[xcd], fused_exchange=exchange, fused_rows=16)
    B, Hh, Lq, Lk, D = 1, 4, 64, 64, 2048
    print(f"[case] fail closed xcd={xcd} {exchange}", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 808)
    ref = oracle.attention(Q, K, V, nthreads=16)
    ws = _ws(am, 0, B, Hh, Lq, Lk, D)
    out = H.empty(Q.shape)
    am.attention_ex(q, k, v, out, workspace=ws)  # one good call first
    hip_rt.synchronize()
    assert am.sync_status(ws, B, Hh) == 0
    word = np.zeros(ws.shape, dtype=np.float32)
    word[...] = ws.bits()
    word.view(np.uint32)[0] = 1  # the status word, as a timeout leaves it
    ws.upload(word)
    out.fill_nan()
    am.attention_ex(q, k, v, out, workspace=ws)
    hip_rt.synchronize()
    got = out.numpy()
    assert np.isnan(got).all(), "fail-closed call wrote non-NaN outputs"
    assert am.sync_status(ws, B, Hh) == am.ATN_ERR_DEVICE_TIMEOUT
    assert am.sync_status(ws, B, Hh) == 0  # reported once
    for _ in range(3):
        out.fill_nan()
        am.attention_ex(q, k, v, out, workspace=ws)
        hip_rt.synchronize()
        n, mabs, mrel = H.check_f32(out.numpy(), ref)
        assert n == 0, f"after recovery: {n} mismatches, max abs {mabs}"
    assert am.sync_status(ws, B, Hh) == 0


@pytest.mark.parametrize("dtype,shape", [("f32", (1, 4, 64, 64, 2048)), ("bf16", (1, 4, 32, 128, 8192))],
                         ids=["cfg2-f32", "cfg3-bf16"])
def test_dropin_reruns_after_a_failed_exchange(am, dev, tuner, dtype, shape):
    """A synchronous drop-in whose single-launch call fails closed -- forced
    from the host: the test control atn_tuning.preset_status presets the
    call's status word as a timed-out call leaves it, so every workgroup
    takes the fail-closed exit and no wait is entered -- recovers the
    workspace and runs the call once more without the single-launch kernel:
    the process goes on, the output is the oracle's and the rerun is
    counted.  Without the control the next drop-in takes the single-launch
    kernel again."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] drop-in rerun {dtype} {shape}", flush=True)
    assert am.path(0 if dtype == "f32" else 1, B, Hh, Lq, Lk, D) == am.ATN_PATH_FUSED_SMALL
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 909, dtype)
    ref = oracle.attention(Q, K, V, nthreads=16)
    fn = am.attention_forward_optimized if dtype == "f32" else am.attention_forward_bf16
    check = H.check_f32 if dtype == "f32" else H.check_bf16

    def call():
        out = H.empty((B, Hh, Lq, D), dtype)
        fn(q, k, v, out)
        hip_rt.synchronize()
        n, a, b = check(out.numpy(), ref)
        assert n == 0, (n, a, b)
        return out.numpy()

    am.rerun_count(reset=True)
    tuner.set(preset_status=True)
    rerun = call()
    tuner.clear()
    assert am.rerun_count(reset=True) == 1
    again = call()
    assert am.rerun_count() == 0
    assert am.sync_status(None, B, Hh) == 0
    if dtype == "f32":  # the single-launch kernel and the split-D pipeline agree to the bar only
        n, mabs, _ = H.check_f32(rerun, again)
        assert n == 0, mabs
