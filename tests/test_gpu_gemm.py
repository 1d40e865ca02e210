"""GPU parity of the long-sequence bf16 path (MFMA QK^T GEMM, row softmax,
MFMA PV GEMM) against the CPU oracle.

bf16 bar: within rel 2e-2 of the fp32 oracle run on the bf16-rounded inputs
(elementwise against |ref| and rms(ref), and norm-wise).  Shapes cover the
256 x 256 tile edges (ragged Lq, Lk, D), every positional encoding, and the
per-head shapes of BASELINE configs 4 and 5 (two heads each, rows sampled
for the oracle).
"""
import numpy as np
import pytest

import helpers as H
import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _gemm_path(tuner):
    """bf16 calls at head_d <= 128 take the flash kernel by default (its own
    tests cover it): these tests hold them on the GEMM path."""
    tuner.set(no_flash=True)


def _ref(pe, Q, K, V, Lq, Lk, D, rows=None):
    if pe == "none":
        return oracle.attention(Q, K, V, rows=rows, nthreads=16)
    if pe == "sinusoidal":
        st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
        return oracle.attention_sinusoidal(Q, K, V, st, ct, rows=rows, nthreads=16)
    c, s = oracle.rope_cache(max(Lq, Lk), D)
    return oracle.attention_rope(Q, K, V, c, s, pairing="half" if pe == "rope_half"
                                 else "interleaved", rows=rows, nthreads=16)


def _desc(am, pe):
    return {"none": None, "rope_half": am.make_pe("rope", pairing="half"),
            "rope_inter": am.make_pe("rope"), "sinusoidal": am.make_pe("sinusoidal")}[pe]


SHAPES = [(1, 2, 128, 128, 64), (1, 2, 256, 384, 256), (2, 1, 300, 200, 136),
          (1, 1, 129, 520, 512)]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("pe", ["none", "rope_half", "rope_inter", "sinusoidal"])
def test_gemm_path(am, dev, shape, pe):
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] gemm path {shape} {pe}", flush=True)
    desc = _desc(am, pe)
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM
    sigma = 0.5 if pe == "sinusoidal" else 1.0
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 101 + D, "bf16",
                                           sigma)
    out = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    ref = _ref(pe, Q, K, V, Lq, Lk, D)
    n, nrel, mabs = H.check_bf16(out.numpy(), ref)
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("cfg", ["cfg4", "cfg5"])
def test_gemm_baseline_head_shapes(am, dev, cfg):
    """Per-head shapes of BASELINE config 4 (RoPE rotate-half, 1024 x 1024,
    D = 4096) and config 5 (sinusoidal, 256 -> 2048, D = 1024, sigma 0.5),
    two heads each; the oracle checks 24 sampled query rows per head."""
    import hip_rt
    if cfg == "cfg4":
        B, Hh, Lq, Lk, D, pe, sigma = 1, 2, 1024, 1024, 4096, "rope_half", 1.0
    else:
        B, Hh, Lq, Lk, D, pe, sigma = 1, 2, 256, 2048, 1024, "sinusoidal", 0.5
    print(f"[case] gemm {cfg} head shape", flush=True)
    desc = _desc(am, pe)
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 7, "bf16", sigma)
    out = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    got = out.numpy().reshape(-1, D)
    rng = np.random.default_rng(3)
    for h in range(B * Hh):
        rows = np.sort(rng.choice(Lq, 24, replace=False)) + h * Lq
        ref = np.concatenate([_ref(pe, Q, K, V, Lq, Lk, D, rows=(int(r), int(r) + 1))
                              .reshape(-1, D)[r:r + 1] for r in rows])
        n, nrel, mabs = H.check_bf16(got[rows], ref)
        assert n == 0, f"head {h}: normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("shape", [(1, 1, 160, 2312, 64), (1, 2, 128, 4096, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemm_path_long_key_rows(am, dev, shape):
    """More than eight 256-key tiles per score row: the PV GEMM takes the
    softmax factors with each A chunk instead of from its LDS table."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] gemm long key rows {shape}", flush=True)
    assert am.path(1, B, Hh, Lq, Lk, D) == am.ATN_PATH_GEMM
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 211 + Lk, "bf16")
    out = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, out)
    hip_rt.synchronize()
    n, nrel, mabs = H.check_bf16(out.numpy(), _ref("none", Q, K, V, Lq, Lk, D))
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("shape,pe", [((2, 8, 300, 512, 2304), "none"),
                                      ((2, 8, 300, 512, 2304), "rope_half"),
                                      ((4, 16, 512, 512, 1024), "none")],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else v)
def test_gemm_pv_more_tiles_than_cus(am, dev, shape, pe):
    """More PV output tiles than compute units (288 and 512 tiles): the
    persistent PV workgroups take several tiles each, the next tile's loads
    overlapping the previous tile's output stores; 2304 columns and 300 rows
    mix edge and interior tiles within one workgroup's sequence."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] gemm pv persistent {shape} {pe}", flush=True)
    desc = _desc(am, pe)
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 307 + D, "bf16")
    out = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    n, nrel, mabs = H.check_bf16(out.numpy(), _ref(pe, Q, K, V, Lq, Lk, D))
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("pe,sigma", [("none", 3.0), ("rope_half", 1.0)])
def test_gemm_path_wide_score_range(am, dev, pe, sigma):
    """Scores spread widely: one 256-key tile of keys is scaled x4, so in
    many rows the other tiles sit far below the row maximum (with sigma 3
    their softmax factors underflow to zero) while the maximum moves between
    tiles from row to row.  Exact bf16 operands take sigma 3 (logits up to
    ~+-40); the fp16-encoded RoPE operands take the config-4 input scale
    (their per-element rounding of 2^-12 grows the logit error with the
    logits' size)."""
    import hip_rt
    B, Hh, Lq, Lk, D = 1, 2, 200, 1104, 256
    print(f"[case] gemm wide score range {pe} sigma {sigma}", flush=True)
    rng = np.random.default_rng(17)
    Qf = rng.standard_normal((B, Hh, Lq, D), dtype=np.float32) * np.float32(sigma)
    Kf = rng.standard_normal((B, Hh, Lk, D), dtype=np.float32) * np.float32(sigma)
    Kf[:, :, 300:556] *= 4.0  # one tile of keys with much larger scores
    Vf = rng.standard_normal((B, Hh, Lk, D), dtype=np.float32)
    q, k, v = (hip_rt.DeviceArray.from_numpy(x, "bf16") for x in (Qf, Kf, Vf))
    Q, K, V = (t.numpy() for t in (q, k, v))
    desc = _desc(am, pe)
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM
    out = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    n, nrel, mabs = H.check_bf16(out.numpy(), _ref(pe, Q, K, V, Lq, Lk, D))
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("shape,pe", [((1, 2, 256, 512, 256), "sinusoidal"),
                                      ((1, 1, 1280, 256, 128), "rope_half"),
                                      ((1, 2, 256, 384, 136), "none")],
                         ids=["fusedK", "qkdma-encK", "register-stage"])
def test_gemm_graph_replays_match_eager(am, dev, shape, pe):
    """Captured HIP graph of three calls on one workspace, replayed four times
    with eager work and synchronizations in between: every replay equals the
    eager result bit for bit.  The shapes take the K encoding inside the
    QK^T GEMM, the K~ pass with the both-tiles-in-LDS QK^T GEMM (five query
    tiles: past the fused encoding's limit of four), and the register-staged
    GEMMs."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] gemm graph replay {shape} {pe}", flush=True)
    desc = _desc(am, pe)
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 77, "bf16",
                                           0.5 if pe == "sinusoidal" else 1.0)
    nb = am.workspace_bytes(am.ATN_DTYPE_BF16, B, Hh, Lq, Lk, D, desc)
    ws = hip_rt.DeviceArray.from_numpy(np.zeros(nb // 4 + 1, np.float32), "f32")
    st = hip_rt.Stream()
    eager = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, eager, pe=desc, workspace=ws, stream=st)
    st.synchronize()
    ref = eager.bits()
    outs = [H.empty(Q.shape, "bf16") for _ in range(3)]
    g = hip_rt.Graph(st, lambda: [am.attention_ex(q, k, v, o, pe=desc, workspace=ws, stream=st)
                                  for o in outs])
    for rep in range(4):
        for o in outs:
            o.fill_nan()
        hip_rt.synchronize()
        g.launch()
        st.synchronize()
        for o in outs:
            assert np.array_equal(o.bits(), ref), f"replay {rep} differs from eager"
        am.attention_ex(q, k, v, eager, pe=desc, workspace=ws, stream=st)
        st.synchronize()
        assert np.array_equal(eager.bits(), ref)
    g.destroy()
    st.destroy()
    n, nrel, mabs = H.check_bf16(eager.numpy(), _ref(pe, Q, K, V, Lq, Lk, D))
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


GAP_SHAPES = [(1, 8, 64, 4096, 2048), (1, 4, 100, 100, 2048), (1, 2, 16, 300, 256),
              (2, 3, 70, 40, 128), (1, 1, 1, 200, 64), (1, 2, 200, 20, 512)]


@pytest.mark.parametrize("shape", GAP_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("pe", ["none", "rope_half", "sinusoidal"])
def test_gemm_path_covers_gap_shapes(am, dev, shape, pe):
    """bf16 shapes outside the single-launch window (len_q <= 64 with
    len_k > 128, or 64 < len_q < 128) and below 128 rows or keys, including
    key counts that are not a multiple of 8 (E rows padded to 8 keys, the
    padding written as zeros): they run on the MFMA GEMM path, not the VALU
    split-D pipeline, and match the oracle."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] gemm gap shape {shape} {pe}", flush=True)
    desc = _desc(am, pe)
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM
    sigma = 0.5 if pe == "sinusoidal" else 1.0
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 313 + Lk, "bf16",
                                           sigma)
    out = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    rows = None if B * Hh * Lq <= 512 else (0, 64)
    ref = _ref(pe, Q, K, V, Lq, Lk, D, rows=rows)
    got = out.numpy()
    if rows is not None:
        got, ref = got.reshape(-1, D)[rows[0]:rows[1]], ref.reshape(-1, D)[rows[0]:rows[1]]
    n, nrel, mabs = H.check_bf16(got, ref)
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"
