"""The flash kernel (fp32 and bf16, head_d <= 256, any sequence length;
flash.hip) against the CPU oracle: tile edges of the key loop, head dims
padded to the kernel's 32/64/128/256 forms, query blocks past the sequence,
positional encodings applied at load, wide logits, values outside fp16's
range (power-of-two linearity), and agreement with the split-D pipeline
(fp32) and the GEMM path (bf16) on the same inputs.  The reference's own
long-sequence test shape (4, 32, 512, 512, 128) (final/attention.cu:522)
runs here too, as in test_gpu_parity.py.

fp32 bar: the reference's (abs and rel above 1e-4).  bf16 bar: within rel
2e-2 of the fp32 oracle run on the bf16-rounded inputs (helpers.check_bf16).
"""
import numpy as np
import pytest

import helpers as H
import oracle

pytestmark = pytest.mark.gpu


def _f32_call(am, Q, K, V, desc=None):
    (q, k, v) = (H.upload(x) for x in (Q, K, V))
    out = H.empty(Q.shape)
    am.attention_ex(q, k, v, out, pe=desc)
    import hip_rt
    hip_rt.synchronize()
    return out.numpy()


def _bf16(x):
    """x rounded to bf16 (nearest even), as float32."""
    import hip_rt
    return hip_rt.bf16_bits_to_f32(hip_rt.f32_to_bf16_bits(np.ascontiguousarray(x)))


def _bf16_call(am, Q, K, V, desc=None):
    """One bf16 call on the bf16 roundings of Q, K, V (the caller passes
    already-rounded values, so the oracle sees what the kernel sees)."""
    import hip_rt
    (q, k, v) = (H.upload(x, "bf16") for x in (Q, K, V))
    out = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    got = out.numpy()
    for x in (q, k, v, out):
        x.free()
    return got


def _ref(pe, Q, K, V, **kw):
    L, D = max(Q.shape[2], K.shape[2]), Q.shape[3]
    if pe == "sinusoidal":
        st, ct = oracle.sinusoidal_table(L, D)
        return oracle.attention_sinusoidal(Q, K, V, st, ct, nthreads=16, **kw)
    if pe in ("rope", "rope_half"):
        c, s = oracle.rope_cache(L, D)
        return oracle.attention_rope(Q, K, V, c, s, rotary_dim=D, nthreads=16,
                                     pairing="half" if pe == "rope_half" else "interleaved", **kw)
    return oracle.attention(Q, K, V, nthreads=16, **kw)


# key lengths around the 64- and 32-key tiles, query lengths around the
# 64-row blocks, head dims at and below each padded form
_SHAPES = [
    (1, 2, 65, 1, 64), (1, 2, 65, 63, 64), (1, 2, 65, 64, 64), (1, 2, 70, 65, 64),
    (1, 3, 130, 129, 32), (1, 1, 200, 300, 128), (1, 2, 129, 513, 100), (1, 1, 80, 1025, 60),
    (1, 2, 96, 200, 256), (1, 1, 70, 65, 200), (1, 1, 65, 33, 160), (2, 3, 100, 140, 8),
    (1, 4, 512, 512, 128), (1, 300, 16, 16, 64),
]


@pytest.mark.parametrize("shape", _SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_flash_f32(am, dev, shape):
    B, Hh, Lq, Lk, D = shape
    print(f"[case] flash f32 {shape}", flush=True)
    assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_FLASH
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=500 + Lk + D)
    got = _f32_call(am, Q, K, V)
    ref = oracle.attention(Q, K, V, nthreads=16)
    n, mabs, mrel = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"


@pytest.mark.parametrize("form", ["4x16", "8x16", "4x32", "8x32"])
@pytest.mark.parametrize("shape,pe", [((1, 3, 130, 129, 32), None), ((1, 2, 200, 300, 128), None),
                                      ((1, 2, 96, 200, 256), None), ((1, 2, 129, 97, 64), "rope"),
                                      ((1, 2, 150, 333, 128), "sinusoidal")],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_flash_workgroup_forms(am, dev, tuner, form, shape, pe):
    """Every workgroup form forced on the same inputs: 4 waves of 16 query
    rows, 8 of 16, 4 of 32 and 8 of 32 (16 x 16 x 32 or 32 x 32 x 16 MFMA
    tiles; 64-, 128-, 128- and 256-row query blocks; key tiles of at least
    one load round); head_d 256 runs 8 of 16 whatever is forced."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] flash f32 form {form} {shape} {pe}", flush=True)
    tuner.set(flash_form=form)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=7 + Lk + len(form),
                           sigma=0.5 if pe == "sinusoidal" else 1.0)
    desc = None if pe is None else am.make_pe(pe)
    got = _f32_call(am, Q, K, V, desc)
    L = max(Lq, Lk)
    if pe == "sinusoidal":
        st, ct = oracle.sinusoidal_table(L, D)
        ref = oracle.attention_sinusoidal(Q, K, V, st, ct, nthreads=16)
    elif pe == "rope":
        c, s = oracle.rope_cache(L, D)
        ref = oracle.attention_rope(Q, K, V, c, s, rotary_dim=D, nthreads=16)
    else:
        ref = oracle.attention(Q, K, V, nthreads=16)
    n, mabs, mrel = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"


@pytest.mark.parametrize("form", ["4x16", "8x16", "4x32", "8x32"])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_flash_tile_counts(am, dev, tuner, form, D):
    """Key lengths of 2 to 17 tiles, two seeds each, both workgroup forms.
    Regression: a build whose softmax read the QK^T accumulators through an
    inline-asm max (which the compiler's MFMA hazard waits do not cover)
    gave wrong rows scattered over these cases whenever the schedule put
    that read right behind the MFMAs."""
    tuner.set(flash_form=form)
    B, Hh, Lq = 1, 2, 70
    for Lk in (65, 70, 96, 97, 128, 129, 200, 513):
        for seed in (1, 2):
            print(f"[case] flash f32 form {form} D={D} Lk={Lk} seed={seed}", flush=True)
            Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=seed * 1000 + Lk + D)
            got = _f32_call(am, Q, K, V)
            n, mabs, mrel = H.check_f32(got, oracle.attention(Q, K, V, nthreads=16))
            assert n == 0, f"Lk={Lk} seed={seed}: {n} mismatches, max abs {mabs}"


def test_flash_reference_long_shape(am, dev):
    """The reference's long-sequence test shape (final/attention.cu:522)."""
    B, Hh, L, D = 4, 32, 512, 128
    print("[case] flash f32 (4,32,512,512,128)", flush=True)
    assert am.path(0, B, Hh, L, L, D) == am.ATN_PATH_FLASH
    Q, K, V = H.rng_inputs((B, Hh, L, D), (B, Hh, L, D), seed=522)
    got = _f32_call(am, Q, K, V)
    n, mabs, mrel = H.check_f32(got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"


@pytest.mark.parametrize("shape", [(1, 2, 200, 300, 128), (1, 1, 96, 200, 256)],
                         ids=lambda s: "x".join(map(str, s)))
def test_flash_wide_logits(am, dev, shape):
    """sigma 3 inputs (logits to about +-40, scores spread over many key
    tiles, so the running maximum moves between tiles)."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] flash f32 sigma 3 {shape}", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=77 + D, sigma=3.0)
    got = _f32_call(am, Q, K, V)
    n, mabs, _ = H.check_f32(got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"{n} mismatches, max abs {mabs}"


def test_flash_increasing_scores(am, dev):
    """Scores that grow key tile by key tile (each tile's maximum above the
    last), so every tile rescales the running output by exp(m_old - m_new)."""
    B, Hh, Lq, Lk, D = 1, 2, 64, 512, 64
    print("[case] flash f32 rising scores", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=91)
    Q[..., 0] = np.abs(Q[..., 0]) + 1.0  # a positive first coordinate,
    Q[..., 1:] *= np.float32(0.1)        # which dominates each score
    K[..., 0] = np.linspace(-40, 40, Lk, dtype=np.float32)[None, None, :]
    got = _f32_call(am, Q, K, V)
    n, mabs, _ = H.check_f32(got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"{n} mismatches, max abs {mabs}"


@pytest.mark.parametrize("exps", [(17, -17, 0), (0, 0, 19), (-12, -12, -12), (17, -17, 21),
                                  (4, -4, 0), (5, -5, 0), (30, 10, 0)],
                         ids=["qk-big", "v-big", "all-small", "all-big", "k-plain-low",
                              "k-scaled-low", "logits-huge"])
def test_flash_outside_fp16_range(am, dev, exps):
    """Head 1 scaled by powers of two (exact, so the oracle on the unscaled V
    times 2^ev is the reference): K tiles carry a power-of-two scale when
    their largest magnitude lies outside [2^-3, 65504) (k-plain-low puts it
    near 2^-2, unscaled; k-scaled-low near 2^-3, either side), V tiles one
    only beyond fp16's range, carried into the running output.  logits-huge
    puts head 1's logits near 2^40, where the softmax subtracts the running
    max from each score before scaling it (as the oracle does)."""
    B, Hh, Lq, Lk, D = 1, 3, 100, 300, 128
    eq, ek, ev = exps
    print(f"[case] flash f32 scaled 2^{exps}", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=31)
    Q[:, 1] *= np.float32(2.0 ** eq)
    K[:, 1] *= np.float32(2.0 ** ek)
    Vs = V.copy()
    Vs[:, 1] *= np.float32(2.0 ** ev)
    got = _f32_call(am, Q, K, Vs)
    assert np.isfinite(got).all()
    got[:, 1] *= np.float32(2.0 ** -ev)
    n, mabs, mrel = H.check_f32(got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"


def test_flash_nonfinite_inputs_propagate(am, dev, tuner):
    """As in the reference: an infinite query element makes its own output
    row non-finite, a NaN value element its output column NaN; every other
    element keeps the bar (the tile scales take finite magnitudes only)."""
    for form in ("8x16", "8x32"):
        B, Hh, Lq, Lk, D = 1, 2, 300, 333, 128
        print(f"[case] flash f32 non-finite inputs, form {form}", flush=True)
        tuner.set(flash_form=form)
        Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=71)
        Q[0, 1, 5, 100] = np.inf
        V[0, 0, 200, 33] = np.nan
        got = _f32_call(am, Q, K, V)
        ref = oracle.attention(Q, K, V, nthreads=16)
        assert not np.isfinite(ref[0, 1, 5]).any() and not np.isfinite(got[0, 1, 5]).any()
        assert np.isnan(ref[0, 0, :, 33]).all() and np.isnan(got[0, 0, :, 33]).all()
        keep = np.ones((Hh, Lq, D), dtype=bool)
        keep[1, 5, :] = False
        keep[0, :, 33] = False
        n, mabs, _ = H.check_f32(got[0][keep], ref[0][keep])
        assert n == 0, mabs


def test_flash_v_scale_changes_between_tiles(am, dev):
    """One key tile of V beyond fp16's range among ordinary ones: its scale
    differs from its neighbours', and the running output is carried across
    the change in both directions."""
    B, Hh, Lq, Lk, D = 1, 1, 64, 256, 64
    print("[case] flash f32 V scale change", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=33, sigma=0.3)
    V[:, :, 64:128] *= np.float32(2.0 ** 18)
    got = _f32_call(am, Q, K, V)
    ref = oracle.attention(Q, K, V, nthreads=16)
    # outputs mix values of 2^18 and 1: compare in units of the largest
    n, mabs, _ = H.check_f32(got / 2.0 ** 18, ref / 2.0 ** 18)
    assert n == 0, f"{n} mismatches, max abs {mabs} (units of 2^18)"


@pytest.mark.parametrize("pe,rot,aq,ak", [("rope", 0, True, True), ("rope", 48, True, True),
                                          ("rope_half", 0, True, True),
                                          ("sinusoidal", 0, True, True),
                                          ("rope", 0, True, False), ("sinusoidal", 0, False, True)],
                         ids=["rope", "rope-partial", "rope-half", "sin", "rope-q", "sin-k"])
def test_flash_encodings(am, dev, pe, rot, aq, ak):
    B, Hh, Lq, Lk, D = 1, 2, 150, 333, 128
    print(f"[case] flash f32 {pe} rot={rot} q={aq} k={ak}", flush=True)
    desc = {"rope": am.make_pe("rope", rotary_dim=rot, apply_q=aq, apply_k=ak),
            "rope_half": am.make_pe("rope", pairing="half", apply_q=aq, apply_k=ak),
            "sinusoidal": am.make_pe("sinusoidal", apply_q=aq, apply_k=ak)}[pe]
    assert am.path(0, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_FLASH
    sigma = 0.5 if pe == "sinusoidal" else 1.0
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=61, sigma=sigma)
    got = _f32_call(am, Q, K, V, desc)
    L = max(Lq, Lk)
    if pe == "sinusoidal":
        st, ct = oracle.sinusoidal_table(L, D)
        ref = oracle.attention_sinusoidal(Q, K, V, st, ct, add_q=aq, add_k=ak, nthreads=16)
    else:
        r = rot or D
        c, s = oracle.rope_cache(L, r)
        ref = oracle.attention_rope(Q, K, V, c, s, rotary_dim=r,
                                    pairing="half" if pe == "rope_half" else "interleaved",
                                    rotate_q=aq, rotate_k=ak, nthreads=16)
    n, mabs, _ = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}"


@pytest.mark.parametrize("shape", [(1, 4, 200, 200, 128), (1, 2, 65, 1025, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_flash_matches_split_d(am, dev, tuner, shape):
    """The flash kernel and the split-D pipeline (forced with
    atn_tuning.no_flash) on the same inputs, both against the oracle."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] flash vs split-D {shape}", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=3 + Lk)
    ref = oracle.attention(Q, K, V, nthreads=16)
    got_f = _f32_call(am, Q, K, V)
    tuner.set(no_flash=True)
    assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_SPLIT_D
    got_s = _f32_call(am, Q, K, V)
    for got in (got_f, got_s):
        n, mabs, _ = H.check_f32(got, ref)
        assert n == 0, mabs
    n, mabs, _ = H.check_f32(got_f, got_s)
    assert n == 0, mabs


def test_flash_graph_replays(am, dev):
    """Captured HIP graph of flash calls replayed with eager work between the
    replays: every replay equals the eager result bit for bit."""
    import hip_rt
    B, Hh, Lq, Lk, D = 1, 4, 200, 300, 128
    print("[case] flash graph replay", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 95)
    st = hip_rt.Stream()
    eager = H.empty(Q.shape)
    am.attention_ex(q, k, v, eager, stream=st)
    st.synchronize()
    ref = eager.bits()
    outs = [H.empty(Q.shape) for _ in range(2)]
    g = hip_rt.Graph(st, lambda: [am.attention_ex(q, k, v, o, stream=st) for o in outs])
    for _ in range(3):
        for o in outs:
            o.fill_nan()
        hip_rt.synchronize()
        g.launch()
        st.synchronize()
        for o in outs:
            assert np.array_equal(o.bits(), ref)
        am.attention_ex(q, k, v, eager, stream=st)
        st.synchronize()
    g.destroy()
    n, mabs, _ = H.check_f32(ref, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, mabs
    st.destroy()


# ---------------------------------------------------------------- bf16
# bf16 inputs are exact in fp16 wherever a power-of-two scale brings a tile
# there, so the kernel stages one fp16 part per operand (64-key tiles in
# every form) and makes one product where fp32 makes three; P goes in as one
# fp16 part and the output is rounded to bf16.

_BF16_SHAPES = [
    (1, 2, 65, 1, 64), (1, 2, 65, 64, 64), (1, 2, 70, 65, 64), (1, 3, 130, 129, 32),
    (1, 1, 200, 300, 128), (1, 2, 129, 513, 100), (1, 1, 80, 1025, 60), (2, 3, 100, 140, 8),
    (1, 2, 96, 200, 252), (1, 1, 70, 65, 196), (1, 300, 16, 16, 64), (1, 1, 2, 3000, 128),
    (1, 2, 96, 200, 256), (1, 1, 70, 300, 200), (2, 2, 129, 513, 136),
]


@pytest.mark.parametrize("shape", _BF16_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_flash_bf16(am, dev, shape):
    """bf16 calls outside the single-launch window with head_d <= 256."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] flash bf16 {shape}", flush=True)
    assert am.path(1, B, Hh, Lq, Lk, D) == am.ATN_PATH_FLASH
    Q, K, V = (_bf16(x) for x in H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=900 + Lk + D))
    got = _bf16_call(am, Q, K, V)
    n, nrel, mabs = H.check_bf16(got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"{n} failures, normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("form", ["4x16", "8x16", "4x32", "8x32"])
@pytest.mark.parametrize("shape,pe", [((1, 3, 130, 129, 32), None), ((1, 2, 200, 300, 128), None),
                                      ((1, 2, 96, 200, 252), None), ((1, 2, 129, 97, 64), "rope"),
                                      ((1, 2, 150, 333, 128), "rope_half"),
                                      ((1, 2, 150, 333, 128), "sinusoidal")],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_flash_bf16_forms(am, dev, tuner, form, shape, pe):
    """Every workgroup form forced, bf16, with and without an encoding
    (head_d 252: the 256-wide form, which the library takes where the GEMM
    path does not run; past head_d 128 every form runs 8 waves of 16 rows)."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] flash bf16 form {form} {shape} {pe}", flush=True)
    tuner.set(flash_form=form)
    Q, K, V = (_bf16(x) for x in H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=17 + Lk,
                                              sigma=0.5 if pe == "sinusoidal" else 1.0))
    desc = {None: None, "rope": am.make_pe("rope"),
            "rope_half": am.make_pe("rope", pairing="half"),
            "sinusoidal": am.make_pe("sinusoidal")}[pe]
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_FLASH
    got = _bf16_call(am, Q, K, V, desc)
    n, nrel, mabs = H.check_bf16(got, _ref(pe, Q, K, V))
    assert n == 0, f"{n} failures, normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("form", ["8x16", "8x32"])
@pytest.mark.parametrize("D", [32, 64, 128])
def test_flash_bf16_tile_counts(am, dev, tuner, form, D):
    """Key lengths of 1 to 9 64-key tiles and the edges between them."""
    tuner.set(flash_form=form)
    B, Hh, Lq = 1, 2, 70
    for Lk in (63, 64, 65, 127, 128, 129, 257, 513):
        print(f"[case] flash bf16 form {form} D={D} Lk={Lk}", flush=True)
        Q, K, V = (_bf16(x) for x in H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D),
                                                  seed=3000 + Lk + D))
        got = _bf16_call(am, Q, K, V)
        n, nrel, mabs = H.check_bf16(got, oracle.attention(Q, K, V, nthreads=16))
        assert n == 0, f"Lk={Lk}: {n} failures, normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("exps", [(30, -30, 0), (0, 0, 40), (0, 0, -40), (-20, -20, -20),
                                  (20, 20, 20), (3, -3, 0), (0, -5, -3)],
                         ids=["qk-big", "v-big", "v-small", "all-small", "all-big",
                              "k-scaled-low", "k-and-v-low"])
def test_flash_bf16_outside_fp16_range(am, dev, exps):
    """bf16's range is fp32's: head 1 scaled by powers of two far outside
    fp16's (exact, so the oracle on the unscaled V times 2^ev is the
    reference).  Q takes a scale per wave, K and V one per key tile whenever
    the tile's largest magnitude lies outside [2^-3, 65504), so that small
    values keep their bits in the one fp16 part too; all-big puts head 1's
    logits near 2^40 (the softmax's exact form)."""
    B, Hh, Lq, Lk, D = 1, 3, 100, 300, 128
    eq, ek, ev = exps
    print(f"[case] flash bf16 scaled 2^{exps}", flush=True)
    Q, K, V = (_bf16(x) for x in H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=37))
    Q[:, 1] *= np.float32(2.0 ** eq)
    K[:, 1] *= np.float32(2.0 ** ek)
    Vs = V.copy()
    Vs[:, 1] *= np.float32(2.0 ** ev)
    got = _bf16_call(am, Q, K, Vs)
    assert np.isfinite(got).all()
    got[:, 1] *= np.float32(2.0 ** -ev)
    n, nrel, mabs = H.check_bf16(got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"{n} failures, normwise rel {nrel}, max abs {mabs}"


def test_flash_bf16_wide_logits_and_rising_scores(am, dev):
    """sigma 3 inputs (logits to about +-40), and scores that rise key tile
    by key tile, so that the running maximum moves and the output is
    rescaled between tiles."""
    B, Hh, Lq, Lk, D = 1, 2, 200, 600, 128
    print("[case] flash bf16 sigma 3", flush=True)
    Q, K, V = (_bf16(x) for x in H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=79, sigma=3.0))
    got = _bf16_call(am, Q, K, V)
    n, nrel, mabs = H.check_bf16(got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"sigma 3: {n} failures, normwise rel {nrel}, max abs {mabs}"
    print("[case] flash bf16 rising scores", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, 64, 64), (B, Hh, 512, 64), seed=93)
    Q[..., 0] = np.abs(Q[..., 0]) + 1.0
    Q[..., 1:] *= np.float32(0.1)
    K[..., 0] = np.linspace(-40, 40, 512, dtype=np.float32)[None, None, :]
    Q, K, V = _bf16(Q), _bf16(K), _bf16(V)
    got = _bf16_call(am, Q, K, V)
    n, nrel, mabs = H.check_bf16(got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"rising: {n} failures, normwise rel {nrel}, max abs {mabs}"


def test_flash_bf16_nonfinite_inputs_propagate(am, dev, tuner):
    """An infinite query element makes its output row non-finite, a NaN
    value element its output column NaN; every other element keeps the bar."""
    for form in ("8x16", "8x32"):
        B, Hh, Lq, Lk, D = 1, 2, 300, 333, 128
        print(f"[case] flash bf16 non-finite inputs, form {form}", flush=True)
        tuner.set(flash_form=form)
        Q, K, V = (_bf16(x) for x in H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=73))
        Q[0, 1, 5, 100] = np.inf
        V[0, 0, 200, 33] = np.nan
        got = _bf16_call(am, Q, K, V)
        ref = oracle.attention(Q, K, V, nthreads=16)
        assert not np.isfinite(got[0, 1, 5]).any() and np.isnan(got[0, 0, :, 33]).all()
        keep = np.ones((Hh, Lq, D), dtype=bool)
        keep[1, 5, :] = False
        keep[0, :, 33] = False
        n, nrel, mabs = H.check_bf16(got[0][keep], ref[0][keep])
        assert n == 0, (nrel, mabs)


@pytest.mark.parametrize("shape,pe", [((1, 4, 200, 200, 128), None), ((1, 2, 65, 1025, 64), None),
                                      ((1, 2, 300, 520, 128), "rope_half")],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_flash_bf16_matches_gemm_path(am, dev, tuner, shape, pe):
    """The bf16 flash kernel and the GEMM path (forced with
    atn_tuning.no_flash) on the same inputs: both within the bar of the
    oracle and of each other."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] flash bf16 vs GEMM {shape} {pe}", flush=True)
    desc = None if pe is None else am.make_pe("rope", pairing="half")
    Q, K, V = (_bf16(x) for x in H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=5 + Lk))
    ref = _ref(pe, Q, K, V)
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_FLASH
    got_f = _bf16_call(am, Q, K, V, desc)
    tuner.set(no_flash=True)
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM
    got_g = _bf16_call(am, Q, K, V, desc)
    for got in (got_f, got_g):
        n, nrel, mabs = H.check_bf16(got, ref)
        assert n == 0, (nrel, mabs)
    n, nrel, mabs = H.check_bf16(got_f, got_g)
    assert n == 0, (nrel, mabs)


def test_flash_bf16_graph_replays(am, dev):
    """Captured HIP graph of bf16 flash calls replayed with eager work
    between the replays: every replay equals the eager result bit for bit."""
    import hip_rt
    B, Hh, Lq, Lk, D = 1, 4, 200, 300, 128
    print("[case] flash bf16 graph replay", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 97, "bf16")
    st = hip_rt.Stream()
    eager = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, eager, stream=st)
    st.synchronize()
    ref = eager.bits()
    outs = [H.empty(Q.shape, "bf16") for _ in range(2)]
    g = hip_rt.Graph(st, lambda: [am.attention_ex(q, k, v, o, stream=st) for o in outs])
    for _ in range(3):
        for o in outs:
            o.fill_nan()
        hip_rt.synchronize()
        g.launch()
        st.synchronize()
        for o in outs:
            assert np.array_equal(o.bits(), ref)
        am.attention_ex(q, k, v, eager, stream=st)
        st.synchronize()
    g.destroy()
    n, nrel, mabs = H.check_bf16(eager.numpy(), oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, (nrel, mabs)
    st.destroy()


# ---------------------------------------------------------------- key splits
# A grid of few (head, query block) pairs leaves CUs idle: such calls split
# the keys into parts (whole 64-key chunks, two at least per part), each
# part writes its normalized output and statistics, and a second kernel
# merges them (weights 2^((m_s - M) c0 + g_s), maxima subtracted first).


def _call(am, dt, Q, K, V, desc=None):
    return _f32_call(am, Q, K, V, desc) if dt == "f32" else _bf16_call(am, Q, K, V, desc)


def _check(dt, got, ref):
    if dt == "f32":
        n, mabs, _ = H.check_f32(got, ref)
        return n, mabs
    n, nrel, mabs = H.check_bf16(got, ref)
    return n, (nrel, mabs)


@pytest.mark.parametrize("dt,shape", [("f32", (1, 4, 2048, 2048, 128)), ("bf16", (1, 4, 2048, 2048, 128)),
                                      ("bf16", (1, 32, 16, 4096, 128)), ("f32", (1, 8, 1, 3000, 64)),
                                      ("f32", (2, 2, 100, 5000, 256)), ("bf16", (1, 1, 200, 700, 252))],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else v)
def test_flash_split_auto(am, dev, dt, shape):
    """Shapes whose grid leaves CUs idle take key splits by themselves;
    against the oracle and against the same call with splits turned off."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] flash split auto {dt} {shape}", flush=True)
    code = 0 if dt == "f32" else 1
    assert am.path(code, B, Hh, Lq, Lk, D) == am.ATN_PATH_FLASH
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=4000 + Lk + D)
    if dt == "bf16":
        Q, K, V = _bf16(Q), _bf16(K), _bf16(V)
    got = _call(am, dt, Q, K, V)
    n, info = _check(dt, got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, info
    am.set_tuning(flash_split=1)
    try:
        whole = _call(am, dt, Q, K, V)
    finally:
        am.set_tuning()
    n, info = _check(dt, got, whole)
    assert n == 0, info


@pytest.mark.parametrize("dt,pe,shape", [("bf16", None, (1, 2, 300, 4100, 128)),
                                         ("bf16", "rope_half", (1, 2, 300, 4100, 128)),
                                         ("f32", "sinusoidal", (1, 1, 257, 4500, 96)),
                                         ("f32", None, (1, 2, 300, 4100, 128)),
                                         ("f32", None, (1, 2, 300, 4100, 64)),
                                         ("bf16", "rope", (1, 1, 100, 8200, 64))],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_flash_long_keys(am, dev, dt, pe, shape):
    """From 4096 keys on, grids below a workgroup per CU take 32-row waves
    with key splits (fp32 without an encoding at head_d <= 64 with 64-key
    tiles): ragged key and query lengths against the oracle."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] flash long keys {dt} {pe} {shape}", flush=True)
    desc = None if pe is None else (am.make_pe("rope", pairing="half") if pe == "rope_half"
                                    else am.make_pe(pe))
    code = 0 if dt == "f32" else 1
    assert am.path(code, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_FLASH
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=700 + D,
                           sigma=0.5 if pe == "sinusoidal" else 1.0)
    if dt == "bf16":
        Q, K, V = _bf16(Q), _bf16(K), _bf16(V)
    got = _call(am, dt, Q, K, V, desc)
    n, info = _check(dt, got, _ref(pe, Q, K, V))
    assert n == 0, info


@pytest.mark.parametrize("nsplit", [2, 3, 7])
@pytest.mark.parametrize("dt,pe,form", [("f32", None, "8x16"), ("bf16", None, "8x32"),
                                        ("f32", "rope", "4x16"), ("bf16", "rope_half", "8x16"),
                                        ("bf16", "sinusoidal", "4x32"), ("f32", "sinusoidal", "8x32")])
def test_flash_split_forced(am, dev, tuner, nsplit, dt, pe, form):
    """Forced split counts on ragged key lengths (the last part short), every
    form, with encodings (a part's keys keep their own positions)."""
    tuner.set(flash_split=nsplit, flash_form=form)
    desc = {None: None, "rope": am.make_pe("rope"), "rope_half": am.make_pe("rope", pairing="half"),
            "sinusoidal": am.make_pe("sinusoidal")}[pe]
    for (B, Hh, Lq, Lk, D) in ((1, 2, 70, 200, 64), (1, 3, 130, 1000, 128), (2, 1, 33, 450, 32)):
        print(f"[case] flash split {nsplit} {dt} {pe} {form} {(B, Hh, Lq, Lk, D)}", flush=True)
        Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=nsplit * 100 + Lk,
                               sigma=0.5 if pe == "sinusoidal" else 1.0)
        if dt == "bf16":
            Q, K, V = _bf16(Q), _bf16(K), _bf16(V)
        got = _call(am, dt, Q, K, V, desc)
        n, info = _check(dt, got, _ref(pe, Q, K, V))
        assert n == 0, (Lk, info)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_flash_split_huge_logits_and_nonfinite(am, dev, tuner, dt):
    """Splits merged with their maxima subtracted first: logits near 2^40
    (head 1) match the oracle; an infinite query element makes its row
    non-finite and a NaN value element its column NaN, the rest keeps the
    bar."""
    tuner.set(flash_split=4)
    B, Hh, Lq, Lk, D = 1, 3, 100, 900, 128
    print(f"[case] flash split huge logits {dt}", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=87)
    if dt == "bf16":
        Q, K, V = _bf16(Q), _bf16(K), _bf16(V)
    Q[:, 1] *= np.float32(2.0 ** 30)
    K[:, 1] *= np.float32(2.0 ** 10)
    got = _call(am, dt, Q, K, V)
    n, info = _check(dt, got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, info
    Q[0, 2, 5, 7] = np.inf
    V[0, 0, 600, 9] = np.nan
    got = _call(am, dt, Q, K, V)
    ref = oracle.attention(Q, K, V, nthreads=16)
    assert not np.isfinite(got[0, 2, 5]).any() and np.isnan(got[0, 0, :, 9]).all()
    keep = np.ones((Hh, Lq, D), dtype=bool)
    keep[2, 5, :] = False
    keep[0, :, 9] = False
    n, info = _check(dt, got[0][keep], ref[0][keep])
    assert n == 0, info


def test_flash_split_graph_replays(am, dev):
    """A captured graph of split calls (parts in the stream's workspace)
    replayed with eager calls between: every replay equals the eager result
    bit for bit."""
    import hip_rt
    B, Hh, Lq, Lk, D = 1, 2, 300, 3000, 128
    print("[case] flash split graph replay", flush=True)
    assert am.workspace_bytes(1, B, Hh, Lq, Lk, D) > 40960  # the parts need scratch
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 99, "bf16")
    st = hip_rt.Stream()
    eager = H.empty(Q.shape, "bf16")
    am.attention_ex(q, k, v, eager, stream=st)
    st.synchronize()
    ref = eager.bits()
    outs = [H.empty(Q.shape, "bf16") for _ in range(2)]
    g = hip_rt.Graph(st, lambda: [am.attention_ex(q, k, v, o, stream=st) for o in outs])
    for _ in range(3):
        for o in outs:
            o.fill_nan()
        hip_rt.synchronize()
        g.launch()
        st.synchronize()
        for o in outs:
            assert np.array_equal(o.bits(), ref)
        am.attention_ex(q, k, v, eager, stream=st)
        st.synchronize()
    g.destroy()
    n, nrel, mabs = H.check_bf16(eager.numpy(), oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, (nrel, mabs)
    st.destroy()
