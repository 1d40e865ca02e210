"""GPU parity: every drop-in entry point vs the CPU oracle on identical inputs.

fp32: element fails iff abs > 1e-4 AND rel > 1e-4.
bf16: within rel 2e-2 of the fp32 oracle run on the bf16-rounded inputs.
Shapes follow the reference's own test lists (final/attention.cu:490-522,
final/rope.cu:1911-1923, final/sinusoidal.cu's test list) plus tile-boundary,
odd-size and misalignment edges.  Every output buffer starts as NaN, so an
element the kernels fail to write fails the check.
"""
import numpy as np
import pytest

import helpers as H
import oracle

pytestmark = pytest.mark.gpu


def _f32_call(fn, Q, K, V):
    import hip_rt
    q, k, v = H.upload(Q), H.upload(K), H.upload(V)
    out = H.empty(Q.shape)
    fn(q, k, v, out)
    hip_rt.synchronize()
    return out.numpy()


@pytest.mark.parametrize("name", ["tiny", "small", "hdim512"])
def test_golden_fixtures(am, dev, name):
    """BASELINE config 1 is the 'tiny' golden set exactly."""
    fx = H.load_fixture(name)
    print(f"[case] golden {name} shape={fx['Q'].shape}", flush=True)
    got = _f32_call(am.attention_forward_optimized, fx["Q"], fx["K"], fx["V"])
    n, mabs, _ = H.check_f32(got, fx["output"])
    assert n == 0, f"{n} mismatches vs PyTorch golden, max abs {mabs}"
    ref = oracle.attention(fx["Q"], fx["K"], fx["V"], nthreads=8)
    n, mabs, _ = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches vs oracle, max abs {mabs}"


SDPA_SHAPES = [  # (B, H, Lq, Lk, D)
    (1, 1, 4, 4, 8), (1, 2, 8, 8, 16), (2, 4, 32, 32, 32), (2, 8, 64, 64, 64),
    (1, 2, 16, 32, 32), (1, 4, 16, 16, 64), (2, 8, 64, 64, 128),
    (1, 4, 64, 64, 512), (1, 4, 64, 64, 2048), (1, 2, 32, 32, 4096), (1, 1, 16, 16, 8192),
    (1, 4, 64, 64, 4096), (1, 4, 64, 64, 8192),
    # tile edges and odd sizes
    (1, 1, 1, 1, 8), (1, 2, 65, 63, 96), (1, 1, 3, 129, 36), (2, 3, 17, 200, 7), (1, 1, 130, 5, 33),
]


@pytest.mark.parametrize("shape", SDPA_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_sdpa_f32(am, dev, shape):
    B, Hh, Lq, Lk, D = shape
    print(f"[case] sdpa f32 {shape}", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=100 + sum(shape))
    got = _f32_call(am.attention_forward_optimized, Q, K, V)
    ref = oracle.attention(Q, K, V, nthreads=8)
    n, mabs, mrel = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"
    got2 = _f32_call(am.attention_forward, Q, K, V)
    assert np.array_equal(got, got2)


_WIDE_SHAPES = [(1, 4, 64, 64, 512), (1, 4, 64, 64, 2048), (1, 4, 64, 64, 8192),
                (1, 4, 32, 128, 2048)]


@pytest.mark.parametrize("sigma", [1.5, 2.0, 3.0])
@pytest.mark.parametrize("shape", _WIDE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_sdpa_f32_wider_logits(am, dev, shape, sigma):
    """Inputs of sigma 1.5, 2 and 3 (logits up to about +-10, +-18 and +-40)
    on the default path (the single-launch kernel at these shapes): its fp32
    products come from hi + lo fp16 parts (22 significant bits each, exact
    products), so the 1e-4 bar holds whatever the logits' size.  At sigma 3
    and D >= 2048 the oracle's own sequential float32 sums miss the bar
    against the exact result (7, 233 and 8153 elements on these shapes, up to
    6.7e-4: test_oracle.py::test_oracle_drift_at_wide_logits), so there an
    element fails only if it misses the bar against the oracle and against
    the exact float64 result; everywhere else the oracle alone is the
    referee."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] sdpa f32 sigma {sigma} {shape}", flush=True)
    assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_FUSED_SMALL
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=7 + D, sigma=sigma)
    got = _f32_call(am.attention_forward_optimized, Q, K, V)
    ref = oracle.attention(Q, K, V, nthreads=16)
    if D >= 2048 and sigma == 3.0:
        n, mabs, mtruth = H.check_f32_or_truth(got, ref, H.sdpa64(Q, K, V))
        assert n == 0, f"{n} mismatches, max abs {mabs} (oracle), {mtruth} (exact)"
    else:
        n, mabs, _ = H.check_f32(got, ref)
        assert n == 0, f"{n} mismatches, max abs {mabs}"


@pytest.mark.parametrize("shape", _WIDE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_sdpa_f32_split_d_wide_logits(am, dev, tuner, shape):
    """The split-D pipeline (fp32 MFMA products; forced here with
    atn_tuning.no_fused) at sigma 3, against the oracle with the exact
    float64 result as second referee (the oracle's drift at D = 8192)."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] sdpa f32 split-D sigma 3 {shape}", flush=True)
    tuner.set(no_fused=True)
    assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_SPLIT_D
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=7 + D, sigma=3.0)
    got = _f32_call(am.attention_forward_optimized, Q, K, V)
    ref = oracle.attention(Q, K, V, nthreads=16)
    n, mabs, mtruth = H.check_f32_or_truth(got, ref, H.sdpa64(Q, K, V))
    assert n == 0, f"{n} mismatches, max abs {mabs} (oracle), {mtruth} (exact)"


@pytest.mark.parametrize("exps", [(17, -17, 0), (-17, 17, 0), (0, 0, 19), (17, -17, 21),
                                  (-9, -9, -9)],
                         ids=["q-big", "k-big", "v-big", "all-big", "all-small"])
@pytest.mark.parametrize("shape", [(1, 4, 64, 64, 2048), (1, 3, 40, 72, 1024),
                                   (1, 2, 16, 128, 8192)], ids=lambda s: "x".join(map(str, s)))
def test_sdpa_f32_outside_fp16_range(am, dev, shape, exps):
    """The single-launch kernel's fp16 split needs |x| < 65504: a workgroup
    whose Q/K or V slice holds a larger value stages that slice again scaled
    by a power of two and multiplies the results back.  Head 1 of each call
    has Q, K and V multiplied by 2^eq, 2^ek and 2^ev (the other heads stay
    N(0,1), so both kinds of workgroup run in one call).  Scaling by powers
    of two is exact, so attention(2^eq Q, 2^ek K, 2^ev V) = 2^ev attention(
    2^eq Q, 2^ek K, V) in the oracle's float32 arithmetic too: the output of
    head 1 is compared, in units of 2^ev, with the oracle on the unscaled V
    (an absolute 1e-4 bar on outputs of magnitude 2^19 would be finer than
    float32 itself).  Also small inputs (2^-9: many fp16 subnormal lo
    parts)."""
    B, Hh, Lq, Lk, D = shape
    eq, ek, ev = exps
    print(f"[case] sdpa f32 outside the fp16 range 2^{exps} {shape}", flush=True)
    assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_FUSED_SMALL
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=31 + D)
    Q[:, 1] *= np.float32(2.0 ** eq)
    K[:, 1] *= np.float32(2.0 ** ek)
    Vs = V.copy()
    Vs[:, 1] *= np.float32(2.0 ** ev)
    got = _f32_call(am.attention_forward_optimized, Q, K, Vs)
    assert np.isfinite(got).all()
    got[:, 1] *= np.float32(2.0 ** -ev)
    ref = oracle.attention(Q, K, V, nthreads=16)
    n, mabs, mrel = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"


def test_sdpa_f32_nonfinite_inputs_propagate(am, dev):
    """An infinite query element makes its own output row non-finite, as in
    the reference (exp(inf - inf) in its softmax); the other rows of that
    row group, whose slice is then staged scaled by its largest finite
    magnitude, and the other heads keep the bar.  A NaN value element makes
    its output column NaN, as in the reference."""
    B, Hh, Lq, Lk, D = 1, 4, 64, 64, 2048
    print("[case] sdpa f32 non-finite inputs", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=77)
    Q[0, 2, 5, 100] = np.inf
    V[0, 1, 9, 33] = np.nan
    got = _f32_call(am.attention_forward_optimized, Q, K, V)
    ref = oracle.attention(Q, K, V, nthreads=16)
    assert not np.isfinite(ref[0, 2, 5]).any() and not np.isfinite(got[0, 2, 5]).any()
    assert np.isnan(ref[0, 1, :, 33]).all() and np.isnan(got[0, 1, :, 33]).all()
    keep = np.ones((Hh, Lq, D), dtype=bool)
    keep[2, 5, :] = False
    keep[1, :, 33] = False
    n, mabs, _ = H.check_f32(got[0][keep], ref[0][keep])
    assert n == 0, mabs


@pytest.mark.parametrize("shape", [(1, 1, 70, 1, 64), (1, 3, 65, 255, 40), (1, 8, 70, 1025, 64),
                                   (1, 4, 65, 2048, 64), (1, 2, 100, 2049, 32)],
                         ids=lambda s: "x".join(map(str, s)))
def test_sdpa_f32_split_d_softmax_rows(am, dev, tuner, shape):
    """fp32 rows on the split-D pipeline (forced: these head dims take the
    flash kernel by default) without D-chunk partials: one key, the edges of
    the one-wave-per-row softmax's register blocks (256, 1024, 2048 keys) and
    the first row length past it (2049 keys, the workgroup-per-row
    softmax)."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] sdpa f32 split-D softmax rows {shape}", flush=True)
    tuner.set(no_flash=True)
    assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_SPLIT_D
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=40 + Lk)
    got = _f32_call(am.attention_forward_optimized, Q, K, V)
    ref = oracle.attention(Q, K, V, nthreads=16)
    n, mabs, _ = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}"


def test_sdpa_llama_shape(am, dev):
    B, Hh, L, D = 4, 32, 512, 128  # final/attention.cu:522
    print("[case] sdpa f32 llama (4,32,512,128)", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, L, D), (B, Hh, L, D), seed=7)
    got = _f32_call(am.attention_forward_optimized, Q, K, V)
    ref = oracle.attention(Q, K, V, nthreads=16)
    n, mabs, _ = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}"


def test_sdpa_misaligned_views(am, dev):
    """Pointers offset by one element take the scalar-load path."""
    import hip_rt
    B, Hh, L, D = 1, 2, 40, 64
    print("[case] sdpa f32 misaligned", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, L, D), (B, Hh, L, D), seed=3)
    views = []
    for x in (Q, K, V, None):
        base = hip_rt.DeviceArray((Q.size + 1,), "f32")
        v = hip_rt.DeviceArray.view(base, 1, (B, Hh, L, D))
        if x is not None:
            v.upload(x)
        views.append(v)
    am.attention_forward_optimized(*views)
    hip_rt.synchronize()
    ref = oracle.attention(Q, K, V)
    nf, mabs, _ = H.check_f32(views[3].numpy(), ref)
    assert nf == 0, mabs


BF16_SHAPES = [(1, 4, 32, 128, 8192), (1, 2, 8, 8, 16), (2, 4, 64, 64, 512), (1, 3, 33, 70, 260)]


@pytest.mark.parametrize("shape", BF16_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_sdpa_bf16(am, dev, shape):
    """BASELINE config 3 is the first shape."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] sdpa bf16 {shape}", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 11, "bf16")
    out = H.empty(Q.shape, "bf16")
    am.attention_forward_bf16(q, k, v, out)
    hip_rt.synchronize()
    ref = oracle.attention(Q, K, V, nthreads=16)
    n, nrel, mabs = H.check_bf16(out.numpy(), ref)
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("shape", [(1, 4, 32, 128, 8192), (2, 4, 64, 64, 512), (1, 2, 16, 100, 2048)],
                         ids=lambda s: "x".join(map(str, s)))
def test_sdpa_bf16_wide_logits(am, dev, shape):
    """bf16 inputs of sigma 3 (logits to about +-40) on the single-launch
    kernel: bf16 operands are exact MFMA inputs and P goes in as hi + lo
    parts, so the bf16 bar holds far outside the unit-scale inputs."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] sdpa bf16 sigma 3 {shape}", flush=True)
    assert am.path(1, B, Hh, Lq, Lk, D) == am.ATN_PATH_FUSED_SMALL
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 13, "bf16", 3.0)
    out = H.empty(Q.shape, "bf16")
    am.attention_forward_bf16(q, k, v, out)
    hip_rt.synchronize()
    ref = oracle.attention(Q, K, V, nthreads=16)
    n, nrel, mabs = H.check_bf16(out.numpy(), ref)
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


# ---------------------------------------------------------------- RoPE
ROPE_SHAPES = [(1, 1, 4, 8), (1, 2, 8, 16), (2, 4, 32, 32), (1, 4, 16, 64), (1, 4, 64, 128),
               (1, 4, 64, 512), (1, 4, 64, 2048)]  # final/rope.cu:1911-1923


@pytest.mark.parametrize("shape", ROPE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_rope_fused_cache(am, dev, shape):
    B, Hh, L, D = shape
    print(f"[case] rope fused cache {shape}", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, L, D), (B, Hh, L, D), seed=21 + D)
    c, s = oracle.rope_cache(L, D)
    tc, ts = H.upload(c), H.upload(s)
    got = _f32_call(lambda q, k, v, o: am.attention_forward_rope_fused(q, k, v, o, tc, ts), Q, K, V)
    ref = oracle.attention_rope(Q, K, V, c, s, nthreads=8)
    n, mabs, _ = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}"


@pytest.mark.parametrize("shape,rot", [((1, 4, 64, 64, 128), 64), ((1, 4, 64, 64, 512), 128),
                                       ((1, 4, 64, 64, 2048), 128), ((1, 2, 24, 40, 96), 96),
                                       ((1, 2, 24, 40, 98), 50)],
                         ids=lambda s: str(s))
def test_rope_v7_hybrid_and_separate(am, dev, shape, rot):
    """K pre-rotated by the pre-pass (bit-exact vs the oracle), Q rotated in
    the attention call; and the separate pipeline (final/rope.cu:1800-1906)."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] rope v7/separate {shape} rot={rot}", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=31 + D)
    c, s = oracle.rope_cache(max(Lq, Lk), rot)
    tc, ts = H.upload(c), H.upload(s)
    q, k, v = H.upload(Q), H.upload(K), H.upload(V)
    k_rot = H.empty(K.shape)
    am.rope_forward(k, k_rot, tc, ts, rot, Lk)
    hip_rt.synchronize()
    k_rot_ref = oracle.apply_rope(K, c, s, rotary_dim=rot)
    assert np.array_equal(k_rot.numpy(), k_rot_ref), "pre-pass not bit-exact"
    out = H.empty(Q.shape)
    am.attention_forward_rope_fused_v7_hybrid(q, k_rot, v, out, rot)
    hip_rt.synchronize()
    ref = oracle.attention_rope(Q, k_rot_ref, V, c, s, rotary_dim=rot, rotate_k=False, nthreads=8)
    n, mabs, _ = H.check_f32(out.numpy(), ref)
    assert n == 0, f"v7: {n} mismatches, max abs {mabs}"
    q_rope, k_rope, out2 = H.empty(Q.shape), H.empty(K.shape), H.empty(Q.shape)
    am.attention_forward_separate_rope(q, k, v, q_rope, k_rope, out2, tc, ts, rot)
    hip_rt.synchronize()
    ref2 = oracle.attention_rope(Q, K, V, c, s, rotary_dim=rot, nthreads=8)
    n, mabs, _ = H.check_f32(out2.numpy(), ref2)
    assert n == 0, f"separate: {n} mismatches, max abs {mabs}"
    assert np.array_equal(q_rope.numpy(), oracle.apply_rope(Q, c, s, rotary_dim=rot))


@pytest.mark.parametrize("shape", [(1, 2, 8, 8, 16), (1, 4, 64, 64, 512), (2, 2, 40, 72, 96),
                                   (1, 4, 64, 64, 2048)], ids=str)
def test_rope_bf16_full_fusion_and_v7(am, dev, shape):
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] rope bf16 {shape}", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 41, "bf16")
    out = H.empty(Q.shape, "bf16")
    am.attention_forward_rope_fused_bf16(q, k, v, out)
    hip_rt.synchronize()
    c, s = oracle.rope_cache(max(Lq, Lk), D)
    ref = oracle.attention_rope(Q, K, V, c, s, nthreads=16)
    n, nrel, mabs = H.check_bf16(out.numpy(), ref)
    assert n == 0, f"full fusion: normwise rel {nrel}, max abs {mabs}"
    # v7 form: K pre-rotated by the caller and stored in bf16
    rot = D // 2 if (D // 2) % 2 == 0 else D
    cr, sr = oracle.rope_cache(max(Lq, Lk), rot)
    k_rot = H.upload(oracle.apply_rope(K, cr, sr, rotary_dim=rot), "bf16")
    out.fill_nan()
    am.attention_forward_rope_bf16(q, k_rot, v, out, rot)
    hip_rt.synchronize()
    ref = oracle.attention_rope(Q, k_rot.numpy(), V, cr, sr, rotary_dim=rot, rotate_k=False,
                                nthreads=16)
    n, nrel, mabs = H.check_bf16(out.numpy(), ref)
    assert n == 0, f"v7: normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("shape", [(1, 2, 16, 16, 64), (1, 2, 64, 96, 512), (2, 2, 33, 65, 256)],
                         ids=str)
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_rope_half_ex(am, dev, shape, dtype):
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] rope half ex {shape} {dtype}", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 51, dtype)
    out = H.empty(Q.shape, dtype)
    am.attention_ex(q, k, v, out, pe=am.make_pe("rope", pairing="half"))
    hip_rt.synchronize()
    c, s = oracle.rope_cache(max(Lq, Lk), D)
    ref = oracle.attention_rope(Q, K, V, c, s, pairing="half", nthreads=16)
    if dtype == "f32":
        n, mabs, _ = H.check_f32(out.numpy(), ref)
        assert n == 0, f"{n} mismatches, max abs {mabs}"
    else:
        n, nrel, mabs = H.check_bf16(out.numpy(), ref)
        assert n == 0, f"normwise rel {nrel}"


# ---------------------------------------------------------------- sinusoidal
SIN_SHAPES = [(1, 1, 4, 4, 8), (1, 2, 8, 8, 16), (2, 4, 32, 32, 32), (1, 4, 64, 64, 512),
              (1, 4, 64, 64, 2048), (1, 2, 32, 32, 4096), (1, 2, 20, 50, 100), (1, 1, 9, 13, 7)]


@pytest.mark.parametrize("shape", SIN_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_sinusoidal_f32(am, dev, shape):
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] sinusoidal f32 {shape}", flush=True)
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=61 + D)
    st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
    ref = oracle.attention_sinusoidal(Q, K, V, st, ct, nthreads=8)
    # exact SDPA of the float32-encoded inputs (the oracle's own float32 sums
    # drift by ~1e-4 here at D = 4096, where scores reach ~30)
    truth = H.sdpa64(oracle.add_sinusoidal(Q, st, ct), oracle.add_sinusoidal(K, st, ct), V)
    got = _f32_call(am.attention_forward_sinusoidal_fused, Q, K, V)
    n, mabs, mtruth = H.check_f32_or_truth(got, ref, truth)
    assert n == 0, f"fused: {n} mismatches, max abs {mabs} (vs exact {mtruth})"
    tst, tct = H.upload(st), H.upload(ct)
    q, k, v = H.upload(Q), H.upload(K), H.upload(V)
    k_emb, q_emb, out = H.empty(K.shape), H.empty(Q.shape), H.empty(Q.shape)
    am.attention_forward_sinusoidal_hybrid(q, k, v, tst, tct, k_emb, out)
    hip_rt.synchronize()
    n, mabs, mtruth = H.check_f32_or_truth(out.numpy(), ref, truth)
    assert n == 0, f"hybrid: {n} mismatches, max abs {mabs} (vs exact {mtruth})"
    assert np.array_equal(k_emb.numpy(), oracle.add_sinusoidal(K, st, ct))
    out.fill_nan()
    am.attention_forward_sinusoidal_separate(q, k, v, tst, tct, q_emb, k_emb, out)
    hip_rt.synchronize()
    n, mabs, mtruth = H.check_f32_or_truth(out.numpy(), ref, truth)
    assert n == 0, f"separate: {n} mismatches, max abs {mabs} (vs exact {mtruth})"
    assert np.array_equal(q_emb.numpy(), oracle.add_sinusoidal(Q, st, ct))
    pe_out = H.empty(Q.shape)
    am.apply_sinusoidal_embeddings(q, tst, tct, pe_out, Lq)
    hip_rt.synchronize()
    assert np.array_equal(pe_out.numpy(), oracle.add_sinusoidal(Q, st, ct))


@pytest.mark.parametrize("shape", [(1, 2, 8, 8, 16), (1, 4, 64, 64, 512), (1, 2, 48, 200, 1024)],
                         ids=str)
def test_sinusoidal_bf16(am, dev, shape):
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] sinusoidal bf16 {shape}", flush=True)
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 71, "bf16", sigma=0.5)
    out = H.empty(Q.shape, "bf16")
    am.attention_forward_sinusoidal_bf16(q, k, v, out)
    hip_rt.synchronize()
    st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
    ref = oracle.attention_sinusoidal(Q, K, V, st, ct, nthreads=16)
    n, nrel, mabs = H.check_bf16(out.numpy(), ref)
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("tile", [64, 128])
@pytest.mark.parametrize("shape,pe", [((1, 2, 200, 300, 520), None), ((1, 3, 130, 129, 1024), None),
                                      ((2, 2, 256, 256, 384), None), ((1, 2, 129, 257, 520), "rope"),
                                      ((1, 2, 140, 200, 640), "sinusoidal")],
                         ids=lambda v: "x".join(map(str, v)) if isinstance(v, tuple) else str(v))
def test_split_d_tiles(am, dev, tuner, tile, shape, pe):
    """The split-D pipeline's fp32 contractions with each output tile forced
    (64 x 64, or 128 x 128 wherever both of a tile's sides reach 128):
    ragged edges of either tile, D-chunks of whole and partial stages, and
    the encodings applied at load."""
    import hip_rt
    B, Hh, Lq, Lk, D = shape
    print(f"[case] split-D f32 tile {tile} {shape} {pe}", flush=True)
    tuner.set(splitd_tile=tile)
    desc = None if pe is None else am.make_pe(pe)
    assert am.path(0, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_SPLIT_D
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=29 + D + tile,
                           sigma=0.5 if pe == "sinusoidal" else 1.0)
    (q, k, v) = (H.upload(x) for x in (Q, K, V))
    out = H.empty(Q.shape)
    am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    got = out.numpy()
    L = max(Lq, Lk)
    if pe == "sinusoidal":
        st_, ct_ = oracle.sinusoidal_table(L, D)
        ref = oracle.attention_sinusoidal(Q, K, V, st_, ct_, nthreads=16)
    elif pe == "rope":
        c_, s_ = oracle.rope_cache(L, D)
        ref = oracle.attention_rope(Q, K, V, c_, s_, rotary_dim=D, nthreads=16)
    else:
        ref = oracle.attention(Q, K, V, nthreads=16)
    n, mabs, _ = H.check_f32(got, ref)
    assert n == 0, f"{n} mismatches, max abs {mabs}"


@pytest.mark.parametrize("tile", [64, 128])
@pytest.mark.parametrize("exps", [(17, -17, 0), (0, 0, 19), (17, -17, 21), (-12, -12, -12)],
                         ids=["qk-big", "v-big", "all-big", "all-small"])
@pytest.mark.parametrize("shape", [(1, 3, 100, 130, 520), (1, 3, 70, 300, 1024),
                                   (1, 2, 200, 300, 520)],
                         ids=lambda s: "x".join(map(str, s)))
def test_split_d_outside_fp16_range(am, dev, tuner, shape, exps, tile):
    """fp32 beyond the single-launch window with head_d > 256 runs the
    split-D pipeline, whose contractions use the fp16 split too: a stage
    with a value outside fp16's range is staged again with power-of-two
    scales (in both output tile sizes).  Head 1 is scaled by 2^eq, 2^ek,
    2^ev (exact); its output is compared in units of 2^ev with the oracle on
    the unscaled V."""
    B, Hh, Lq, Lk, D = shape
    eq, ek, ev = exps
    print(f"[case] split-D f32 tile {tile} scaled 2^{exps} {shape}", flush=True)
    tuner.set(splitd_tile=tile)
    assert am.path(0, B, Hh, Lq, Lk, D) == am.ATN_PATH_SPLIT_D
    Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=37 + D)
    Q[:, 1] *= np.float32(2.0 ** eq)
    K[:, 1] *= np.float32(2.0 ** ek)
    Vs = V.copy()
    Vs[:, 1] *= np.float32(2.0 ** ev)
    got = _f32_call(am.attention_forward_optimized, Q, K, Vs)
    assert np.isfinite(got).all()
    got[:, 1] *= np.float32(2.0 ** -ev)
    n, mabs, mrel = H.check_f32(got, oracle.attention(Q, K, V, nthreads=16))
    assert n == 0, f"{n} mismatches, max abs {mabs}, max rel {mrel}"
