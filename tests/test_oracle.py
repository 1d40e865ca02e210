"""Pins the CPU oracle (oracle/attention_oracle.c) -- runs on the CPU.

The oracle restates the reference's CPU attention paths; these tests check
it against what fixes its results independently of its own code:
  * the reference's golden vectors (PyTorch SDPA outputs shipped in
    pytorch_reference_data/, committed here as small fixtures; the full sets
    are re-read when /root/reference is present);
  * closed forms and invariants of SDPA (equal V rows, Q = 0, Lk = 1,
    constant inputs, joint K/V row permutation, float64 brute force at 64-key
    tile boundaries);
  * for RoPE and the sinusoidal encoding: the float64 mathematics of the
    angle tables, pos-0 identities, norm preservation, the relative-position
    property, and the rotate-half <-> interleaved permutation identity;
  * bf16 rounding against torch's own fp32 -> bfloat16 conversion.
Each group also plants a known mistake in the oracle (oracle.set_mutation)
and shows that the same check then fails.
"""
import hashlib
import os

import numpy as np
import pytest

import helpers as H
import oracle


@pytest.fixture(autouse=True)
def _no_mutation():
    oracle.set_mutation(0)
    yield
    oracle.set_mutation(0)


def sdpa64(Q, K, V):
    """Float64 SDPA brute force (softmax(QK^T/sqrt(D)) V), independent of the oracle."""
    Q, K, V = (np.asarray(x, dtype=np.float64) for x in (Q, K, V))
    s = Q @ np.swapaxes(K, -1, -2) / np.sqrt(Q.shape[-1])
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return p @ V


# ------------------------------------------------------------------ golden vectors
@pytest.mark.parametrize("name", ["tiny", "small", "hdim512"])
def test_attention_vs_committed_golden(name):
    fx = H.load_fixture(name)
    got = oracle.attention(fx["Q"], fx["K"], fx["V"])
    n, mabs, _ = H.check_f32(got, fx["output"])
    assert n == 0, f"{n} elements outside abs/rel 1e-4, max abs {mabs}"
    assert mabs < 2e-6


def test_tiny_golden_is_baseline_config_1():
    m = H.manifest()["sets"]["tiny"]
    assert m["shape"] == [1, 1, 4, 8] and m["seed"] == 42
    raw = open(os.path.join(H.GOLDEN, "tiny_output.bin"), "rb").read()
    assert hashlib.sha256(raw).hexdigest() == m["sha256"]["output"]


REF_SETS = ["tiny", "small", "hdim512", "hdim2048", "hdim4096", "hdim8192"]


@pytest.mark.skipif(not os.path.isdir(H.REF_DATA), reason="reference data not mounted")
@pytest.mark.parametrize("name", REF_SETS)
def test_attention_vs_full_reference_golden(name):
    """All six reference golden sets (hdim2048 is BASELINE config 2 exactly)."""
    m = H.manifest()["sets"][name]
    arrs = {}
    for t in ("Q", "K", "V", "output"):
        raw = open(os.path.join(H.REF_DATA, f"pytorch_ref_{name}_{t}.bin"), "rb").read()
        assert hashlib.sha256(raw).hexdigest() == m["sha256"][t]
        arrs[t] = np.frombuffer(raw, dtype="<f4").reshape(m["shape"])
    got = oracle.attention(arrs["Q"], arrs["K"], arrs["V"], nthreads=8)
    n, mabs, _ = H.check_f32(got, arrs["output"])
    # float32 sums over D = 8192 terms drift a few 1e-6 from PyTorch's result
    assert n == 0 and mabs < 1e-5, (n, mabs)


def test_planted_scale_mistake_fails_golden():
    fx = H.load_fixture("small")
    oracle.set_mutation(1)  # drops the 1/sqrt(D) scale
    got = oracle.attention(fx["Q"], fx["K"], fx["V"])
    n, _, _ = H.check_f32(got, fx["output"])
    assert n > 0


# ------------------------------------------------------------------ SDPA closed forms
def test_equal_v_rows_give_that_row():
    rng = np.random.default_rng(0)
    Q = rng.standard_normal((1, 2, 5, 32), dtype=np.float32)
    K = rng.standard_normal((1, 2, 9, 32), dtype=np.float32)
    row = rng.standard_normal(32, dtype=np.float32)
    V = np.broadcast_to(row, (1, 2, 9, 32)).copy()
    got = oracle.attention(Q, K, V)
    assert np.allclose(got, np.broadcast_to(row, got.shape), rtol=1e-5, atol=1e-6)


def test_zero_q_gives_mean_of_v():
    rng = np.random.default_rng(1)
    Q = np.zeros((1, 1, 3, 16), dtype=np.float32)
    K = rng.standard_normal((1, 1, 7, 16), dtype=np.float32)
    V = rng.standard_normal((1, 1, 7, 16), dtype=np.float32)
    got = oracle.attention(Q, K, V)
    assert np.allclose(got[0, 0], V[0, 0].astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)


def test_single_key_gives_v0():
    rng = np.random.default_rng(2)
    Q = rng.standard_normal((2, 2, 4, 24), dtype=np.float32)
    K = rng.standard_normal((2, 2, 1, 24), dtype=np.float32)
    V = rng.standard_normal((2, 2, 1, 24), dtype=np.float32)
    got = oracle.attention(Q, K, V)
    assert np.array_equal(got, np.broadcast_to(V, got.shape))


def test_constant_inputs_known_answer():
    """Q = K = V = 0.1 -> every output is 0.1 (final/rope.cu:1658-1662)."""
    Q = np.full((1, 2, 8, 64), 0.1, dtype=np.float32)
    got = oracle.attention(Q, Q, Q)
    assert np.allclose(got, 0.1, rtol=1e-6, atol=0)
    c, s = oracle.rope_cache(8, 64)
    got = oracle.attention_rope(Q, Q, Q, c, s)
    assert np.allclose(got, 0.1, rtol=1e-6, atol=0)


def test_joint_kv_permutation_invariance():
    rng = np.random.default_rng(3)
    Q = rng.standard_normal((1, 1, 6, 40), dtype=np.float32)
    K = rng.standard_normal((1, 1, 33, 40), dtype=np.float32)
    V = rng.standard_normal((1, 1, 33, 40), dtype=np.float32)
    perm = rng.permutation(33)
    a = oracle.attention(Q, K, V)
    b = oracle.attention(Q, K[:, :, perm], V[:, :, perm])
    assert np.allclose(a, b, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("Lk", [1, 63, 64, 65, 127, 128, 200])
def test_fp64_brute_force_tile_edges(Lk):
    rng = np.random.default_rng(10 + Lk)
    Q = rng.standard_normal((1, 2, 5, 96), dtype=np.float32)
    K = rng.standard_normal((1, 2, Lk, 96), dtype=np.float32)
    V = rng.standard_normal((1, 2, Lk, 96), dtype=np.float32)
    n, mabs, _ = H.check_f32(oracle.attention(Q, K, V), sdpa64(Q, K, V))
    assert n == 0, mabs


def test_large_score_shift_invariance():
    """Scores of magnitude ~1e3 must not overflow the exponentials."""
    rng = np.random.default_rng(4)
    Q = rng.standard_normal((1, 1, 4, 64), dtype=np.float32) * 40
    K = rng.standard_normal((1, 1, 9, 64), dtype=np.float32) * 40
    V = rng.standard_normal((1, 1, 9, 64), dtype=np.float32)
    got = oracle.attention(Q, K, V)
    assert np.all(np.isfinite(got))
    assert np.allclose(got, sdpa64(Q, K, V), atol=2e-5)


def test_row_ranges_and_threads_match_serial():
    rng = np.random.default_rng(5)
    Q = rng.standard_normal((2, 3, 9, 32), dtype=np.float32)
    K = rng.standard_normal((2, 3, 11, 32), dtype=np.float32)
    V = rng.standard_normal((2, 3, 11, 32), dtype=np.float32)
    full = oracle.attention(Q, K, V)
    par = oracle.attention(Q, K, V, nthreads=4)
    assert np.array_equal(full, par)
    part = oracle.attention(Q, K, V, rows=(5, 20))
    flat, pflat = full.reshape(-1, 32), part.reshape(-1, 32)
    assert np.array_equal(flat[5:20], pflat[5:20])
    assert np.all(np.isnan(pflat[:5])) and np.all(np.isnan(pflat[20:]))


def test_check_results_semantics():
    """final/attention.cu:296-331: fail iff abs > atol AND rel > rtol."""
    ref = np.array([1.0, 1e-6, 100.0], dtype=np.float32)
    got = np.array([1.0 + 5e-4, 1e-6 + 5e-4, 100.5], dtype=np.float32)
    n, _, _ = oracle.check_results(got, ref, 1e-3, 1e-2)
    assert n == 0
    got2 = np.array([1.0 + 2e-2, 0.0, 100.0], dtype=np.float32)
    n, _, _ = oracle.check_results(got2, ref, 1e-3, 1e-2)
    assert n == 1


# ------------------------------------------------------------------ RoPE
def _angles64(npos, r, base=10000.0):
    i = np.arange(r // 2, dtype=np.float64)
    freq = 1.0 / base ** (2.0 * i / r)
    return np.arange(npos, dtype=np.float64)[:, None] * freq[None, :]


@pytest.mark.parametrize("npos,r", [(64, 8), (1024, 128), (2048, 64), (300, 4096)])
def test_rope_cache_matches_float64_math(npos, r):
    """cache[pos][2i] = cache[pos][2i+1] = cos/sin(pos / base^(2i/r))
    (final/rope.cu:20-40) within the float32 rounding of the angle."""
    c, s = oracle.rope_cache(npos, r)
    th = _angles64(npos, r)
    tol = 1e-6 + 2.5e-7 * np.arange(npos)[:, None]
    for tab, fn in ((c, np.cos), (s, np.sin)):
        assert np.array_equal(tab[:, 0::2], tab[:, 1::2])
        assert np.all(np.abs(tab[:, 0::2] - fn(th)) <= tol)


@pytest.mark.parametrize("r,base", [(8, 10000.0), (128, 10000.0), (4096, 10000.0), (64, 500.0)])
def test_rope_freqs_match_float64_and_cache(r, base):
    """oracle_rope_freqs (final/rope.cu:96-98, :132-134): freq_i =
    1/base^(2i/r) within float32 rounding of powf and the division, and at
    position 1 the (separately pinned) cache holds exactly cos/sin of these
    frequencies, since theta = 1 * freq_i."""
    f = oracle.rope_freqs(r, base)
    exact = 1.0 / base ** (2.0 * np.arange(r // 2, dtype=np.float64) / r)
    assert f.shape == (r // 2,) and f[0] == 1.0
    assert np.all(np.abs(f / exact - 1.0) <= 4e-7)
    c, s = oracle.rope_cache(2, r, base)
    f64 = f.astype(np.float64)
    assert np.all(np.abs(c[1, 0::2] - np.cos(f64)) <= 1.2e-7)
    assert np.all(np.abs(s[1, 0::2] - np.sin(f64)) <= 1.2e-7)
    # a frequency table off by one pair index (the exponent of pair i + 1)
    # fails the float64 check
    shifted = 1.0 / base ** (2.0 * (np.arange(r // 2, dtype=np.float64) + 1) / r)
    assert not np.all(np.abs(f / shifted - 1.0) <= 4e-7)


@pytest.mark.parametrize("D", [8, 7, 1024, 8192])
def test_sinusoidal_freqs_match_float64_and_table(D):
    """oracle_sinusoidal_freqs (final/sinusoidal.cu:112-114): freq[d] =
    1/1e4^(2*(d//2)/D), equal on each (even, odd) pair, and at position 1 the
    (separately pinned) table holds sin (even d) / cos (odd d) of them."""
    f = oracle.sinusoidal_freqs(D)
    d = np.arange(D)
    exact = 1.0 / 10000.0 ** (2.0 * (d // 2) / D)
    assert np.all(np.abs(f / exact - 1.0) <= 4e-7)
    assert np.array_equal(f[0:D - 1:2], f[1:D:2])
    st, ct = oracle.sinusoidal_table(2, D)
    f64 = f.astype(np.float64)
    assert np.all(np.abs(st[1] - np.sin(f64)) <= 1.2e-7)
    assert np.all(np.abs(ct[1] - np.cos(f64)) <= 1.2e-7)
    # using d instead of d // 2 in the exponent fails the float64 check
    wrong = 1.0 / 10000.0 ** (2.0 * d / D)
    assert D < 3 or not np.all(np.abs(f / wrong - 1.0) <= 4e-7)


def test_rope_planted_swap_fails_table_check():
    oracle.set_mutation(2)
    c, _ = oracle.rope_cache(16, 8)
    assert not np.allclose(c[:, 0::2], np.cos(_angles64(16, 8)), atol=1e-3)


def test_rope_pos0_identity_and_norms():
    rng = np.random.default_rng(6)
    X = rng.standard_normal((1, 1, 50, 64), dtype=np.float32)
    c, s = oracle.rope_cache(50, 64)
    for pairing in ("interleaved", "half"):
        Y = oracle.apply_rope(X, c, s, pairing=pairing)
        assert np.array_equal(Y[..., 0, :], X[..., 0, :])
        n_in = np.linalg.norm(X.astype(np.float64), axis=-1)
        n_out = np.linalg.norm(Y.astype(np.float64), axis=-1)
        assert np.allclose(n_in, n_out, rtol=1e-5)
    # per-pair norms for the interleaved form
    Y = oracle.apply_rope(X, c, s)
    pin = np.hypot(X[..., 0::2].astype(np.float64), X[..., 1::2])
    pout = np.hypot(Y[..., 0::2].astype(np.float64), Y[..., 1::2])
    assert np.allclose(pin, pout, rtol=1e-5, atol=1e-6)


def test_rope_relative_position_property():
    """<R_m q, R_n k> depends only on m - n (both pairings)."""
    rng = np.random.default_rng(7)
    D = 32
    q = rng.standard_normal(D, dtype=np.float32)
    k = rng.standard_normal(D, dtype=np.float32)
    c, s = oracle.rope_cache(64, D)
    X = np.broadcast_to(q, (64, D)).copy()
    Y = np.broadcast_to(k, (64, D)).copy()
    for pairing in ("interleaved", "half"):
        RX = oracle.apply_rope(X, c, s, pairing=pairing).astype(np.float64)
        RY = oracle.apply_rope(Y, c, s, pairing=pairing).astype(np.float64)
        for delta in (0, 3, 17):
            dots = [RX[m] @ RY[m - delta] for m in range(delta, 40)]
            assert np.ptp(dots) < 2e-3 * (1 + abs(np.mean(dots))), (pairing, delta)


def test_rope_transposed_rotation_fails_relative_position_check():
    """A planted transposed rotation (sin sign flipped on one side only is
    what a transposed operand produces) breaks the pairing consistency."""
    rng = np.random.default_rng(8)
    D = 16
    c, s = oracle.rope_cache(32, D)
    X = np.broadcast_to(rng.standard_normal(D, dtype=np.float32), (32, D)).copy()
    Y = np.broadcast_to(rng.standard_normal(D, dtype=np.float32), (32, D)).copy()
    RX = oracle.apply_rope(X, c, s).astype(np.float64)
    oracle.set_mutation(3)
    RY = oracle.apply_rope(Y, c, s).astype(np.float64)
    dots = [RX[m] @ RY[m - 2] for m in range(2, 30)]
    assert np.ptp(dots) > 1e-2


def test_rope_composition():
    """R(a) R(b) = R(a + b): rotating the rotated rows again by the pos-1
    table equals rotating by pos + 1 (within float32 rounding)."""
    rng = np.random.default_rng(9)
    D, L = 64, 40
    c, s = oracle.rope_cache(L + 1, D)
    X = rng.standard_normal((1, 1, L, D), dtype=np.float32)
    once = oracle.apply_rope(X, c, s, pos0=1)
    c1 = np.broadcast_to(c[1], (L + 1, D)).copy()
    s1 = np.broadcast_to(s[1], (L + 1, D)).copy()
    twice = oracle.apply_rope(oracle.apply_rope(X, c, s), c1, s1)
    assert np.allclose(once, twice, atol=5e-5)


@pytest.mark.parametrize("r", [8, 64, 96])
def test_rotate_half_permutation_identity(r):
    """rotate_half(x) = P^-1 interleaved(P x), (P x)[2i] = x[i],
    (P x)[2i+1] = x[i + r/2]; dims >= r pass through."""
    rng = np.random.default_rng(11 + r)
    D = r + 6
    X = rng.standard_normal((1, 1, 30, D), dtype=np.float32)
    c, s = oracle.rope_cache(30, r)
    perm = np.empty(r, dtype=np.int64)
    perm[0::2] = np.arange(r // 2)
    perm[1::2] = np.arange(r // 2) + r // 2
    PX = X.copy()
    PX[..., :r] = X[..., perm]
    inter = oracle.apply_rope(PX, c, s, rotary_dim=r)
    back = inter.copy()
    back[..., perm] = inter[..., :r]
    half = oracle.apply_rope(X, c, s, rotary_dim=r, pairing="half")
    assert np.array_equal(half, back)


def test_attention_rope_equals_attention_of_rotated():
    rng = np.random.default_rng(12)
    B, Hh, Lq, Lk, D = 1, 2, 20, 33, 48
    Q = rng.standard_normal((B, Hh, Lq, D), dtype=np.float32)
    K = rng.standard_normal((B, Hh, Lk, D), dtype=np.float32)
    V = rng.standard_normal((B, Hh, Lk, D), dtype=np.float32)
    c, s = oracle.rope_cache(max(Lq, Lk), D)
    for pairing in ("interleaved", "half"):
        a = oracle.attention_rope(Q, K, V, c, s, pairing=pairing)
        b = oracle.attention(oracle.apply_rope(Q, c, s, pairing=pairing),
                             oracle.apply_rope(K, c, s, pairing=pairing), V)
        assert np.array_equal(a, b)
        assert np.allclose(a, sdpa64(oracle.apply_rope(Q, c, s, pairing=pairing),
                                     oracle.apply_rope(K, c, s, pairing=pairing), V), atol=2e-6)
    oracle.set_mutation(4)  # keys start at position 1
    c2, s2 = oracle.rope_cache(max(Lq, Lk) + 1, D)
    oracle.set_mutation(0)
    ok = oracle.attention_rope(Q, K, V, c2, s2)
    oracle.set_mutation(4)
    bad = oracle.attention_rope(Q, K, V, c2, s2)
    assert not np.allclose(ok, bad, atol=1e-3)


def test_rope_partial_rotary_passthrough():
    rng = np.random.default_rng(13)
    X = rng.standard_normal((1, 1, 10, 40), dtype=np.float32)
    c, s = oracle.rope_cache(10, 16)
    Y = oracle.apply_rope(X, c, s, rotary_dim=16)
    assert np.array_equal(Y[..., 16:], X[..., 16:])
    assert not np.array_equal(Y[..., 1:, :16], X[..., 1:, :16])


# ------------------------------------------------------------------ sinusoidal
@pytest.mark.parametrize("npos,D", [(64, 8), (2048, 1024), (100, 7)])
def test_sinusoidal_table_matches_float64_math(npos, D):
    """table[pos][d] = sin/cos(pos / 1e4^(2*(d//2)/D)) (final/sinusoidal.cu:838-855)."""
    st, ct = oracle.sinusoidal_table(npos, D)
    f = 1.0 / 10000.0 ** (2.0 * (np.arange(D) // 2) / D)
    th = np.arange(npos, dtype=np.float64)[:, None] * f[None, :]
    tol = 1e-6 + 2.5e-7 * np.arange(npos)[:, None]
    assert np.all(np.abs(st - np.sin(th)) <= tol)
    assert np.all(np.abs(ct - np.cos(th)) <= tol)


def test_sinusoidal_pos0_pattern():
    st, ct = oracle.sinusoidal_table(4, 10)
    X = np.zeros((1, 1, 4, 10), dtype=np.float32)
    Y = oracle.add_sinusoidal(X, st, ct)
    assert np.array_equal(Y[0, 0, 0], np.array([0, 1] * 5, dtype=np.float32))
    oracle.set_mutation(2)
    st2, ct2 = oracle.sinusoidal_table(4, 10)
    Y2 = oracle.add_sinusoidal(X, st2, ct2)
    assert not np.array_equal(Y2[0, 0, 0], Y[0, 0, 0])


def test_sinusoidal_linearity_and_positions():
    """attn_sin(Q,K,V) == attn(Q + PE_q, K + PE_k, V), positions 0.. for each side."""
    rng = np.random.default_rng(14)
    B, Hh, Lq, Lk, D = 1, 2, 12, 30, 36
    Q = rng.standard_normal((B, Hh, Lq, D), dtype=np.float32) * 0.5
    K = rng.standard_normal((B, Hh, Lk, D), dtype=np.float32) * 0.5
    V = rng.standard_normal((B, Hh, Lk, D), dtype=np.float32)
    st, ct = oracle.sinusoidal_table(max(Lq, Lk), D)
    a = oracle.attention_sinusoidal(Q, K, V, st, ct)
    ref = sdpa64(oracle.add_sinusoidal(Q, st, ct), oracle.add_sinusoidal(K, st, ct), V)
    assert np.allclose(a, ref, atol=3e-6)
    only_q = oracle.attention_sinusoidal(Q, K, V, st, ct, add_k=False)
    assert np.allclose(only_q, sdpa64(oracle.add_sinusoidal(Q, st, ct), K, V), atol=3e-6)
    oracle.set_mutation(4)  # keys take the query's position
    bad = oracle.attention_sinusoidal(Q, K, V, st, ct)
    assert not np.allclose(bad, ref, atol=1e-3)


# ------------------------------------------------------------------ bf16 rounding
def test_bf16_rne_matches_torch():
    import torch
    rng = np.random.default_rng(15)
    x = np.concatenate([
        rng.standard_normal(20000, dtype=np.float32) * 10,
        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38], dtype=np.float32),
        # exact ties: low 16 bits == 0x8000 with even and odd upper halves
        (np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x00008000], dtype=np.uint32)
         .view(np.float32)),
    ])
    ours = oracle.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    back = oracle.bf16_bits_to_f32(ours)
    assert np.array_equal(back, torch.from_numpy(x).to(torch.bfloat16).float().numpy())
    nan = oracle.f32_to_bf16_bits(np.array([np.nan], dtype=np.float32))
    assert np.isnan(oracle.bf16_bits_to_f32(nan)[0])


def test_oracle_drift_at_wide_logits():
    """The oracle restates the reference's CPU loops (float accumulators,
    sequential sums over head_d): at sigma 3 inputs (logits up to about +-40)
    and head_d >= 2048 those float32 sums themselves miss the 1e-4 bar
    against the exact float64 SDPA of the same inputs, while at head_d = 512
    they stay within it.  The GPU parity tests at these shapes therefore take
    the exact result as a second referee (tests/helpers.py
    check_f32_or_truth).  Seeds and shapes are those of
    test_gpu_parity.py::test_sdpa_f32_wider_logits."""
    cases = {(1, 4, 64, 64, 512): (0, 1e-4), (1, 4, 64, 64, 2048): (1, 2e-4),
             (1, 4, 32, 128, 2048): (100, 4e-4)}
    for (B, Hh, Lq, Lk, D), (min_fails, max_abs) in cases.items():
        Q, K, V = H.rng_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), seed=7 + D, sigma=3.0)
        ref = oracle.attention(Q, K, V, nthreads=8)
        n, mabs, _ = H.check_f32(ref, H.sdpa64(Q, K, V))
        assert n >= min_fails and (min_fails > 0 or n == 0), ((B, Hh, Lq, Lk, D), n)
        assert mabs < max_abs, ((B, Hh, Lq, Lk, D), mabs)
