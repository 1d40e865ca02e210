"""Seeded random shapes through atn_attention_fwd_ex (and, for some plain
cases, the allocation-free entry point) against the CPU oracle: fp32 and
bf16; no encoding, interleaved RoPE (full or partial rotary width),
rotate-half RoPE and sinusoidal; encodings on both sides, Q only or K only;
query and key lengths inside and outside the single-launch window and
across the GEMM path's 256-row tiles; head dims from 8 to 4096.  The cases
are fixed by the seed, so a failure names a reproducible case.

fp32: element fails iff abs > 1e-4 AND rel > 1e-4 against the oracle (for
sinusoidal shapes with D >= 4096 the exact float64 result is a second
referee, as in test_gpu_parity.py).  bf16: rel 2e-2 against the fp32 oracle
on the bf16-rounded inputs.
"""
import numpy as np
import pytest

import helpers as H
import oracle

pytestmark = pytest.mark.gpu

N_CASES = 150
SEED = 20261202
D_CHOICES = [8, 16, 36, 64, 96, 128, 200, 256, 512, 520, 1024, 2048, 4096]


def _cases():
    rng = np.random.default_rng(SEED)
    out = []
    for i in range(N_CASES):
        dt = str(rng.choice(["f32", "bf16"]))
        pe = str(rng.choice(["none", "none", "rope", "rope_half", "sinusoidal"]))
        B, Hh = int(rng.integers(1, 3)), int(rng.integers(1, 4))
        kind = int(rng.integers(0, 3))
        if kind == 0:  # the single-launch window
            Lq, Lk = int(rng.integers(1, 65)), int(rng.integers(1, 129))
        elif kind == 1:
            Lq, Lk = int(rng.integers(1, 300)), int(rng.integers(1, 600))
        else:
            Lq, Lk = int(rng.integers(100, 520)), int(rng.integers(100, 1100))
        D = int(rng.choice(D_CHOICES))
        if B * Hh * max(Lq, Lk) * D > 6_000_000:  # keeps the oracle at a second or less
            D = max(8, 6_000_000 // (B * Hh * max(Lq, Lk)) // 8 * 8)
        aq, ak = [(True, True), (True, True), (True, False), (False, True)][int(rng.integers(0, 4))]
        rot = D
        if pe == "rope" and rng.integers(0, 3) == 0:
            rot = int(rng.integers(1, D // 2 + 1)) * 2
        noalloc = pe == "none" and int(rng.integers(0, 3)) == 0
        out.append((i, dt, pe, (B, Hh, Lq, Lk, D), aq, ak, rot, noalloc))
    return out


CASES = _cases()

# A second set weighted toward long key rows with few query rows (the flash
# kernel's 32-row waves with key splits from 4096 keys on) and encodings in
# the single-launch window, rotate-half at partial rotary widths too.
N_LONG = 60
SEED_LONG = 20261203


def _long_cases():
    rng = np.random.default_rng(SEED_LONG)
    out = []
    for i in range(N_LONG):
        dt = str(rng.choice(["f32", "bf16"]))
        pe = str(rng.choice(["none", "rope", "rope_half", "sinusoidal"]))
        if rng.integers(0, 2) == 0:  # long keys
            B, Hh = 1, int(rng.integers(1, 3))
            Lq, Lk = int(rng.integers(1, 260)), int(rng.integers(3000, 9000))
            D = int(rng.choice([32, 64, 100, 128, 192, 256]))
        else:  # the single-launch window
            B, Hh = int(rng.integers(1, 3)), int(rng.integers(1, 4))
            Lq, Lk = int(rng.integers(1, 65)), int(rng.integers(1, 129))
            D = int(rng.choice([64, 128, 512, 1024, 2048, 4096]))
        if B * Hh * max(Lq, Lk) * D > 8_000_000:
            D = max(8, 8_000_000 // (B * Hh * max(Lq, Lk)) // 8 * 8)
        aq, ak = [(True, True), (True, True), (True, False), (False, True)][int(rng.integers(0, 4))]
        rot = D
        if pe in ("rope", "rope_half") and rng.integers(0, 3) == 0:
            rot = int(rng.integers(1, D // 2 + 1)) * 2
        out.append((1000 + i, dt, pe, (B, Hh, Lq, Lk, D), aq, ak, rot, False))
    return out


LONG_CASES = _long_cases()


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[1]}-{c[2]}-" + "x".join(map(str, c[3])))
def test_random_shape(am, dev, case):
    _run_case(am, case)


@pytest.mark.parametrize("case", LONG_CASES,
                         ids=lambda c: f"{c[0]}-{c[1]}-{c[2]}-" + "x".join(map(str, c[3])))
def test_random_long_keys_and_encodings(am, dev, case):
    _run_case(am, case)


def _run_case(am, case):
    import hip_rt
    i, dt, pe, shape, aq, ak, rot, noalloc = case
    B, Hh, Lq, Lk, D = shape
    print(f"[case] random {i}: {dt} {pe} rot={rot} q={aq} k={ak} {shape} noalloc={noalloc}",
          flush=True)
    desc = {"none": None,
            "rope": am.make_pe("rope", rotary_dim=rot, apply_q=aq, apply_k=ak),
            "rope_half": am.make_pe("rope", pairing="half", rotary_dim=rot, apply_q=aq,
                                    apply_k=ak),
            "sinusoidal": am.make_pe("sinusoidal", apply_q=aq, apply_k=ak)}[pe]
    sigma = 0.5 if pe == "sinusoidal" else 1.0
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 1000 + i, dt, sigma)
    out = H.empty((B, Hh, Lq, D), dt)
    if noalloc:
        am.attention_noalloc_ex(q, k, v, out)
    else:
        am.attention_ex(q, k, v, out, pe=desc)
    hip_rt.synchronize()
    got = out.numpy()
    L = max(Lq, Lk)
    if pe == "none":
        ref = oracle.attention(Q, K, V, nthreads=16)
    elif pe == "sinusoidal":
        st, ct = oracle.sinusoidal_table(L, D)
        ref = oracle.attention_sinusoidal(Q, K, V, st, ct, add_q=aq, add_k=ak, nthreads=16)
    else:
        c, s = oracle.rope_cache(L, rot)
        ref = oracle.attention_rope(Q, K, V, c, s, rotary_dim=rot,
                                    pairing="half" if pe == "rope_half" else "interleaved",
                                    rotate_q=aq, rotate_k=ak, nthreads=16)
    if dt == "f32":
        if pe == "sinusoidal" and D >= 4096:
            Qe = oracle.add_sinusoidal(Q, st, ct) if aq else Q
            Ke = oracle.add_sinusoidal(K, st, ct) if ak else K
            n, mabs, _ = H.check_f32_or_truth(got, ref, H.sdpa64(Qe, Ke, V))
        else:
            n, mabs, _ = H.check_f32(got, ref)
        assert n == 0, f"{n} mismatches, max abs {mabs}"
    else:
        n, nrel, mabs = H.check_bf16(got, ref)
        assert n == 0, f"normwise rel {nrel}, max abs {mabs}"
