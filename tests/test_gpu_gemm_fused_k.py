"""GPU parity of the GEMM path's fused K encoding and of its gated fallback.

With a positional encoding, D % 128 == 0, the library's tables and at most
four 256-row query tiles, the QK^T GEMM reads raw bf16 K and encodes it on
its way to LDS from fp16 tables (no K~ pass).  Every case here runs twice,
with the fusion forced on (ATN_GEMM_FUSED_K=1) and switched off (=-1: K~
from the row-scaled encoder), and both results must meet the bf16 bar
against the CPU oracle: within rel 2e-2 of the fp32 oracle run on the
bf16-rounded inputs (elementwise against |ref| and rms(ref), and
norm-wise).

Keys whose encoded magnitude exceeds fp16's range (65504) make the
workgroups whose key tiles hold them compute their tiles a second time with
per-row power-of-two scales (those of the row-scaled K~ pass); tiles
without such keys keep the first pass.
"""
import os

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

# (name, desc kwargs, oracle call)
MODES = {
    "rope_half": dict(kind="rope", pairing="half"),
    "rope_inter": dict(kind="rope"),
    "rope_inter_r128": dict(kind="rope", rotary_dim=128),
    "sinusoidal": dict(kind="sinusoidal"),
    "rope_q_only": dict(kind="rope", pairing="half", apply_k=False),
    "sin_k_only": dict(kind="sinusoidal", apply_q=False),
}


def _ref(mode, Q, K, V, rows=None):
    kw = MODES[mode]
    Lq, Lk, D = Q.shape[2], K.shape[2], Q.shape[3]
    n = max(Lq, Lk)
    if kw["kind"] == "sinusoidal":
        st, ct = oracle.sinusoidal_table(n, D)
        return oracle.attention_sinusoidal(Q, K, V, st, ct, add_q=kw.get("apply_q", True),
                                           add_k=kw.get("apply_k", True), rows=rows, nthreads=16)
    r = kw.get("rotary_dim", 0) or D
    c, s = oracle.rope_cache(n, r)
    return oracle.attention_rope(Q, K, V, c, s, rotary_dim=r, pairing=kw.get("pairing", "interleaved"),
                                 rotate_q=kw.get("apply_q", True), rotate_k=kw.get("apply_k", True),
                                 rows=rows, nthreads=16)


def _run(am, q, k, v, shape, desc, fused):
    import hip_rt
    old = os.environ.get("ATN_GEMM_FUSED_K")
    os.environ["ATN_GEMM_FUSED_K"] = "1" if fused else "-1"
    try:
        out = H.empty(shape, "bf16")
        am.attention_ex(q, k, v, out, pe=desc)
        hip_rt.synchronize()
        return out.numpy()
    finally:
        if old is None:
            del os.environ["ATN_GEMM_FUSED_K"]
        else:
            os.environ["ATN_GEMM_FUSED_K"] = old


@pytest.mark.parametrize("shape", [(1, 2, 256, 640, 256), (1, 1, 300, 512, 384)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("mode", list(MODES))
def test_fused_k_encoding(am, dev, shape, mode):
    """Interior and edge tiles (ragged Lq / Lk), every encoding, partial
    rotary width (pass-through pairs), query-only and key-only encodings
    (the key-only GEMM converts raw K)."""
    B, Hh, Lq, Lk, D = shape
    print(f"[case] fused K {shape} {mode}", flush=True)
    desc = am.make_pe(**MODES[mode])
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM
    sigma = 0.5 if MODES[mode]["kind"] == "sinusoidal" else 1.0
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 31 + Lk, "bf16",
                                           sigma)
    ref = _ref(mode, Q, K, V)
    for fused in (True, False):
        got = _run(am, q, k, v, Q.shape, desc, fused)
        n, nrel, mabs = H.check_bf16(got, ref)
        assert n == 0, f"fused={fused}: normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("mode", list(MODES))
def test_fused_k_four_query_tiles(am, dev, mode):
    """1000 query rows are four 256-row query tiles, the most the planner
    fuses (the last one ragged), over 520 keys (a ragged key tile); fused
    and K~-pass results both meet the bf16 bar against the oracle."""
    B, Hh, Lq, Lk, D = 1, 1, 1000, 520, 256
    print(f"[case] fused K four query tiles {mode}", flush=True)
    desc = am.make_pe(**MODES[mode])
    assert am.path(1, B, Hh, Lq, Lk, D, desc) == am.ATN_PATH_GEMM
    sigma = 0.5 if MODES[mode]["kind"] == "sinusoidal" else 1.0
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 1031, "bf16", sigma)
    ref = _ref(mode, Q, K, V)
    for fused in (True, False):
        got = _run(am, q, k, v, Q.shape, desc, fused)
        n, nrel, mabs = H.check_bf16(got, ref)
        assert n == 0, f"fused={fused}: normwise rel {nrel}, max abs {mabs}"


def test_fused_k_config4_head_shape(am, dev):
    """The fused rotate-half GEMM forced on at config 4's per-head shape
    (1024 x 1024, D = 4096: interior tiles only, 64 K steps), two heads;
    the oracle checks 16 sampled query rows per head."""
    B, Hh, Lq, Lk, D = 1, 2, 1024, 1024, 4096
    print("[case] fused K config-4 head shape", flush=True)
    desc = am.make_pe(**MODES["rope_half"])
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 9, "bf16", 1.0)
    got = _run(am, q, k, v, Q.shape, desc, True).reshape(-1, D)
    rng = np.random.default_rng(4)
    for h in range(B * Hh):
        rows = np.sort(rng.choice(Lq, 16, replace=False)) + h * Lq
        ref = np.concatenate([_ref("rope_half", Q, K, V, rows=(int(r), int(r) + 1))
                              .reshape(-1, D)[r:r + 1] for r in rows])
        n, nrel, mabs = H.check_bf16(got[rows], ref)
        assert n == 0, f"head {h}: normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("mode", ["rope_half", "rope_inter", "sin_k_only", "rope_q_only"])
def test_fused_k_range_scaled_pass(am, dev, mode):
    """Two key rows carry ~1e5 (beyond fp16) in dims 8, 9, 8 + D/2, 9 + D/2,
    where every query is zero (so after the encodings, which pair dims
    within those sets, those products are exactly zero and the scores stay
    well conditioned): the workgroups of those rows' key tiles redo their
    tiles with row scales, the others do not.  Then a call on ordinary keys
    must be right as well."""
    import hip_rt
    B, Hh, Lq, Lk, D = 1, 2, 256, 512, 256
    print(f"[case] fused K scaled pass {mode}", flush=True)
    desc = am.make_pe(**MODES[mode])
    rng = np.random.default_rng(5)
    Qf = rng.standard_normal((B, Hh, Lq, D), dtype=np.float32)
    Kf = rng.standard_normal((B, Hh, Lk, D), dtype=np.float32)
    Vf = rng.standard_normal((B, Hh, Lk, D), dtype=np.float32)
    big = [8, 9, 8 + D // 2, 9 + D // 2]
    Qf[..., big] = 0.0
    Kbig = Kf.copy()
    Kbig[:, :, 37, big] *= np.float32(1e5)
    Kbig[:, 1, 300, big] *= np.float32(3e5)
    q, kb, v = (hip_rt.DeviceArray.from_numpy(x, "bf16") for x in (Qf, Kbig, Vf))
    Q, Kb, V = (t.numpy() for t in (q, kb, v))
    assert np.abs(Kb).max() > 65504
    got = _run(am, q, kb, v, Q.shape, desc, True)
    n, nrel, mabs = H.check_bf16(got, _ref(mode, Q, Kb, V))
    assert n == 0, f"large keys: normwise rel {nrel}, max abs {mabs}"
    k = hip_rt.DeviceArray.from_numpy(Kf, "bf16")
    K = k.numpy()
    got = _run(am, q, k, v, Q.shape, desc, True)
    n, nrel, mabs = H.check_bf16(got, _ref(mode, Q, K, V))
    assert n == 0, f"ordinary keys: normwise rel {nrel}, max abs {mabs}"


@pytest.mark.parametrize("mode", ["sinusoidal", "rope_half"])
def test_fused_k_batch_and_heads(am, dev, mode):
    """B = 2 and H = 2 (head strides of Q~, K, the table rows shared by every
    head) through the fused form."""
    B, Hh, Lq, Lk, D = 2, 2, 256, 512, 256
    print(f"[case] fused K batch x heads {mode}", flush=True)
    desc = am.make_pe(**MODES[mode])
    sigma = 0.5 if MODES[mode]["kind"] == "sinusoidal" else 1.0
    (q, k, v), (Q, K, V) = H.device_inputs((B, Hh, Lq, D), (B, Hh, Lk, D), 55, "bf16", sigma)
    got = _run(am, q, k, v, Q.shape, desc, True)
    n, nrel, mabs = H.check_bf16(got, _ref(mode, Q, K, V))
    assert n == 0, f"normwise rel {nrel}, max abs {mabs}"
