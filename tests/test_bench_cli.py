"""bench.py's command-line contract on the CPU: this build measures one GPU,
so more than one (by flag or by a launcher's WORLD_SIZE) is refused with a
message and exit status 2 before any GPU work."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT,
                          env=env, capture_output=True, text=True, timeout=120)


def test_bench_refuses_more_than_one_gpu():
    r = _run(["--gpus", "2"])
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_bench_refuses_a_multi_rank_launch():
    r = _run([], {"WORLD_SIZE": "2"})
    assert r.returncode == 2
    assert "one GPU only" in r.stderr


def test_bench_help_lists_the_contract_flags():
    r = _run(["--help"])
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--config", "--head-dim"):
        assert flag in r.stdout


def _bench_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_sampled_check_passes_oracle_rows_and_fails_a_perturbed_output():
    """The bench's parity gate: rows of the first, a middle and the last head
    equal to the oracle pass; an output off by 2e-4 in one element fails the
    fp32 bar, and a bf16 output off by 5 % fails the bf16 bar."""
    import numpy as np
    b = _bench_module()
    rng = np.random.default_rng(3)
    for cfg in (("t f32", "f32", 1, 3, 20, 24, 64, "none", 1.0),
                ("t bf16 sin", "bf16", 2, 2, 20, 40, 32, "sinusoidal", 0.5),
                ("t bf16 rope", "bf16", 1, 3, 16, 16, 32, "rope_half", 1.0)):
        _, dt, B, Hh, Lq, Lk, D, pe, sg = cfg
        host = [rng.standard_normal(s, dtype=np.float32) * np.float32(sg)
                for s in ((B, Hh, Lq, D), (B, Hh, Lk, D), (B, Hh, Lk, D))]
        full = {bh: b.oracle_rows(cfg, host, bh, 0, Lq) for bh in range(B * Hh)}
        good = b.sampled_check(cfg, host, lambda bh, r0, r1: full[bh][r0:r1])
        assert good["ok"] and good["fails"] == 0 and good["heads_checked"][-1] == B * Hh - 1
        assert good["rows_checked"] >= 12

        def bad_rows(bh, r0, r1):
            x = full[bh][r0:r1].copy()
            if bh == B * Hh - 1 and r1 == Lq:
                x[-1, 0] += np.float32(2e-4 if dt == "f32" else 0.05 * (abs(x[-1, 0]) + 1))
            return x
        bad = b.sampled_check(cfg, host, bad_rows)
        assert not bad["ok"], cfg


def test_cpu_baseline_reports_a_bounded_sample():
    import numpy as np
    b = _bench_module()
    cfg = ("t", "f32", 1, 2, 16, 16, 64, "none", 1.0)
    rng = np.random.default_rng(4)
    host = [rng.standard_normal(s, dtype=np.float32) for s in ((1, 2, 16, 64), (1, 2, 16, 64),
                                                              (1, 2, 16, 64))]
    gbs, job_ms, sample = b.cpu_baseline(cfg, host, 0.05)
    assert gbs > 0 and job_ms > 0 and "single thread" in sample
    info = b.host_info()
    assert info["nproc_usable"] >= 1 and info["cpu_model"]
