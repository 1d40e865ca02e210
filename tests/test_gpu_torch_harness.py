"""The PyTorch comparison harness on the GPU (the reference's harness:
final/benchmark_pytorch_wrapper.cu:147-247).

torch_compare.py hands torch's device tensors and stream to this library.
It runs here as its own process on BASELINE config 2 and one of the
reference harness's shapes.  The test then checks three things:
  - the process mapped exactly one HIP runtime (the harness stops
    otherwise, and records the runtime's path in each JSON row);
  - the library's output, saved by the harness, meets the fp32 bar against
    the CPU oracle on the same inputs;
  - the timings are positive.
torch's first import on a fresh box can take a minute or two, hence the
longer time limit.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import helpers as H
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "accelerated-final-project_amd", "torch_compare.py")

pytestmark = pytest.mark.gpu


@pytest.mark.timeout(600)
def test_torch_harness_runs_with_one_runtime_and_oracle_parity(am, dev, tmp_path):
    print("[case] torch_compare.py on cfg2 and ref hdim=512", flush=True)
    out_json = tmp_path / "rows.json"
    save = tmp_path / "saved"
    r = subprocess.run([sys.executable, HARNESS, "--iters", "5", "--warmup", "2",
                        "--shapes", "cfg2,ref hdim=512", "--json", str(out_json),
                        "--save", str(save)],
                       capture_output=True, text=True, timeout=580)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-2000:])
    rows = json.load(open(out_json))
    assert [row["shape"] for row in rows] == ["ref hdim=512", "cfg2"]
    runtimes = {row["hip_runtime"] for row in rows}
    assert len(runtimes) == 1 and "libamdhip64" in next(iter(runtimes))
    for idx, row in enumerate(rows):
        assert row["ours_ms"] > 0 and row["torch_sdpa_ms"] > 0 and row["torch_naive_ms"] > 0
        Q, K, V, got = (np.load(save / f"{idx}_{t}.npy") for t in ("Q", "K", "V", "out"))
        ref = oracle.attention(Q, K, V, nthreads=16)
        n, mabs, mrel = H.check_f32(got, ref)
        assert n == 0, f"{row['shape']}: {n} mismatches, max abs {mabs}, max rel {mrel}"
