import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("accelerated-final-project_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (runs on the MI355X box)")


@pytest.fixture(scope="session")
def am():
    """The product binding; fails loudly if the HIP library is not built."""
    import attn_mi355x
    attn_mi355x.lib()
    return attn_mi355x


@pytest.fixture(scope="session")
def dev(am):
    """Device 0 through the library's own HIP runtime (no PyTorch)."""
    import hip_rt
    if hip_rt.device_count() < 1:
        pytest.fail("GPU test collected on a host without a HIP device")
    print(f"[gpu] device: {hip_rt.device_name(0)}", flush=True)
    return 0


@pytest.fixture
def tuner(am):
    """Tuning overrides (atn_set_tuning_ex) for one test, reset after it.
    tuner.set(**kw) adds to the test's overrides; tuner.clear() drops them."""
    class _Tuner:
        def __init__(self):
            self.kw = {}

        def set(self, **kw):
            self.kw.update(kw)
            am.set_tuning(**self.kw)

        def clear(self):
            self.kw = {}
            am.set_tuning()

    t = _Tuner()
    yield t
    am.set_tuning()


@pytest.fixture(autouse=True)
def _no_silent_rerun(request):
    """Every GPU test ends with no synchronous drop-in rerun after a timed-out
    single-launch wait (a test that forces one resets the count itself)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    import attn_mi355x
    n = attn_mi355x.rerun_count(reset=True)
    assert n == 0, f"{n} drop-in call(s) were rerun after a device-side wait timed out"
