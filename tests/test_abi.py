"""C-ABI boundary tests that need no GPU.

* libattn_mi355x.so loads and exports every function include/attn_mi355x.h
  declares;
* every argument error of the _ex entry points is reported with its status
  code before any HIP call (fake, never dereferenced device addresses are
  passed: validation rejects them first);
* on a host without a HIP device a valid call reports ATN_ERR_NO_DEVICE;
* the drop-in entry points keep the reference's error convention (print,
  then exit(EXIT_FAILURE); final/attention.cu:12-21) -- checked in a child
  process;
* the host-side table builders (precompute_rope_cache,
  precompute_sinusoidal_table) give the oracle's bits.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Fake device addresses: 256-byte aligned, far apart, never dereferenced
# (every call below is rejected by validation before any HIP call).
QA, KA, VA, OA, WA = (0x7F0000000000 + i * 0x100000000 for i in range(5))


@pytest.fixture(scope="module")
def L(am):
    return am.lib()


def test_exports_every_header_function(am, L):
    names = am.header_functions()
    assert "attention_forward_optimized" in names and len(names) >= 20
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/attn_mi355x.h but not exported"


def test_reference_dropin_names_present(am):
    """The drop-in names of the reference's host launchers."""
    names = set(am.header_functions())
    for n in ["attention_forward_optimized", "attention_forward", "attention_forward_rope_fused",
              "attention_forward_rope_fused_v7_hybrid", "attention_forward_separate_rope",
              "attention_forward_sinusoidal_hybrid", "attention_forward_sinusoidal_separate",
              "attention_forward_bf16", "attention_forward_rope_bf16",
              "attention_forward_sinusoidal_bf16", "precompute_rope_cache"]:
        assert n in names


def test_status_strings(am, L):
    for code in range(0, -12, -1):
        s = am.status_string(code)
        assert s and s != "unknown status"
    assert am.status_string(-99) == "unknown status"


def fwd(am, L, dtype=0, q=QA, k=KA, v=VA, o=OA, B=1, H=4, Lq=64, Lk=64, D=2048, pe=None,
        ws=None, wsb=0):
    return L.atn_attention_fwd_ex(dtype, q, k, v, o, B, H, Lq, Lk, D,
                                  ctypes.byref(pe) if pe is not None else None, ws, wsb, None)


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=7), -9),
    (dict(q=None), -1), (dict(k=None), -1), (dict(v=None), -1), (dict(o=None), -1),
    (dict(B=0), -2), (dict(H=-1), -2), (dict(Lq=0), -2), (dict(Lk=0), -2), (dict(D=0), -2),
    (dict(B=1 << 20, H=1 << 20, Lq=1 << 20, D=1 << 20), -4),
    (dict(Lq=1 << 20, D=1 << 12), -4),  # one head's Lq*D beyond 32-bit row indexing
    (dict(q=QA + 2), -10), (dict(o=OA + 1), -10),
    (dict(dtype=1, v=VA + 1), -10),
    (dict(o=QA + 64), -5),  # out overlaps Q
    (dict(o=VA), -5),
    (dict(ws=WA, wsb=16), -8),
])
def test_fwd_ex_validation(am, L, kw, code):
    assert fwd(am, L, **kw) == code


@pytest.mark.parametrize("pe_kw,code", [
    (dict(kind="rope", rotary_dim=7), -3),
    (dict(kind="rope", rotary_dim=4096), -3),
    (dict(kind="rope", rotary_dim=-2), -3),
])
def test_fwd_ex_rope_validation(am, L, pe_kw, code):
    pe = am.make_pe(**pe_kw)
    assert fwd(am, L, pe=pe) == code


def test_fwd_ex_pe_descriptor_errors(am, L):
    pe = am.make_pe("rope")
    pe.pairing = 5
    assert fwd(am, L, pe=pe) == -9
    pe = am.make_pe("rope")
    pe.table_a = 0x1000
    assert fwd(am, L, pe=pe) == -1  # one table without the other
    pe = am.make_pe("sinusoidal")
    pe.kind = 9
    assert fwd(am, L, pe=pe) == -9
    pe = am.make_pe("rope")
    pe.base = -1.0
    assert fwd(am, L, pe=pe) == -9
    pe = am.make_pe("rope", rotary_dim=0)
    assert fwd(am, L, pe=pe, D=9) == -3  # rotary = head_d must be even


def test_pe_apply_ex_validation(am, L):
    pe = am.make_pe("rope")
    f = L.atn_pe_apply_ex
    assert f(0, None, OA, 10, 10, 64, ctypes.byref(pe), None) == -1
    assert f(0, QA, OA, 0, 10, 64, ctypes.byref(pe), None) == -2
    assert f(0, QA, OA, 10, 0, 64, ctypes.byref(pe), None) == -2
    assert f(0, QA, QA + 8, 10, 10, 64, ctypes.byref(pe), None) == -5
    assert f(3, QA, OA, 10, 10, 64, ctypes.byref(pe), None) == -9
    assert f(0, QA, OA, 10, 10, 64, None, None) == -1
    none = am.PeDesc()
    assert f(0, QA, OA, 10, 10, 64, ctypes.byref(none), None) == -9  # kind NONE


def test_workspace_bytes(am):
    n = am.workspace_bytes(0, 1, 4, 64, 64, 2048)
    assert n > 0 and n % 4 == 0
    assert am.workspace_bytes(0, 0, 4, 64, 64, 2048) == 0
    assert am.workspace_bytes(9, 1, 4, 64, 64, 2048) == 0
    assert am.workspace_bytes(0, 1, 4, 64, 64, 2048, am.make_pe("rope", rotary_dim=3)) == 0


@pytest.mark.parametrize("dtype,shape", [(0, (1, 4, 64, 64, 2048)), (0, (1, 16, 64, 64, 512)),
                                         (0, (1, 1, 16, 16, 8192)), (1, (1, 4, 32, 128, 8192))])
def test_workspace_bytes_bound_every_plan(am, tuner, dtype, shape):
    """The size query reports the largest workspace of every single-launch
    plan it could take, so that a plan forced through the tuning overrides
    (or chosen for a device of another capacity) never needs more."""
    base = am.workspace_bytes(dtype, *shape)
    assert base > 0
    for rows, dc, x in [(16, 32, "gather"), (16, 32, "rsag"), (32, 64, "rsag"),
                        (64, 128, "rsag"), (16, 256, "gather")]:
        tuner.set(fused_rows=rows, fused_dc=dc, fused_exchange=x)
        assert am.workspace_bytes(dtype, *shape) == base, (rows, dc, x)


def test_path_selection_without_device(am, tuner):
    """Short sequences take the single-launch kernel, long ones the pipeline."""
    assert am.path(0, 1, 4, 64, 64, 2048) == am.ATN_PATH_FUSED_SMALL       # config 2
    assert am.path(1, 1, 4, 32, 128, 8192) == am.ATN_PATH_FUSED_SMALL      # config 3
    assert am.path(0, 1, 1, 4, 4, 8) == am.ATN_PATH_FUSED_SMALL            # config 1
    # fp32 outside the single-launch window with head_d <= 256 (128 with an
    # encoding) and head_d % 4 == 0 runs on the flash kernel
    assert am.path(0, 4, 32, 512, 512, 128) == am.ATN_PATH_FLASH
    assert am.path(0, 1, 1, 3, 129, 36) == am.ATN_PATH_FLASH
    assert am.path(0, 1, 300, 16, 16, 64) == am.ATN_PATH_FLASH             # more heads than CUs
    assert am.path(0, 1, 4, 512, 512, 256) == am.ATN_PATH_FLASH
    assert am.path(0, 1, 4, 512, 512, 128, am.make_pe("rope")) == am.ATN_PATH_FLASH
    assert am.path(0, 1, 4, 512, 512, 256, am.make_pe("rope")) == am.ATN_PATH_SPLIT_D
    assert am.path(0, 1, 4, 512, 512, 260) == am.ATN_PATH_SPLIT_D           # head_d > 256
    assert am.path(0, 1, 4, 512, 512, 130) == am.ATN_PATH_SPLIT_D           # head_d % 4 != 0
    assert am.path(0, 1, 4, 512, 512, 2048) == am.ATN_PATH_SPLIT_D
    # bf16 outside the single-launch window: the flash kernel at head_d <=
    # 256 (128 with an encoding; head_d % 4 == 0), past that the MFMA GEMM
    # path whenever D % 8 == 0, whatever len_q and len_k are
    assert am.path(1, 4, 32, 512, 512, 128) == am.ATN_PATH_FLASH
    assert am.path(1, 1, 4, 512, 512, 128, am.make_pe("rope")) == am.ATN_PATH_FLASH
    assert am.path(1, 1, 2, 200, 20, 36) == am.ATN_PATH_FLASH
    assert am.path(1, 1, 4, 512, 512, 256) == am.ATN_PATH_FLASH
    assert am.path(1, 1, 4, 512, 512, 256, am.make_pe("rope")) == am.ATN_PATH_GEMM
    assert am.path(1, 1, 4, 512, 512, 264) == am.ATN_PATH_GEMM
    assert am.path(1, 8, 8, 1024, 1024, 4096) == am.ATN_PATH_GEMM          # config 4
    assert am.path(1, 1, 8, 64, 4096, 2048) == am.ATN_PATH_GEMM
    assert am.path(1, 1, 4, 100, 100, 2048) == am.ATN_PATH_GEMM
    assert am.path(1, 1, 2, 200, 20, 512) == am.ATN_PATH_GEMM
    assert am.path(1, 1, 2, 200, 20, 34) == am.ATN_PATH_SPLIT_D           # D % 4 != 0
    assert am.path(1, 1, 2, 200, 20, 516) == am.ATN_PATH_SPLIT_D          # D % 8 != 0
    assert am.path(0, 0, 4, 64, 64, 2048) == -2
    tuner.set(no_flash=True)
    assert am.path(0, 4, 32, 512, 512, 128) == am.ATN_PATH_SPLIT_D
    assert am.path(1, 4, 32, 512, 512, 128) == am.ATN_PATH_GEMM


def test_no_device_path(am, L):
    if am.device_count() > 0:
        pytest.skip("a HIP device is visible; the no-device path is exercised on the CPU host")
    assert fwd(am, L) == -6
    assert L.atn_prepare_pe_ex(ctypes.byref(am.make_pe("rope")), 64, 64) == -6


def _child(code: str):
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join(
        [os.path.join(ROOT, "accelerated-final-project_amd"), env.get("PYTHONPATH", "")])
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                          timeout=120, env=env)


def test_dropin_exits_on_bad_argument():
    """Reference convention: print the error and exit(EXIT_FAILURE)."""
    r = _child("import attn_mi355x as a; a.lib().attention_forward_optimized("
               f"{QA}, {KA}, {VA}, {OA}, 0, 4, 64, 64, 2048)")
    assert r.returncode == 1
    assert "attn_mi355x error -2" in r.stderr and "attention_forward_optimized" in r.stderr


def test_dropin_exits_on_aliasing():
    r = _child("import attn_mi355x as a; a.lib().attention_forward_bf16("
               f"{QA}, {KA}, {VA}, {QA}, 1, 4, 64, 64, 2048)")
    assert r.returncode == 1 and "attn_mi355x error -5" in r.stderr


def test_host_rope_cache_matches_oracle(am):
    for npos, r in [(16, 8), (1024, 128), (64, 2048)]:
        c, s = am.precompute_rope_cache(npos, r)
        oc, os_ = oracle.rope_cache(npos, r)
        assert np.array_equal(c, oc) and np.array_equal(s, os_)


def test_host_sinusoidal_table_matches_oracle(am):
    for npos, d in [(16, 8), (2048, 1024), (33, 7)]:
        s, c = am.precompute_sinusoidal_table(npos, d)
        os_, oc = oracle.sinusoidal_table(npos, d)
        assert np.array_equal(s, os_) and np.array_equal(c, oc)


def test_python_binding_checks_shapes(am):
    import hip_rt

    class Fake:
        pass
    with pytest.raises(ValueError):
        am._check(Fake(), "f32", (1,), "Q")
    assert hip_rt.bf16_bits_to_f32(hip_rt.f32_to_bf16_bits(np.float32([1.5])))[0] == 1.5


def test_workspace_bytes_bounded_by_the_cap(am, tuner):
    """The size query never asks for more than the library's scratch cap
    (1 GiB by default): a larger shape runs in chunks of heads or query rows,
    and the query reports the largest chunk's need."""
    big = am.workspace_bytes(1, 1, 64, 8192, 8192, 128)   # E alone would be 8 GiB
    assert 0 < big <= 1 << 30
    small = am.workspace_bytes(1, 1, 4, 512, 512, 128)
    assert small < 1 << 30
    tuner.set(workspace_cap_mib=1)
    assert am.workspace_bytes(1, 1, 4, 512, 512, 128) <= 1 << 20
    assert am.workspace_bytes(1, 1, 64, 8192, 8192, 128) <= 1 << 20


def test_torch_and_library_share_one_hip_runtime():
    """torch's bundled libamdhip64 and /opt/rocm's share the SONAME
    libamdhip64.so.7: with torch imported first, loading the library maps no
    second HIP runtime (what torch_compare.py relies on to pass torch's
    device pointers in)."""
    code = ("import torch, sys; sys.path.insert(0, %r); import attn_mi355x as am; am.lib(); "
            "import torch_compare as tc; r = tc.hip_runtimes_mapped(); print(len(r), r)"
            % os.path.join(ROOT, "accelerated-final-project_amd"))
    r = _child(code)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.split()[0] == "1", r.stdout


def test_tuning_round_trip_and_plan_overrides(am, tuner):
    """atn_set_tuning_ex / atn_get_tuning_ex round trip; a forced plan is
    taken where it is possible, an impossible one falls back to the
    planner's choice; the reset restores the default plan."""
    default = am.fused_plan(0, 1, 4, 64, 64, 2048)
    assert default is not None and default["rows"] == 16
    tuner.set(fused_rows=32, fused_exchange="rsag", fused_xcd="device")
    t = am.get_tuning()
    assert (t.fused_rows, t.fused_exchange, t.fused_xcd) == (32, 2, 2)
    p = am.fused_plan(0, 1, 4, 64, 64, 2048)
    assert (p["rows"], p["gather1"], p["xcd"]) == (32, 0, 0)
    tuner.set(fused_rows=48)  # 48-row groups only for a padded head of 33-48 rows
    assert am.fused_plan(0, 1, 4, 64, 64, 2048)["rows"] in (16, 32, 64)
    tuner.clear()
    assert am.fused_plan(0, 1, 4, 64, 64, 2048) == default
    tuner.set(no_fused=True)
    assert am.fused_plan(0, 1, 4, 64, 64, 2048) is None
    assert am.path(0, 1, 4, 64, 64, 2048) == am.ATN_PATH_SPLIT_D
    tuner.set(flash_form="4x32")
    assert am.get_tuning().flash_form == 3
    with pytest.raises(KeyError):
        am.set_tuning(flash_form="6x16")


@pytest.mark.parametrize("cus,xccs", [(32, 1), (64, 2), (128, 4), (256, 4), (252, 8), (256, 8)])
def test_xcd_local_plans_need_the_whole_chip(am, tuner, cus, xccs):
    """Exchanges inside one XCD's L2 assume 8 XCDs dealt workgroup ids round
    robin; a partitioned MI355X (a device of 1, 2 or 4 XCDs) or a CU count
    not divisible by 8 gets device-scope plans only, also when such a plan
    is forced."""
    tuner.set(model_cus=cus, model_xccs=xccs)
    whole = cus % 8 == 0 and xccs == 8
    for shape in [(1, 4, 64, 64, 2048), (1, 4, 64, 64, 512), (1, 8, 32, 64, 1024),
                  (1, 1, 16, 16, 8192)]:
        p = am.fused_plan(0, *shape)
        assert p is not None, shape
        assert p["workgroups"] <= cus * 8
        if not whole:
            assert p["xcd"] == 0, (shape, p)
    tuner.set(fused_xcd="xcd")
    p = am.fused_plan(0, 1, 4, 64, 64, 2048)
    assert p["xcd"] == (1 if whole else 0)


def test_library_reads_no_environment(am):
    """Tuning is an API call, never an environment variable: a child process
    with the former override variables set plans exactly as without them."""
    code = ("import attn_mi355x as am; p = am.fused_plan(0, 1, 4, 64, 64, 2048); "
            "print(p['rows'], p['dc'], p['gather1'], p['xcd'], "
            "am.path(0, 1, 4, 64, 64, 2048), am.workspace_bytes(1, 1, 64, 8192, 8192, 128))")
    plain = _child(code)
    assert plain.returncode == 0, plain.stderr[-2000:]
    env_code = ("import os; os.environ.update(ATN_FUSED_ROWS='64', ATN_FUSED_DC='512', "
                "ATN_FUSED_EXCHANGE='rsag', ATN_FUSED_XCD='0', ATN_F32_FULL='1', "
                "ATN_WORKSPACE_CAP_MIB='1', ATN_FUSED_PRESET_STATUS='1'); " + code)
    forced = _child(env_code)
    assert forced.returncode == 0, forced.stderr[-2000:]
    assert forced.stdout == plain.stdout
    src = open(os.path.join(ROOT, "accelerated-final-project_amd", "csrc", "host",
                            "attn_api.cpp")).read()
    assert "getenv" not in src


def test_rerun_counter_starts_at_zero(am):
    assert am.rerun_count() == 0
    assert am.rerun_count(reset=True) == 0
