"""Python binding of libattn_mi355x.so (the C ABI in include/attn_mi355x.h).

This is a thin ctypes layer for tests, the benchmark and Python callers.
Device memory, streams and events come from hip_rt (ctypes over the same
libamdhip64.so.7 the library links); the compute is the library's HIP
kernels.  There is no fallback: if the shared library is missing, lib()
raises.

Drop-in functions keep the reference names and argument order
(e.g. attention_forward_optimized(Q, K, V, out, batch_sz, num_heads, len_q,
len_k, head_d), final/attention.cu:195-205) and take hip_rt.DeviceArray
objects in place of raw device pointers; like the reference they
synchronize and terminate the process on a HIP error, so the wrappers here
check shapes and dtypes first and raise ValueError instead.
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

_PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(_PKG)
LIB_PATH = os.path.join(_PKG, "lib", "libattn_mi355x.so")
HEADER_PATH = os.path.join(ROOT, "include", "attn_mi355x.h")

# status codes (include/attn_mi355x.h)
ATN_OK = 0
ATN_ERR_NULL_POINTER = -1
ATN_ERR_BAD_DIMENSION = -2
ATN_ERR_BAD_ROTARY = -3
ATN_ERR_SIZE_OVERFLOW = -4
ATN_ERR_ALIASING = -5
ATN_ERR_NO_DEVICE = -6
ATN_ERR_HIP = -7
ATN_ERR_WORKSPACE = -8
ATN_ERR_BAD_ARGUMENT = -9
ATN_ERR_MISALIGNED = -10
ATN_ERR_DEVICE_TIMEOUT = -11
ATN_ERR_CAPTURE = -12
ATN_ERR_SCRATCH_LIMIT = -13
ATN_ERR_NOT_PREPARED = -14

ATN_DTYPE_F32 = 0
ATN_DTYPE_BF16 = 1
ATN_PE_NONE = 0
ATN_PE_ROPE = 1
ATN_PE_SINUSOIDAL = 2
ATN_ROPE_INTERLEAVED = 0
ATN_ROPE_HALF = 1
ATN_PATH_FUSED_SMALL = 1
ATN_PATH_SPLIT_D = 2
ATN_PATH_GEMM = 3
ATN_PATH_FLASH = 4


class PeDesc(ctypes.Structure):
    """atn_pe_desc."""
    _fields_ = [
        ("kind", ctypes.c_int),
        ("pairing", ctypes.c_int),
        ("rotary_dim", ctypes.c_int),
        ("apply_q", ctypes.c_int),
        ("apply_k", ctypes.c_int),
        ("base", ctypes.c_float),
        ("table_a", ctypes.c_void_p),
        ("table_b", ctypes.c_void_p),
    ]


class Tuning(ctypes.Structure):
    """atn_tuning (process-wide overrides for measurement and tests)."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "fused_rows", "fused_dc", "fused_exchange", "fused_xcd", "no_fused", "no_flash",
        "gemm_fused_k",
        "workspace_cap_mib", "model_cus", "model_xccs", "preset_status", "flash_form",
        "splitd_tile", "flash_split")]


class FusedPlanInfo(ctypes.Structure):
    """atn_fused_plan_info."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "rows", "dc", "nchunk", "gather1", "xcd", "workgroups", "lds")]


class AtnError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        hip = lib().atn_last_hip_error() if status in (ATN_ERR_HIP, ATN_ERR_NO_DEVICE) else 0
        msg = f"{where}: status {status} ({status_string(status)})"
        if hip:
            msg += f", hip error {hip}"
        super().__init__(msg)


def build(jobs: int = 8) -> None:
    """Compile lib/libattn_mi355x.so for gfx950 (always recompiles)."""
    subprocess.run(["make", "-s", "-B", "-C", _PKG, f"-j{jobs}"], check=True)


_lib = None
_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float

_SIGS = {
    "atn_status_string": ([_i], ctypes.c_char_p),
    "atn_last_hip_error": ([], _i),
    "atn_device_count": ([], _i),
    "atn_attention_fwd_ex": ([_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                              ctypes.POINTER(PeDesc), _vp, ctypes.c_size_t, _vp], _i),
    "atn_attention_fwd_noalloc_ex": ([_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                      ctypes.POINTER(PeDesc), _vp], _i),
    "atn_attention_workspace_bytes": ([_i, _i, _i, _i, _i, _i, ctypes.POINTER(PeDesc)],
                                      ctypes.c_size_t),
    "atn_pe_apply_ex": ([_i, _vp, _vp, ctypes.c_long, _i, _i, ctypes.POINTER(PeDesc), _vp], _i),
    "atn_prepare_pe_ex": ([ctypes.POINTER(PeDesc), _i, _i], _i),
    "atn_sync_status_ex": ([_vp, _i, _i, _vp], _i),
    "atn_attention_path_ex": ([_i] * 6 + [ctypes.POINTER(PeDesc)], _i),
    "atn_set_tuning_ex": ([ctypes.POINTER(Tuning)], _i),
    "atn_get_tuning_ex": ([ctypes.POINTER(Tuning)], _i),
    "atn_fused_plan_ex": ([_i] * 6 + [ctypes.POINTER(PeDesc), ctypes.POINTER(FusedPlanInfo)],
                          _i),
    "atn_rerun_count": ([_i], ctypes.c_long),
    "atn_retained_bytes_ex": ([], ctypes.c_size_t),
    "atn_release_ex": ([], _i),
    "attention_forward_optimized": ([_vp] * 4 + [_i] * 5, None),
    "attention_forward": ([_vp] * 4 + [_i] * 5, None),
    "attention_forward_rope_fused": ([_vp] * 6 + [_i] * 5, None),
    "attention_forward_rope_fused_v7_hybrid": ([_vp] * 4 + [_i] * 6, None),
    "attention_forward_separate_rope": ([_vp] * 8 + [_i] * 6, None),
    "rope_forward": ([_vp] * 4 + [_i] * 4, None),
    "apply_sinusoidal_embeddings": ([_vp] * 4 + [_i] * 3, None),
    "attention_forward_sinusoidal_fused": ([_vp] * 4 + [_i] * 5, None),
    "attention_forward_sinusoidal_hybrid": ([_vp] * 7 + [_i] * 5, None),
    "attention_forward_sinusoidal_separate": ([_vp] * 8 + [_i] * 5, None),
    "attention_forward_bf16": ([_vp] * 4 + [_i] * 5, None),
    "attention_forward_rope_bf16": ([_vp] * 4 + [_i] * 6, None),
    "attention_forward_rope_fused_bf16": ([_vp] * 4 + [_i] * 5, None),
    "attention_forward_sinusoidal_bf16": ([_vp] * 4 + [_i] * 5, None),
    "precompute_rope_cache": ([_vp, _vp, _i, _i, _f], None),
    "precompute_sinusoidal_table": ([_vp, _vp, _i, _i], None),
}


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                               "(the HIP library has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def status_string(status: int) -> str:
    return lib().atn_status_string(status).decode()


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of every function declared in include/attn_mi355x.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return [n for n in names if n not in ("defined",)]


def device_count() -> int:
    return lib().atn_device_count()


# ---------------------------------------------------------------- tuning
_EXCHANGE = {None: 0, "gather": 1, "rsag": 2}
_SCOPE = {None: 0, "xcd": 1, "device": 2}
_FUSED_K = {None: 0, "on": 1, "off": 2}


_FLASH_FORM = {None: 0, "4x16": 1, "8x16": 2, "4x32": 3, "8x32": 4}


def set_tuning(fused_rows: int = 0, fused_dc: int = 0, fused_exchange: str | None = None,
               fused_xcd: str | None = None, no_fused: bool = False, no_flash: bool = False,
               gemm_fused_k: str | None = None, workspace_cap_mib: int = 0, model_cus: int = 0,
               model_xccs: int = 0, preset_status: bool = False, flash_form: str | None = None,
               splitd_tile: int = 0, flash_split: int = 0) -> None:
    """atn_set_tuning_ex with named fields (every field not given is reset).
    flash_form: "4x16", "8x16", "4x32" or "8x32" (waves x query rows per
    wave); flash_split: 1 never split the flash kernel's keys, n >= 2 into
    n parts."""
    t = Tuning(fused_rows, fused_dc, _EXCHANGE[fused_exchange], _SCOPE[fused_xcd],
               int(no_fused), int(no_flash), _FUSED_K[gemm_fused_k], workspace_cap_mib,
               model_cus, model_xccs, int(preset_status), _FLASH_FORM[flash_form], splitd_tile,
               flash_split)
    st = lib().atn_set_tuning_ex(ctypes.byref(t))
    if st != ATN_OK:
        raise AtnError(st, "atn_set_tuning_ex")


def get_tuning() -> Tuning:
    t = Tuning()
    lib().atn_get_tuning_ex(ctypes.byref(t))
    return t


class tuning:
    """Context manager: overrides for the block, the previous ones restored
    after it (``with tuning(fused_rows=16): ...``)."""

    def __init__(self, **kw):
        self.kw = kw

    def __enter__(self):
        self.saved = get_tuning()
        set_tuning(**self.kw)
        return self

    def __exit__(self, *exc):
        lib().atn_set_tuning_ex(ctypes.byref(self.saved))
        return False


def fused_plan(dtype_code: int, B, H, Lq, Lk, D, pe: PeDesc | None = None) -> dict | None:
    """The single-launch kernel's plan for the shape (None when the shape
    does not run on it)."""
    info = FusedPlanInfo()
    r = lib().atn_fused_plan_ex(dtype_code, B, H, Lq, Lk, D,
                                ctypes.byref(pe) if pe is not None else None,
                                ctypes.byref(info))
    if r < 0:
        raise AtnError(r, "atn_fused_plan_ex")
    if r == 0:
        return None
    return {n: getattr(info, n) for n, _ in FusedPlanInfo._fields_}


def rerun_count(reset: bool = False) -> int:
    return lib().atn_rerun_count(int(reset))


def retained_bytes() -> int:
    return lib().atn_retained_bytes_ex()


def release() -> None:
    st = lib().atn_release_ex()
    if st != ATN_OK:
        raise AtnError(st, "atn_release_ex")


# ---------------------------------------------------------------- array helpers
# Arguments are hip_rt.DeviceArray objects ([B,H,L,D], 'f32' or 'bf16').
def _ptr(t):
    return None if t is None else t.ptr


def _check(t, dtype, shape, name):
    from hip_rt import DeviceArray
    if not isinstance(t, DeviceArray):
        raise ValueError(f"{name} must be a hip_rt.DeviceArray")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def _dtype_code(t) -> int:
    if t.dtype == "f32":
        return ATN_DTYPE_F32
    if t.dtype == "bf16":
        return ATN_DTYPE_BF16
    raise ValueError(f"unsupported dtype {t.dtype}")


def _stream_handle(stream) -> int | None:
    return None if stream is None else stream.handle


def make_pe(kind: str = "none", pairing: str = "interleaved", rotary_dim: int = 0,
            apply_q: bool = True, apply_k: bool = True, base: float = 10000.0,
            table_a=None, table_b=None) -> PeDesc | None:
    """Build an atn_pe_desc.  kind: none | rope | sinusoidal; tables are
    device arrays in the reference's layouts, or None for library tables."""
    if kind == "none":
        return None
    d = PeDesc()
    d.kind = {"rope": ATN_PE_ROPE, "sinusoidal": ATN_PE_SINUSOIDAL}[kind]
    d.pairing = {"interleaved": ATN_ROPE_INTERLEAVED, "half": ATN_ROPE_HALF}[pairing]
    d.rotary_dim = rotary_dim
    d.apply_q = int(apply_q)
    d.apply_k = int(apply_k)
    d.base = base
    d.table_a = _ptr(table_a)
    d.table_b = _ptr(table_b)
    return d


def attention_ex(Q, K, V, out=None, pe: PeDesc | None = None, workspace=None, stream=None):
    """atn_attention_fwd_ex on device arrays [B,H,L,D]; asynchronous on
    `stream` (hip_rt.Stream or None = null stream).  Raises AtnError."""
    from hip_rt import DeviceArray
    B, H, Lq, D = Q.shape
    Lk = K.shape[2]
    _check(Q, Q.dtype, (B, H, Lq, D), "Q")
    _check(K, Q.dtype, (B, H, Lk, D), "K")
    _check(V, Q.dtype, (B, H, Lk, D), "V")
    if out is None:
        out = DeviceArray(Q.shape, Q.dtype)
    _check(out, Q.dtype, (B, H, Lq, D), "out")
    ws_ptr, ws_bytes = (None, 0)
    if workspace is not None:
        ws_ptr, ws_bytes = workspace.ptr, workspace.nbytes
    st = lib().atn_attention_fwd_ex(_dtype_code(Q), _ptr(Q), _ptr(K), _ptr(V), _ptr(out), B, H,
                                    Lq, Lk, D, ctypes.byref(pe) if pe is not None else None,
                                    ws_ptr, ws_bytes, _stream_handle(stream))
    if st != ATN_OK:
        raise AtnError(st, "atn_attention_fwd_ex")
    return out


def attention_noalloc_ex(Q, K, V, out=None, pe: PeDesc | None = None, stream=None):
    """atn_attention_fwd_noalloc_ex (scratch in the library's per-device
    static array, no allocation); raises AtnError."""
    from hip_rt import DeviceArray
    B, H, Lq, D = Q.shape
    Lk = K.shape[2]
    _check(Q, Q.dtype, (B, H, Lq, D), "Q")
    _check(K, Q.dtype, (B, H, Lk, D), "K")
    _check(V, Q.dtype, (B, H, Lk, D), "V")
    if out is None:
        out = DeviceArray(Q.shape, Q.dtype)
    _check(out, Q.dtype, (B, H, Lq, D), "out")
    st = lib().atn_attention_fwd_noalloc_ex(_dtype_code(Q), _ptr(Q), _ptr(K), _ptr(V), _ptr(out),
                                            B, H, Lq, Lk, D,
                                            ctypes.byref(pe) if pe is not None else None,
                                            _stream_handle(stream))
    if st != ATN_OK:
        raise AtnError(st, "atn_attention_fwd_noalloc_ex")
    return out


def path(dtype_code: int, B, H, Lq, Lk, D, pe: PeDesc | None = None) -> int:
    """ATN_PATH_* that atn_attention_fwd_ex takes for this shape."""
    return lib().atn_attention_path_ex(dtype_code, B, H, Lq, Lk, D,
                                       ctypes.byref(pe) if pe is not None else None)


def sync_status(workspace=None, B: int = 1, H: int = 1, stream=None) -> int:
    """atn_sync_status_ex: ATN_OK or ATN_ERR_DEVICE_TIMEOUT."""
    return lib().atn_sync_status_ex(None if workspace is None else workspace.ptr, B, H,
                                    _stream_handle(stream))


def workspace_bytes(dtype_code: int, B, H, Lq, Lk, D, pe: PeDesc | None = None) -> int:
    return lib().atn_attention_workspace_bytes(dtype_code, B, H, Lq, Lk, D,
                                               ctypes.byref(pe) if pe is not None else None)


def pe_apply_ex(x, out, seq_len: int, pe: PeDesc, stream=None):
    """atn_pe_apply_ex over the rows of x ([..., D]); position = row % seq_len."""
    D = x.shape[-1]
    n_rows = x.size // D
    st = lib().atn_pe_apply_ex(_dtype_code(x), _ptr(x), _ptr(out), n_rows, seq_len, D,
                               ctypes.byref(pe), _stream_handle(stream))
    if st != ATN_OK:
        raise AtnError(st, "atn_pe_apply_ex")
    return out


def _dropin_check(dtype, Q, K, V, out):
    B, H, Lq, D = Q.shape
    Lk = K.shape[2]
    _check(Q, dtype, (B, H, Lq, D), "Q")
    _check(K, dtype, (B, H, Lk, D), "K")
    _check(V, dtype, (B, H, Lk, D), "V")
    _check(out, dtype, (B, H, Lq, D), "out")
    return B, H, Lq, Lk, D


def _rot_check(rotary_dim, D):
    if rotary_dim < 2 or rotary_dim > D or rotary_dim % 2:
        raise ValueError("rotary_dim must be even and in [2, head_d]")


def attention_forward_optimized(Q, K, V, out):
    B, H, Lq, Lk, D = _dropin_check("f32", Q, K, V, out)
    lib().attention_forward_optimized(Q.ptr, K.ptr, V.ptr, out.ptr, B, H, Lq, Lk, D)
    return out


def attention_forward(Q, K, V, out):
    B, H, Lq, Lk, D = _dropin_check("f32", Q, K, V, out)
    lib().attention_forward(Q.ptr, K.ptr, V.ptr, out.ptr, B, H, Lq, Lk, D)
    return out


def attention_forward_rope_fused(Q, K, V, out, cos_cache, sin_cache):
    B, H, Lq, Lk, D = _dropin_check("f32", Q, K, V, out)
    for n, t in (("cos_cache", cos_cache), ("sin_cache", sin_cache)):
        if t.shape[-1] != D or t.size < max(Lq, Lk) * D:
            raise ValueError(f"{n} must be [>= max(len_q, len_k)][head_d]")
    lib().attention_forward_rope_fused(Q.ptr, K.ptr, V.ptr, out.ptr, cos_cache.ptr, sin_cache.ptr,
                                       B, H, Lq, Lk, D)
    return out


def attention_forward_rope_fused_v7_hybrid(Q, K_rotated, V, out, rotary_dim: int):
    B, H, Lq, Lk, D = _dropin_check("f32", Q, K_rotated, V, out)
    _rot_check(rotary_dim, D)
    lib().attention_forward_rope_fused_v7_hybrid(Q.ptr, K_rotated.ptr, V.ptr, out.ptr, B, H, Lq,
                                                 Lk, D, rotary_dim)
    return out


def attention_forward_separate_rope(Q, K, V, Q_rope, K_rope, out, cos_cache, sin_cache,
                                    rotary_dim: int):
    B, H, Lq, Lk, D = _dropin_check("f32", Q, K, V, out)
    _check(Q_rope, "f32", Q.shape, "Q_rope")
    _check(K_rope, "f32", K.shape, "K_rope")
    _rot_check(rotary_dim, D)
    lib().attention_forward_separate_rope(Q.ptr, K.ptr, V.ptr, Q_rope.ptr, K_rope.ptr, out.ptr,
                                          cos_cache.ptr, sin_cache.ptr, B, H, Lq, Lk, D,
                                          rotary_dim)
    return out


def rope_forward(x, out, cos_cache, sin_cache, rotary_dim: int, seq_len: int):
    D = x.shape[-1]
    _rot_check(rotary_dim, D)
    lib().rope_forward(x.ptr, out.ptr, cos_cache.ptr, sin_cache.ptr, x.size // D, D, rotary_dim,
                       seq_len)
    return out


def apply_sinusoidal_embeddings(x, sin_table, cos_table, out, seqlen: int):
    D = x.shape[-1]
    lib().apply_sinusoidal_embeddings(x.ptr, sin_table.ptr, cos_table.ptr, out.ptr, x.size // D,
                                      D, seqlen)
    return out


def attention_forward_sinusoidal_fused(Q, K, V, out):
    B, H, Lq, Lk, D = _dropin_check("f32", Q, K, V, out)
    lib().attention_forward_sinusoidal_fused(Q.ptr, K.ptr, V.ptr, out.ptr, B, H, Lq, Lk, D)
    return out


def attention_forward_sinusoidal_hybrid(Q, K, V, sin_table, cos_table, K_emb, out):
    B, H, Lq, Lk, D = _dropin_check("f32", Q, K, V, out)
    _check(K_emb, "f32", K.shape, "K_emb")
    lib().attention_forward_sinusoidal_hybrid(Q.ptr, K.ptr, V.ptr, sin_table.ptr, cos_table.ptr,
                                              K_emb.ptr, out.ptr, B, H, Lq, Lk, D)
    return out


def attention_forward_sinusoidal_separate(Q, K, V, sin_table, cos_table, Q_emb, K_emb, out):
    B, H, Lq, Lk, D = _dropin_check("f32", Q, K, V, out)
    _check(Q_emb, "f32", Q.shape, "Q_emb")
    _check(K_emb, "f32", K.shape, "K_emb")
    lib().attention_forward_sinusoidal_separate(Q.ptr, K.ptr, V.ptr, sin_table.ptr, cos_table.ptr,
                                                Q_emb.ptr, K_emb.ptr, out.ptr, B, H, Lq, Lk, D)
    return out


def attention_forward_bf16(Q, K, V, out):
    B, H, Lq, Lk, D = _dropin_check("bf16", Q, K, V, out)
    lib().attention_forward_bf16(Q.ptr, K.ptr, V.ptr, out.ptr, B, H, Lq, Lk, D)
    return out


def attention_forward_rope_bf16(Q, K_rotated, V, out, rotary_dim: int):
    B, H, Lq, Lk, D = _dropin_check("bf16", Q, K_rotated, V, out)
    _rot_check(rotary_dim, D)
    lib().attention_forward_rope_bf16(Q.ptr, K_rotated.ptr, V.ptr, out.ptr, B, H, Lq, Lk, D,
                                      rotary_dim)
    return out


def attention_forward_rope_fused_bf16(Q, K, V, out):
    B, H, Lq, Lk, D = _dropin_check("bf16", Q, K, V, out)
    if D % 2:
        raise ValueError("head_d must be even for RoPE")
    lib().attention_forward_rope_fused_bf16(Q.ptr, K.ptr, V.ptr, out.ptr, B, H, Lq, Lk, D)
    return out


def attention_forward_sinusoidal_bf16(Q, K, V, out):
    B, H, Lq, Lk, D = _dropin_check("bf16", Q, K, V, out)
    lib().attention_forward_sinusoidal_bf16(Q.ptr, K.ptr, V.ptr, out.ptr, B, H, Lq, Lk, D)
    return out


def precompute_rope_cache(max_seq_len: int, rotary_dim: int, base: float = 10000.0):
    """Host cos/sin caches [pos][rotary_dim] (final/rope.cu:20-40) as numpy."""
    import numpy as np
    c = np.zeros((max_seq_len, rotary_dim), dtype=np.float32)
    s = np.zeros((max_seq_len, rotary_dim), dtype=np.float32)
    lib().precompute_rope_cache(c.ctypes.data, s.ctypes.data, max_seq_len, rotary_dim, base)
    return c, s


def precompute_sinusoidal_table(seqlen: int, hdim: int):
    """Host sin/cos tables [pos][hdim] (final/sinusoidal.cu:838-855) as numpy."""
    import numpy as np
    s = np.zeros((seqlen, hdim), dtype=np.float32)
    c = np.zeros((seqlen, hdim), dtype=np.float32)
    lib().precompute_sinusoidal_table(s.ctypes.data, c.ctypes.data, seqlen, hdim)
    return s, c
