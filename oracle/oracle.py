"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker.  The product library never calls it.

Every function takes and returns contiguous numpy float32 arrays laid out
[B][H][L][D], like the reference's host buffers (final/attention.cu:342-353).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i = ctypes.c_int
_l = ctypes.c_long


def build() -> None:
    """Compile liboracle.so with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_attention_rows.argtypes = [_f32p] * 4 + [_i] * 5 + [_l, _l, _i]
        L.oracle_attention_rope_rows.argtypes = [_f32p] * 6 + [_i] * 9 + [_l, _l, _i]
        L.oracle_attention_sinusoidal_rows.argtypes = [_f32p] * 6 + [_i] * 7 + [_l, _l, _i]
        L.oracle_rope_cache.argtypes = [_f32p, _f32p, _i, _i, ctypes.c_float]
        L.oracle_rope_freqs.argtypes = [_f32p, _i, ctypes.c_float]
        L.oracle_sinusoidal_freqs.argtypes = [_f32p, _i]
        L.oracle_apply_rope_interleaved.argtypes = [_f32p] * 4 + [_i] * 4
        L.oracle_apply_rope_half.argtypes = [_f32p] * 4 + [_i] * 4
        L.oracle_sinusoidal_table.argtypes = [_f32p, _f32p, _i, _i]
        L.oracle_add_sinusoidal.argtypes = [_f32p] * 4 + [_i] * 3
        L.oracle_f32_to_bf16.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.oracle_bf16_to_f32.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.oracle_set_mutation.argtypes = [_i]
        L.oracle_get_mutation.restype = _i
        L.oracle_openmp_enabled.restype = _i
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def set_mutation(m: int) -> None:
    """Plant a known mistake in the oracle (tests that prove checks can fail)."""
    lib().oracle_set_mutation(int(m))


def attention(Q, K, V, rows=None, nthreads: int = 1) -> np.ndarray:
    """attention_cpu (final/attention.cu:228-283).  Q: [B,H,Lq,D], K/V: [B,H,Lk,D].

    rows: optional (begin, end) over the flattened (b*H+h)*Lq+i row index;
    rows outside the range are left as NaN.
    """
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    B, H, Lq, D = Q.shape
    Lk = K.shape[2]
    out = np.full(Q.shape, np.nan, dtype=np.float32)
    r0, r1 = rows if rows is not None else (0, B * H * Lq)
    lib().oracle_attention_rows(_p(Q), _p(K), _p(V), _p(out), B, H, Lq, Lk, D, r0, r1, nthreads)
    return out


def rope_cache(max_seq_len: int, rotary_dim: int, base: float = 10000.0):
    """precompute_rope_cache (final/rope.cu:20-40) -> (cos, sin), [pos][rotary_dim]."""
    c = np.zeros((max_seq_len, rotary_dim), dtype=np.float32)
    s = np.zeros((max_seq_len, rotary_dim), dtype=np.float32)
    lib().oracle_rope_cache(_p(c), _p(s), max_seq_len, rotary_dim, base)
    return c, s


def rope_freqs(rotary_dim: int, base: float = 10000.0) -> np.ndarray:
    f = np.zeros(rotary_dim // 2, dtype=np.float32)
    lib().oracle_rope_freqs(_p(f), rotary_dim, base)
    return f


def sinusoidal_freqs(hdim: int) -> np.ndarray:
    f = np.zeros(hdim, dtype=np.float32)
    lib().oracle_sinusoidal_freqs(_p(f), hdim)
    return f


def apply_rope(X, cos_c, sin_c, rotary_dim=None, pairing: str = "interleaved", pos0: int = 0):
    """Rotate every row of X ([..., L, D]); row p of each [L, D] slab gets
    position pos0 + p.  Interleaved follows apply_rope_cpu (final/rope.cu:1418-1435)."""
    X = _f32(X)
    L, D = X.shape[-2], X.shape[-1]
    r = D if rotary_dim is None else rotary_dim
    cos_c, sin_c = _f32(cos_c), _f32(sin_c)
    out = np.empty_like(X)
    fn = lib().oracle_apply_rope_half if pairing == "half" else lib().oracle_apply_rope_interleaved
    flat_in = X.reshape(-1, L, D)
    flat_out = out.reshape(-1, L, D)
    for s in range(flat_in.shape[0]):
        xi = np.ascontiguousarray(flat_in[s])
        xo = np.empty_like(xi)
        fn(_p(xi), _p(xo), _p(cos_c), _p(sin_c), L, D, r, pos0)
        flat_out[s] = xo
    return out


def attention_rope(Q, K, V, cos_c, sin_c, rotary_dim=None, pairing: str = "interleaved",
                   rotate_q: bool = True, rotate_k: bool = True, rows=None, nthreads: int = 1):
    """attention_rope_cpu (final/rope.cu:1439-1499) with rotary width, pairing
    and per-side switches (v7 hybrid: rotate_k=False, K pre-rotated)."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    B, H, Lq, D = Q.shape
    Lk = K.shape[2]
    r = D if rotary_dim is None else rotary_dim
    cos_c, sin_c = _f32(cos_c), _f32(sin_c)
    out = np.full(Q.shape, np.nan, dtype=np.float32)
    r0, r1 = rows if rows is not None else (0, B * H * Lq)
    lib().oracle_attention_rope_rows(_p(Q), _p(K), _p(V), _p(out), _p(cos_c), _p(sin_c), B, H,
                                     Lq, Lk, D, r, 1 if pairing == "half" else 0, int(rotate_q),
                                     int(rotate_k), r0, r1, nthreads)
    return out


def sinusoidal_table(max_seq_len: int, hdim: int):
    """generate_sinusoidal_embeddings_cpu (final/sinusoidal.cu:838-855) -> (sin, cos)."""
    s = np.zeros((max_seq_len, hdim), dtype=np.float32)
    c = np.zeros((max_seq_len, hdim), dtype=np.float32)
    lib().oracle_sinusoidal_table(_p(s), _p(c), max_seq_len, hdim)
    return s, c


def add_sinusoidal(X, sin_t, cos_t, pos0: int = 0):
    X = _f32(X)
    L, D = X.shape[-2], X.shape[-1]
    out = np.empty_like(X)
    flat_in = X.reshape(-1, L, D)
    flat_out = out.reshape(-1, L, D)
    for s in range(flat_in.shape[0]):
        xi = np.ascontiguousarray(flat_in[s])
        xo = np.empty_like(xi)
        lib().oracle_add_sinusoidal(_p(xi), _p(xo), _p(_f32(sin_t)), _p(_f32(cos_t)), L, D, pos0)
        flat_out[s] = xo
    return out


def attention_sinusoidal(Q, K, V, sin_t, cos_t, add_q: bool = True, add_k: bool = True,
                         rows=None, nthreads: int = 1):
    """attention_sinusoidal_cpu (final/sinusoidal.cu:858-928)."""
    Q, K, V = _f32(Q), _f32(K), _f32(V)
    B, H, Lq, D = Q.shape
    Lk = K.shape[2]
    out = np.full(Q.shape, np.nan, dtype=np.float32)
    r0, r1 = rows if rows is not None else (0, B * H * Lq)
    lib().oracle_attention_sinusoidal_rows(_p(Q), _p(K), _p(V), _p(_f32(sin_t)), _p(_f32(cos_t)),
                                           _p(out), B, H, Lq, Lk, D, int(add_q), int(add_k), r0,
                                           r1, nthreads)
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(_p(x), out.ctypes.data_as(_u16p), x.size)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().oracle_bf16_to_f32(b.ctypes.data_as(_u16p), _p(out), b.size)
    return out


def check_results(gpu_out, cpu_out, abs_tol: float = 1e-3, rel_tol: float = 1e-2):
    """Tolerance semantics of check_results (final/attention.cu:296-331): an
    element fails iff abs_diff > abs_tol AND abs_diff/(|cpu|+1e-8) > rel_tol.
    Returns (n_errors, max_abs_diff, max_rel_diff)."""
    g = np.asarray(gpu_out, dtype=np.float32).ravel()
    c = np.asarray(cpu_out, dtype=np.float32).ravel()
    abs_diff = np.abs(g - c)
    rel_diff = abs_diff / (np.abs(c) + np.float32(1e-8))
    err = (abs_diff > abs_tol) & (rel_diff > rel_tol)
    nan = ~np.isfinite(g)
    return int(err.sum() + nan.sum()), float(np.nanmax(abs_diff)) if g.size else 0.0, \
        float(np.nanmax(rel_diff)) if g.size else 0.0
