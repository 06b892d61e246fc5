"""TEST INFRASTRUCTURE: ctypes binding of the double-precision C oracle.

``attnres_oracle.c`` restates the reference's forward (reference.py:130-133),
closed-form backward (triton_op.py:205-214), ``attn_with_stats``/merge
(reference.py:195-233) and the batched contract (triton_op.py:438-462) with
plain loops, plus the gradients of attn_with_stats, of the merge and of the
batched operator, which the reference does not have (derived in the C file). Arrays are numpy float64, layout ``v [N, T, D]`` with ``T`` the
flattened token count. Build with ``make -C oracle``.
"""

from __future__ import annotations

import ctypes
import pathlib

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle_attnres.so"
_lib = None

_dp = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.c_int64


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            raise FileNotFoundError(f"{_LIB_PATH} is missing; build it with `make -C oracle`")
        so = ctypes.CDLL(str(_LIB_PATH))
        so.oracle_forward.argtypes = [_dp, _dp, _dp, _dp, _i64, _i64, _i64, ctypes.c_double]
        so.oracle_backward.argtypes = [_dp, _dp, _dp, _dp, _dp, _i64, _i64, _i64, ctypes.c_double]
        so.oracle_attn_with_stats.argtypes = [_dp, _dp, _dp, _dp, _dp, _i64, _i64, _i64, ctypes.c_double]
        so.oracle_merge.argtypes = [_dp] * 9 + [_i64, _i64]
        so.oracle_batched.argtypes = [_dp, _dp, _dp, _i64, _i64, _i64, _i64, ctypes.c_double]
        so.oracle_attn_with_stats_backward.argtypes = [_dp] * 7 + [_i64, _i64, _i64, ctypes.c_double]
        so.oracle_merge_backward.argtypes = [_dp] * 15 + [_i64, _i64]
        so.oracle_batched_backward.argtypes = [_dp] * 5 + [_i64] * 4 + [ctypes.c_double]
        for f in (so.oracle_forward, so.oracle_backward, so.oracle_attn_with_stats, so.oracle_batched,
                  so.oracle_attn_with_stats_backward, so.oracle_batched_backward):
            f.restype = ctypes.c_int
        so.oracle_merge.restype = None
        so.oracle_merge_backward.restype = None
        _lib = so
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.float64 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_dp)


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def forward(v, w, eps: float = 1e-6, return_alpha: bool = False):
    """``v [N, T, D]``, ``w [D]`` -> ``out [T, D]`` (and ``alpha [N, T]``)."""
    v, w = _f64(v), _f64(w)
    n, t, d = v.shape
    out = np.empty((t, d))
    alpha = np.empty((n, t)) if return_alpha else None
    rc = lib().oracle_forward(_p(v), _p(w), _p(out), _p(alpha) if alpha is not None else None, n, t, d, eps)
    if rc:
        raise ValueError(f"oracle_forward rejected the shape (rc={rc})")
    return (out, alpha) if return_alpha else out


def backward(v, w, g, eps: float = 1e-6):
    """Closed-form ``(dv [N, T, D], dw [D])`` for upstream gradient ``g [T, D]``."""
    v, w, g = _f64(v), _f64(w), _f64(g)
    n, t, d = v.shape
    dv = np.empty_like(v)
    dw = np.empty(d)
    rc = lib().oracle_backward(_p(v), _p(w), _p(g), _p(dv), _p(dw), n, t, d, eps)
    if rc:
        raise ValueError(f"oracle_backward rejected the shape (rc={rc})")
    return dv, dw


def attn_with_stats(v, w, eps: float = 1e-6):
    v, w = _f64(v), _f64(w)
    n, t, d = v.shape
    o, m, ell = np.empty((t, d)), np.empty(t), np.empty(t)
    rc = lib().oracle_attn_with_stats(_p(v), _p(w), _p(o), _p(m), _p(ell), n, t, d, eps)
    if rc:
        raise ValueError(f"oracle_attn_with_stats rejected the shape (rc={rc})")
    return o, m, ell


def merge(o1, m1, l1, o2, m2, l2):
    o1, m1, l1, o2, m2, l2 = map(_f64, (o1, m1, l1, o2, m2, l2))
    t, d = o1.shape
    o, m, ell = np.empty((t, d)), np.empty(t), np.empty(t)
    lib().oracle_merge(_p(o1), _p(m1), _p(l1), _p(o2), _p(m2), _p(l2), _p(o), _p(m), _p(ell), t, d)
    return o, m, ell


def batched(v, q, eps: float = 1e-6):
    """``v [N, T, D]``, ``q [S, D]`` -> ``[S, T, D]``."""
    v, q = _f64(v), _f64(q)
    n, t, d = v.shape
    s = q.shape[0]
    out = np.empty((s, t, d))
    rc = lib().oracle_batched(_p(v), _p(q), _p(out), n, s, t, d, eps)
    if rc:
        raise ValueError(f"oracle_batched rejected the shape (rc={rc})")
    return out


def attn_with_stats_backward(v, w, go, gm, gl, eps: float = 1e-6):
    """Gradient of ``attn_with_stats`` for upstream ``(go [T, D], gm [T], gl [T])``."""
    v, w, go, gm, gl = map(_f64, (v, w, go, gm, gl))
    n, t, d = v.shape
    dv, dw = np.empty_like(v), np.empty(d)
    rc = lib().oracle_attn_with_stats_backward(_p(v), _p(w), _p(go), _p(gm), _p(gl), _p(dv), _p(dw),
                                               n, t, d, eps)
    if rc:
        raise ValueError(f"oracle_attn_with_stats_backward rejected the shape (rc={rc})")
    return dv, dw


def merge_backward(o1, m1, l1, o2, m2, l2, go, gm, gl):
    """Gradient of ``merge`` for upstream ``(go, gm, gl)``: six arrays."""
    o1, m1, l1, o2, m2, l2, go, gm, gl = map(_f64, (o1, m1, l1, o2, m2, l2, go, gm, gl))
    t, d = o1.shape
    do1, do2 = np.empty((t, d)), np.empty((t, d))
    dm1, dl1, dm2, dl2 = (np.empty(t) for _ in range(4))
    lib().oracle_merge_backward(_p(o1), _p(m1), _p(l1), _p(o2), _p(m2), _p(l2), _p(go), _p(gm),
                                _p(gl), _p(do1), _p(dm1), _p(dl1), _p(do2), _p(dm2), _p(dl2), t, d)
    return do1, dm1, dl1, do2, dm2, dl2


def batched_backward(v, q, g, eps: float = 1e-6):
    """``v [N, T, D]``, ``q [S, D]``, ``g [S, T, D]`` -> ``(dv [N, T, D], dq [S, D])``."""
    v, q, g = _f64(v), _f64(q), _f64(g)
    n, t, d = v.shape
    s = q.shape[0]
    dv, dq = np.empty_like(v), np.empty((s, d))
    rc = lib().oracle_batched_backward(_p(v), _p(q), _p(g), _p(dv), _p(dq), n, s, t, d, eps)
    if rc:
        raise ValueError(f"oracle_batched_backward rejected the shape (rc={rc})")
    return dv, dq
