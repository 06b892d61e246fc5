"""ctypes binding of ``libswitchyard_hip.so`` (the C ABI in include/switchyard.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already loaded (same ``libamdhip64.so.7`` soname): one runtime
per process. It is built in-tree by ``make -C blackwell-switchyard_amd/csrc``
(or ``__graft_entry__.build()``). There is no fallback: if the library is
missing every operator raises.
"""

from __future__ import annotations

import contextlib
import ctypes
import pathlib
import threading

import torch  # noqa: F401  -- must precede the load: provides the HIP runtime

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libswitchyard_hip.so"

SY_F32, SY_F16, SY_BF16 = 0, 1, 2
OP_FWD, OP_BWD, OP_BATCHED, OP_SOL, OP_BWD_BATCHED = 0, 1, 2, 3, 4
FAMILY_NAMES = {0: "resident", 1: "chunked", 2: "generic", 3: "per_query", 4: "matrix"}

_DTYPE_CODES = {torch.float32: SY_F32, torch.float16: SY_F16, torch.bfloat16: SY_BF16}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_vpp = ctypes.POINTER(ctypes.c_void_p)  # host array of device pointers

#: Largest source count of the pointer-table entry points (SY_MAX_TABLE_ROWS).
MAX_TABLE_ROWS = 16


class Plan(ctypes.Structure):
    """Mirror of ``sy_plan``."""

    _fields_ = [
        ("family", ctypes.c_int32),
        ("waves_per_token", ctypes.c_int32),
        ("chunks_per_lane", ctypes.c_int32),
        ("rows_per_tile", ctypes.c_int32),
        ("elems_per_chunk", ctypes.c_int32),
        ("block_threads", ctypes.c_int32),
        ("tokens_per_block", ctypes.c_int32),
        ("n_chunks", ctypes.c_int32),
    ]

    def as_dict(self) -> dict:
        d = {name: int(getattr(self, name)) for name, _ in self._fields_}
        d["family_name"] = FAMILY_NAMES.get(d["family"], "?")
        return d


class Tuning(ctypes.Structure):
    """Mirror of ``sy_tuning`` (measurement-only launch overrides)."""

    _fields_ = [
        ("fwd_tile", ctypes.c_int32 * 3),
        ("bwd_tile", ctypes.c_int32 * 3),
        ("batched_tile", ctypes.c_int32 * 3),
        ("sol_tile", ctypes.c_int32 * 3),
        ("bwd_blocks_per_cu", ctypes.c_int32),
        ("mx_slots", ctypes.c_int32),
        ("bmx_waves", ctypes.c_int32),
    ]


#: Every symbol include/switchyard.h declares, with (restype, argtypes).
SIGNATURES = {
    "sy_abi_version": (_i32, []),
    "sy_plan_for": (_i32, [_i32, _i64, _i64, _i64, _i32, _i32, _i32, ctypes.POINTER(Plan)]),
    "sy_plan_for_tokens": (_i32, [_i32, _i64, _i64, _i64, _i64, _i32, _i32, _i32, ctypes.POINTER(Plan)]),
    "sy_fwd": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, ctypes.c_float, _vp]),
    "sy_bwd_workspace_bytes": (_i64, [_i64, _i64, _i64, _i32, _i32]),
    "sy_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _i32,
                      ctypes.c_float, _vp]),
    "sy_bwd_partial_rows": (_i64, [_i64, _i64, _i64, _i32, _i32, _i32, _i32]),
    "sy_kernel_info": (_i32, [_i32, _i64, _i64, _i64, _i32, _i32, ctypes.POINTER(ctypes.c_int32)]),
    "sy_bwd_main": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _i32,
                           ctypes.c_float, _vp]),
    "sy_dw_reduce": (_i32, [_vp, _i64, _i64, _vp, _i32, _vp]),
    "sy_fwd_batched": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, ctypes.c_float, _vp]),
    "sy_sol": (_i32, [_vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp]),
    "sy_fwd_table": (_i32, [_vpp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, ctypes.c_float, _vp]),
    "sy_bwd_static": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32,
                             ctypes.c_float, _vp]),
    "sy_bwd_table": (_i32, [_vpp, _vp, _vp, _vp, _vpp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32,
                            ctypes.c_float, _vp]),
    "sy_fwd_batched_table": (_i32, [_vpp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, ctypes.c_float,
                                    _vp]),
    "sy_attn_with_stats": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32,
                                  ctypes.c_float, _vp]),
    "sy_attn_with_stats_bwd": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                      _i64, _i64, _i32, _i32, ctypes.c_float, _vp]),
    "sy_batched_with_stats": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32,
                                     ctypes.c_float, _vp]),
    "sy_attn_with_stats_merge": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                                        _i32, _i32, ctypes.c_float, _i32, _vp]),
    "sy_merge_stats": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp]),
    "sy_merge_stats_bwd": (_i32, [_vp] * 15 + [_i64, _i64, _i32, _vp]),
    "sy_bwd_batched_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64, _i32]),
    "sy_bwd_batched": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
                              ctypes.c_float, _vp]),
    "sy_bw_probe": (_i32, [_i32, _vp, _vp, _i64, _vp]),
    "sy_probe_grid": (_i64, [_i64]),
    "sy_tuning_set": (_i32, [ctypes.POINTER(Tuning)]),
    "sy_tuning_get": (_i32, [ctypes.POINTER(Tuning)]),
    "sy_strerror": (ctypes.c_char_p, [_i32]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library with typed entry points. Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"switchyard HIP library not found at {LIB_PATH}; build it with "
                    "`make -C blackwell-switchyard_amd/csrc` (there is no fallback path)"
                )
            so = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(so, name)
                fn.restype = res
                fn.argtypes = args
            _lib = so
    return _lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected bfloat16, float16 or float32") from None


def strerror(rc: int) -> str:
    return lib().sy_strerror(rc).decode()


def check(rc: int, what: str) -> None:
    """Raise RuntimeError for a nonzero C-ABI status."""
    if rc != 0:
        raise RuntimeError(f"{what} failed ({rc}): {strerror(rc)}")


def plan(op: int, n_src: int, d: int, dtype: torch.dtype, *, n_q: int = 0,
         w_dtype: torch.dtype | None = None, aligned: bool = True, n_tok: int | None = None) -> dict:
    """The execution plan the library picks for a shape (pure host arithmetic).
    With ``n_tok``, the tile a launch of that many tokens runs on the current
    device (``sy_plan_for_tokens``: the forward and backward also depend on
    the token count)."""
    p = Plan()
    if n_tok is None:
        rc = lib().sy_plan_for(op, n_src, n_q, d, dtype_code(dtype), dtype_code(w_dtype or dtype),
                               int(aligned), ctypes.byref(p))
    else:
        rc = lib().sy_plan_for_tokens(op, n_src, n_q, n_tok, d, dtype_code(dtype),
                                      dtype_code(w_dtype or dtype), int(aligned), ctypes.byref(p))
    check(rc, "sy_plan_for")
    return p.as_dict()


def pointer_table(tensors) -> ctypes.Array:
    """A host array of the tensors' device addresses, for the *_table entry points."""
    return (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])


def stream_ptr(device: torch.device) -> ctypes.c_void_p:
    """The HIP stream torch is currently issuing work on for ``device``."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


@contextlib.contextmanager
def tuning(**overrides):
    """Install measurement-only launch overrides (``sy_tuning_set``) for the
    duration of a ``with`` block, then restore what was installed before.

    Keys: ``fwd_tile``, ``bwd_tile``, ``batched_tile``, ``sol_tile`` as
    ``(W, VPL, NR)`` tuples; ``bwd_blocks_per_cu``, ``mx_slots``,
    ``bmx_waves`` as ints. Only sweeps and tile-forcing tests use this; the
    library's default launches read nothing but their arguments.
    """
    so = lib()
    before = Tuning()
    check(so.sy_tuning_get(ctypes.byref(before)), "sy_tuning_get")
    t = Tuning()
    ctypes.memmove(ctypes.byref(t), ctypes.byref(before), ctypes.sizeof(Tuning))
    for key, val in overrides.items():
        if key.endswith("_tile"):
            getattr(t, key)[:] = [int(x) for x in val]
        else:
            setattr(t, key, int(val))
    check(so.sy_tuning_set(ctypes.byref(t)), "sy_tuning_set")
    try:
        yield
    finally:
        if any(getattr(before, f)[k] if f.endswith("_tile") else getattr(before, f)
               for f, _ in Tuning._fields_ for k in (range(3) if f.endswith("_tile") else [0])):
            so.sy_tuning_set(ctypes.byref(before))
        else:
            so.sy_tuning_set(None)
