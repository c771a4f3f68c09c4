"""ctypes wrapper around ``oracle/ple_oracle.c`` (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg use this module, as the checker.  See ``ple_oracle.c`` for the reference
lines each routine restates.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libple_oracle.so")
_LIB = None

QUANT_CODES = {"f32": 0, "f16": 1, "bf16": 2}


def build(force: bool = False) -> str:
    """Compile the C oracle with ``oracle/Makefile`` (gcc)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        lib.ple_oracle_forward_f32.argtypes = [p, p, p, p, p, p, ctypes.c_int, i64, i64, i64, i64, p, p, p]
        lib.ple_oracle_forward_f32.restype = None
        lib.ple_oracle_backward_f64.argtypes = [p, p, p, p, p, p, p, p, ctypes.c_int, i64, i64, i64, i64,
                                                p, p, p, p, p, p, p, p, p, p]
        lib.ple_oracle_backward_f64.restype = None
        lib.ple_oracle_quantize.argtypes = [ctypes.c_float, ctypes.c_int]
        lib.ple_oracle_quantize.restype = ctypes.c_float
        _LIB = lib
    return _LIB


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def quantize_scalar(v: float, quant: str) -> float:
    return float(_lib().ple_oracle_quantize(float(v), QUANT_CODES[quant]))


def forward_f32(x, bin_edges, inv_bin_widths, n_bins, weight, bias=None, quant="f32"):
    """fp32 mirror of the reference forward arithmetic.

    Returns ``(out float32 [N, F, D], idx int32 [N, F])``.  With ``quant`` other
    than f32 the values of ``out`` are exactly representable in that dtype
    (before the optional bias add).
    """
    x = _c(x, np.float32)
    e = _c(bin_edges, np.float32)
    iw = _c(inv_bin_widths, np.float32)
    nb = _c(n_bins, np.int32)
    w = _c(weight, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    n, f = x.shape
    _, bmax, d = w.shape
    out = np.empty((n, f, d), dtype=np.float32)
    idx = np.empty((n, f), dtype=np.int32)
    scratch = np.empty((f, bmax, d), dtype=np.float32)
    _lib().ple_oracle_forward_f32(_ptr(x), _ptr(e), _ptr(iw), _ptr(nb), _ptr(w), _ptr(b),
                                  QUANT_CODES[quant], n, f, bmax, d, _ptr(out), _ptr(idx), _ptr(scratch))
    return out, idx


def backward_f64(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, idx, quant="f32",
                 grad_bias_source=None, want_dx=True, want_dw=True):
    """float64 closed-form backward; returns a dict like ``ple_oracle.backward``."""
    g = _c(grad_output, np.float32)
    gb = None if grad_bias_source is None else _c(grad_bias_source, np.float32)
    x = _c(x, np.float32)
    e = _c(bin_edges, np.float32)
    iw = _c(inv_bin_widths, np.float32)
    nb = _c(n_bins, np.int32)
    w = _c(weight, np.float32)
    ix = _c(idx, np.int32)
    n, f = x.shape
    _, bmax, d = w.shape
    res = {}
    dx = dxa = dw = dwa = db = dba = None
    if want_dx:
        dx = np.empty((n, f)); dxa = np.empty((n, f))
    if want_dw:
        dw = np.empty((f, bmax, d)); dwa = np.empty((f, bmax, d))
        db = np.empty((f, d)); dba = np.empty((f, d))
    scr = [np.empty((f, bmax, d)) for _ in range(4)] if want_dw else [None] * 4
    _lib().ple_oracle_backward_f64(_ptr(g), _ptr(gb), _ptr(x), _ptr(e), _ptr(iw), _ptr(nb), _ptr(w), _ptr(ix),
                                   QUANT_CODES[quant], n, f, bmax, d,
                                   _ptr(dx), _ptr(dxa), _ptr(dw), _ptr(dwa), _ptr(db), _ptr(dba),
                                   *[_ptr(s) for s in scr])
    if want_dx:
        res["dx"], res["dx_abs"] = dx, dxa
    if want_dw:
        res["dw"], res["dw_abs"], res["db"], res["db_abs"] = dw, dwa, db, dba
        res["bucket"], res["weighted"] = scr[0], scr[1]
    return res
