"""ctypes binding of the C ABI in ``include/ple_hip.h`` (``libple_hip.so``).

This is the binding a caller without the torch operators would use: plain
device pointers, sizes, dtype codes and a stream handle.  The helpers below
take torch tensors only to read their pointers and sizes; nothing here copies
or allocates except :func:`backward`, which takes a workspace from the caller
or allocates one through torch.

Every entry point returns an ``int`` code; non-zero codes raise
:class:`PleError` with ``ple_error_string``'s text.
"""

from __future__ import annotations

import ctypes
import os

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libple_hip.so")

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

# planner overrides (PLE_TUNE_* of the header; 0 = the planner's choice)
TUNE = {
    "FWD_FS": 0, "FWD_WG_PER_CU": 1, "FWD_FB": 2, "FWD_VEC": 3, "FWD_WIDE": 4, "BWD_SIMPLE": 5,
    "BWD_SIMPLE_GLOBAL": 6, "BWD_VEC": 7, "BWD_FS": 8, "BWD_RB": 9, "BWD_WG_PER_CU": 10, "BWD_MFMA": 11,
}
_DTYPE_CODES = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}

_lib = None


class Epilogue(ctypes.Structure):
    """``ple_epilogue_t``: the module tail fused into the kernels."""

    _fields_ = [
        ("bias", ctypes.c_void_p),
        ("lin_weight", ctypes.c_void_p),
        ("lin_bias", ctypes.c_void_p),
        ("relu", ctypes.c_int),
        ("relu_mask", ctypes.c_void_p),
    ]


class BackwardPlanInfo(ctypes.Structure):
    """``ple_backward_plan_info_t``: the backward's launch plan for a shape."""

    _fields_ = [
        ("sorted", ctypes.c_int),
        ("chunks", ctypes.c_int),
        ("features_per_group", ctypes.c_int),
        ("columns_per_lane", ctypes.c_int),
        ("lanes_per_row", ctypes.c_int),
        ("threads", ctypes.c_int),
        ("lds_bytes", ctypes.c_size_t),
        ("workspace_bytes", ctypes.c_size_t),
        ("bins_per_window", ctypes.c_int),
        ("windows", ctypes.c_int),
        ("matrix_cores", ctypes.c_int),
    ]


class PleError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{message} (code {code})")
        self.code = code


def lib() -> ctypes.CDLL:
    """Loads ``libple_hip.so`` once and declares every prototype."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built; run piecewiselinearembeddings_optimized_amd._build")
        L = ctypes.CDLL(_LIB_PATH)
        p, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
        L.ple_abi_version.argtypes, L.ple_abi_version.restype = [], i32
        L.ple_bin_index_bytes.argtypes, L.ple_bin_index_bytes.restype = [i64], i32
        L.ple_error_string.argtypes, L.ple_error_string.restype = [i32], ctypes.c_char_p
        L.ple_set_tuning.argtypes, L.ple_set_tuning.restype = [i32, i32], i32
        L.ple_forward_launch.argtypes = [p, p, p, p, p, p, p, p, i64, i64, i64, i64, i32, i32, p]
        L.ple_forward_launch.restype = i32
        L.ple_backward_workspace_bytes.argtypes = [i64, i64, i64, i64]
        L.ple_backward_workspace_bytes.restype = sz
        L.ple_backward_launch.argtypes = [p, p, p, p, p, p, p, p, p, p, i64, i64, i64, i64, i32, i32, p, sz, p]
        L.ple_backward_launch.restype = i32
        L.ple_backward_launch_noalloc.argtypes = [p, p, p, p, p, p, p, p, p, p, i64, i64, i64, i64, i32, i32, p]
        L.ple_backward_launch_noalloc.restype = i32
        L.ple_backward_plan_query.argtypes = [p, i64, i64, i64, i64, i32, i32, i32, i32,
                                              ctypes.POINTER(BackwardPlanInfo)]
        L.ple_backward_plan_query.restype = i32
        ep = ctypes.POINTER(Epilogue)
        L.ple_forward_epilogue_launch.argtypes = [p, p, p, p, p, ep, p, p, i64, i64, i64, i64, i32, p]
        L.ple_forward_epilogue_launch.restype = i32
        L.ple_backward_epilogue_launch.argtypes = [p, p, p, p, p, p, p, ep, p, p, p, p, p, i64, i64, i64, i64, i32,
                                                   p, sz, p]
        L.ple_backward_epilogue_launch.restype = i32
        L.ple_encode_launch.argtypes = [p, p, p, p, p, p, i64, i64, i64, i64, p]
        L.ple_encode_launch.restype = i32
        L.ple_encode_backward_launch.argtypes = [p, p, p, p, p, p, p, i64, i64, i64, i64, p]
        L.ple_encode_backward_launch.restype = i32
        L.ple_timing_start.argtypes, L.ple_timing_start.restype = [i32], i32
        L.ple_timing_stop.argtypes, L.ple_timing_stop.restype = [], i32
        L.ple_timing_read.argtypes = [i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int)]
        L.ple_timing_read.restype = i32
        _lib = L
    return _lib


def set_tuning(knob: str, value: int) -> int:
    """Sets planner override ``knob`` (a key of :data:`TUNE`); returns the
    previous value.  0 restores the planner's own choice."""
    return lib().ple_set_tuning(TUNE[knob], int(value))


TIMER_FORWARD, TIMER_BACKWARD = 0, 1


def timing_start(slots: int) -> None:
    """``ple_timing_start``: time the main kernel of the next ``slots``
    forward and backward launches (0 releases the events)."""
    check(lib().ple_timing_start(int(slots)))


def timing_stop() -> None:
    check(lib().ple_timing_stop())


def timing_read(which: int):
    """``(total_ms, launches)`` recorded for ``TIMER_FORWARD`` / ``TIMER_BACKWARD``."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int(0)
    check(lib().ple_timing_read(int(which), ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value


def check(code: int) -> None:
    if code != 0:
        raise PleError(code, lib().ple_error_string(code).decode())


def dtype_code(dtype: torch.dtype) -> int:
    return _DTYPE_CODES[dtype]


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def forward(x, bin_edges, inv_bin_widths, n_bins, weight, bias, output, bin_indices, quant_dtype,
            stream=None) -> None:
    """``ple_forward_launch`` into caller-provided ``output`` / ``bin_indices``."""
    n, f = x.shape
    _, bmax, d = weight.shape
    check(lib().ple_forward_launch(
        _ptr(x), _ptr(bin_edges), _ptr(inv_bin_widths), _ptr(n_bins), _ptr(weight), _ptr(bias),
        _ptr(output), _ptr(bin_indices), n, f, bmax, d, dtype_code(quant_dtype), dtype_code(output.dtype),
        _stream(stream)))


def workspace_bytes(n: int, f: int, bmax: int, d: int) -> int:
    return int(lib().ple_backward_workspace_bytes(n, f, bmax, d))


def backward_plan(n: int, f: int, bmax: int, d: int, grad_dtype=torch.float32, quant_dtype=None,
                  relu: bool = False, linear0: bool = False, grad_output=None) -> dict:
    """``ple_backward_plan_query``: the plan a backward launch of this shape
    takes, as a dict of :class:`BackwardPlanInfo`'s fields."""
    info = BackwardPlanInfo()
    q = grad_dtype if quant_dtype is None else quant_dtype
    check(lib().ple_backward_plan_query(_ptr(grad_output), n, f, bmax, d, dtype_code(grad_dtype), dtype_code(q),
                                        1 if relu else 0, 1 if linear0 else 0, ctypes.byref(info)))
    return {name: getattr(info, name) for name, _ in BackwardPlanInfo._fields_}


def backward(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices, grad_x, grad_weight,
             grad_bias, quant_dtype, workspace=None, stream=None) -> None:
    """``ple_backward_launch``; ``grad_*`` are caller-provided fp32 tensors or None."""
    n, f = x.shape
    _, bmax, d = weight.shape
    need = workspace_bytes(n, f, bmax, d)
    if workspace is None and need > 0:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().ple_backward_launch(
        _ptr(grad_output), _ptr(x), _ptr(bin_edges), _ptr(inv_bin_widths), _ptr(n_bins), _ptr(weight),
        _ptr(bin_indices), _ptr(grad_x), _ptr(grad_weight), _ptr(grad_bias), n, f, bmax, d,
        dtype_code(grad_output.dtype), dtype_code(quant_dtype), _ptr(workspace), ws_bytes, _stream(stream)))


def epilogue(bias=None, lin_weight=None, lin_bias=None, relu=False, relu_mask=None) -> Epilogue:
    def addr(t):
        return None if t is None else t.data_ptr()

    return Epilogue(addr(bias), addr(lin_weight), addr(lin_bias), 1 if relu else 0, addr(relu_mask))


def forward_epilogue(x, bin_edges, inv_bin_widths, n_bins, weight, epi: Epilogue, output, bin_indices,
                     quant_dtype, stream=None) -> None:
    """``ple_forward_epilogue_launch`` (fp32 ``output``)."""
    n, f = x.shape
    _, bmax, d = weight.shape
    check(lib().ple_forward_epilogue_launch(
        _ptr(x), _ptr(bin_edges), _ptr(inv_bin_widths), _ptr(n_bins), _ptr(weight), ctypes.byref(epi),
        _ptr(output), _ptr(bin_indices), n, f, bmax, d, dtype_code(quant_dtype), _stream(stream)))


def backward_epilogue(grad_output, x, bin_edges, inv_bin_widths, n_bins, weight, bin_indices, epi: Epilogue,
                      grad_x, grad_weight, grad_bias, grad_lin_weight, grad_lin_bias, quant_dtype,
                      workspace=None, stream=None) -> None:
    """``ple_backward_epilogue_launch``; gradients are caller-provided fp32 tensors or None."""
    n, f = x.shape
    _, bmax, d = weight.shape
    need = workspace_bytes(n, f, bmax, d)
    if workspace is None and need > 0:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    check(lib().ple_backward_epilogue_launch(
        _ptr(grad_output), _ptr(x), _ptr(bin_edges), _ptr(inv_bin_widths), _ptr(n_bins), _ptr(weight),
        _ptr(bin_indices), ctypes.byref(epi), _ptr(grad_x), _ptr(grad_weight), _ptr(grad_bias),
        _ptr(grad_lin_weight), _ptr(grad_lin_bias), n, f, bmax, d, dtype_code(quant_dtype), _ptr(workspace),
        ws_bytes, _stream(stream)))


def encode(x, bin_edges, inv_bin_widths, n_bins, offsets, output, stream=None) -> None:
    """``ple_encode_launch`` into a caller-provided fp32 ``output`` [N, total_bins]."""
    n, f = x.shape
    check(lib().ple_encode_launch(
        _ptr(x), _ptr(bin_edges), _ptr(inv_bin_widths), _ptr(n_bins), _ptr(offsets), _ptr(output), n, f,
        inv_bin_widths.shape[1], output.shape[1], _stream(stream)))


def encode_backward(grad_output, x, bin_edges, inv_bin_widths, n_bins, offsets, grad_x, stream=None) -> None:
    """``ple_encode_backward_launch`` into a caller-provided fp32 ``grad_x`` [N, F]."""
    n, f = x.shape
    check(lib().ple_encode_backward_launch(
        _ptr(grad_output), _ptr(x), _ptr(bin_edges), _ptr(inv_bin_widths), _ptr(n_bins), _ptr(offsets),
        _ptr(grad_x), n, f, inv_bin_widths.shape[1], grad_output.shape[1], _stream(stream)))
