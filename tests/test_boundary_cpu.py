"""Boundary checks that need no GPU: the C ABI library and its exports, the
operator schemas, the FakeTensor contract, the module surface and its CPU
path (the dense upstream formulation) against the oracle."""

from __future__ import annotations

import ctypes
import os
import re
import warnings

import numpy as np
import pytest
import torch

import piecewiselinearembeddings_optimized_amd as pkg
from oracle import ple_oracle as po
from tests.ple_cases import (
    BIN_CASE_NAMES, FORWARD_ATOL, FORWARD_RTOL, GRAD_ATOL, GRAD_RTOL, init_parameters_, make_bins,
    sample_features,
)

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "ple_hip.h")
LIB = os.path.join(REPO, "piecewiselinearembeddings_optimized_amd", "libple_hip.so")

REFERENCE_SCHEMAS = {
    # reference csrc/ops.cpp:35-58
    "forward": "rtdl_num_embeddings_cuda::forward(Tensor x, Tensor bin_edges, Tensor inv_bin_widths, "
               "Tensor n_bins, Tensor weight, ScalarType output_dtype) -> (Tensor output, Tensor bin_indices)",
    "backward": "rtdl_num_embeddings_cuda::backward(Tensor grad_output, Tensor x, Tensor bin_edges, "
                "Tensor inv_bin_widths, Tensor n_bins, Tensor weight, Tensor bin_indices, bool compute_grad_x, "
                "bool compute_grad_weight) -> (Tensor grad_x, Tensor grad_weight)",
}


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ple_[a-z_0-9]+)\s*\(", text)))


def _lib():
    return ctypes.CDLL(LIB)


def test_library_exports_every_declared_symbol():
    names = _header_functions()
    assert {"ple_forward_launch", "ple_backward_launch", "ple_backward_workspace_bytes"} <= set(names)
    lib = _lib()
    for n in names:
        assert hasattr(lib, n), n


def test_host_only_entry_points():
    lib = _lib()
    lib.ple_bin_index_bytes.argtypes = [ctypes.c_int64]
    assert [lib.ple_bin_index_bytes(b) for b in (1, 256, 257, 32768, 32769)] == [1, 1, 2, 2, 4]
    lib.ple_error_string.restype = ctypes.c_char_p
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8, -9):
        assert lib.ple_error_string(code)
    assert lib.ple_abi_version() >> 16 == 1
    assert pkg._C.abi_version() == lib.ple_abi_version()


def test_c_abi_rejects_bad_arguments_without_launching():
    lib = _lib()
    p = ctypes.c_void_p
    i64 = ctypes.c_int64
    lib.ple_forward_launch.argtypes = [p, p, p, p, p, p, p, p, i64, i64, i64, i64, ctypes.c_int, ctypes.c_int, p]
    dummy = p(256)
    args = [dummy] * 5 + [None, dummy, dummy]
    assert lib.ple_forward_launch(*args, 4, 0, 3, 2, 0, 0, None) == -2       # F = 0
    assert lib.ple_forward_launch(*args, 0, 2, 3, 65, 0, 0, None) == 0       # D > 64: accepted (any D)
    assert lib.ple_forward_launch(*args, 4, 2, 3, 1 << 29, 0, 0, None) == -5  # F * B * 2D beyond int32 offsets
    assert lib.ple_forward_launch(*args, 4, 2, (1 << 24) + 1, 2, 0, 0, None) == -5   # max bins > 2^24
    assert lib.ple_forward_launch(*args, 0, 2, 40000, 4, 0, 0, None) == 0    # int32 indices: accepted
    assert lib.ple_forward_launch(*args, 0, 2, 32768, 64, 0, 0, None) == 0   # tables far beyond LDS: accepted
    assert lib.ple_forward_launch(*args, 4, 2, 3, 2, 9, 0, None) == -3       # bad dtype
    assert lib.ple_forward_launch(*args, 0, 2, 3, 2, 0, 0, None) == 0        # empty batch: no launch
    nulls = [None] * 8
    assert lib.ple_forward_launch(*nulls, 4, 2, 3, 2, 0, 0, None) == -1
    lib.ple_backward_launch.argtypes = [p, p, p, p, p, p, p, p, p, p, i64, i64, i64, i64, ctypes.c_int,
                                        ctypes.c_int, p, ctypes.c_size_t, p]
    assert lib.ple_backward_launch(*[None] * 10, 4, 2, 3, 2, 0, 0, None, 0, None) == 0   # nothing requested
    assert lib.ple_backward_launch(*[None] * 7, dummy, None, None, 4, 2, 3, 2, 0, 0, None, 0, None) == -1


def test_ctypes_binding_declares_the_header_and_maps_errors():
    from piecewiselinearembeddings_optimized_amd import capi

    L = capi.lib()
    for n in _header_functions():
        assert getattr(L, n).argtypes is not None, n
    capi.check(0)
    with pytest.raises(capi.PleError, match="combination not supported") as ei:
        capi.check(-7)
    assert ei.value.code == -7
    assert capi.workspace_bytes(0, 2, 3, 4) == 0
    assert capi.workspace_bytes(1024, 8, 48, 24) > 0
    assert capi.workspace_bytes(1024, 8, 48, 1 << 29) == 0   # rejected sizes need nothing
    assert capi.workspace_bytes(4096, 8, 48, 96) > 0         # wider rows than the module's: accepted
    # tables beyond LDS: the fallback's chunk partials
    assert capi.workspace_bytes(2048, 4, 40000, 4) >= 4 * 40000 * 2 * 4 * 4


def test_backward_plan_query_and_workspace_sizes():
    """The plan query needs no device (the planner assumes 256 CUs without
    one, as on an MI355X), and the workspace holds chunk partials only: a
    sorted plan of one chunk -- more feature groups than resident
    workgroups -- writes dW / db from the gradient kernel and needs none."""
    from piecewiselinearembeddings_optimized_amd import capi

    one = capi.backward_plan(1024, 8192, 48, 32)
    assert one["sorted"] == 1 and one["chunks"] == 1
    assert one["workspace_bytes"] == 0
    assert capi.workspace_bytes(1024, 8192, 48, 32) == 0
    c1 = capi.backward_plan(65536, 128, 48, 32)      # the headline shape: several chunks
    assert c1["sorted"] == 1 and c1["chunks"] > 1
    assert c1["features_per_group"] * c1["lanes_per_row"] >= 1 and c1["columns_per_lane"] == 4
    assert c1["workspace_bytes"] >= c1["chunks"] * 128 * 48 * 2 * 32 * 4
    assert capi.workspace_bytes(65536, 128, 48, 32) >= c1["workspace_bytes"]
    c4 = capi.backward_plan(8192, 1024, 96, 24, grad_dtype=torch.bfloat16)
    # a 16-bit gradient in its own dtype: the matrix-core kernel, groups of
    # four features, 512-thread workgroups, one chunk
    assert c4["matrix_cores"] == 1 and c4["sorted"] == 0 and c4["chunks"] == 1 and c4["workspace_bytes"] == 0
    assert c4["features_per_group"] == 4 and c4["threads"] == 512 and c4["lds_bytes"] <= 160 * 1024
    # ... not past 96 bins, nor where it would take more than 8 chunks
    assert capi.backward_plan(8192, 1024, 128, 24, grad_dtype=torch.bfloat16)["matrix_cores"] == 0
    assert capi.backward_plan(65536, 32, 96, 24, grad_dtype=torch.bfloat16)["matrix_cores"] == 0
    assert capi.backward_plan(65536, 128, 48, 32, grad_dtype=torch.bfloat16)["chunks"] == 8
    c4s = capi.backward_plan(8192, 1024, 96, 24, grad_dtype=torch.float32, quant_dtype=torch.bfloat16)
    assert c4s["matrix_cores"] == 0 and c4s["sorted"] == 1 and c4s["columns_per_lane"] == 4
    assert c1["matrix_cores"] == 0
    assert c1["windows"] == 1 and c1["bins_per_window"] == 48
    with pytest.raises(capi.PleError):
        capi.backward_plan(1024, 8, 48, 24, grad_dtype=torch.bfloat16, quant_dtype=torch.float16)


@pytest.mark.parametrize("n,f,bmax,d", [(2048, 4, 40000, 4), (65536, 128, 1024, 32), (65536, 64, 4096, 16),
                                        (65536, 32, 48, 256), (2048, 3, 32768, 2), (1000, 3, 700, 62)])
def test_backward_plan_bin_windows(n, f, bmax, d):
    """Tables beyond LDS take the sorted path in windows of bins: the
    windows cover every bin (bins_per_window * windows >= B, no empty last
    window), each fits the 12-bit bin field of a piece and two workgroups'
    LDS per CU, and the partials (whole tables, every chunk) are in the
    workspace even for one chunk.  Plans with the per-feature sums of the
    module epilogues keep the fallback kernels."""
    from piecewiselinearembeddings_optimized_amd import capi

    pl = capi.backward_plan(n, f, bmax, d)
    assert pl["sorted"] == 1 and pl["windows"] > 1 and pl["features_per_group"] == 1
    bw, nw = pl["bins_per_window"], pl["windows"]
    assert bw <= 4096 and bw * nw >= bmax and bw * (nw - 1) < bmax
    assert pl["lds_bytes"] <= 80 * 1024
    assert pl["workspace_bytes"] >= pl["chunks"] * f * bmax * 2 * d * 4
    lin = capi.backward_plan(n, f, bmax, d, linear0=True) if d <= 64 else None
    assert lin is None or lin["sorted"] == 0


def test_timing_api_without_a_device():
    """Kernel timing: argument errors, and start(0) / stop / read with nothing
    recorded need no device."""
    import ctypes

    from piecewiselinearembeddings_optimized_amd import capi

    L = capi.lib()
    assert L.ple_timing_start(-1) == -2
    assert L.ple_timing_start(0) == 0
    assert L.ple_timing_stop() == 0
    ms, n = ctypes.c_double(1.0), ctypes.c_int(5)
    assert L.ple_timing_read(2, ctypes.byref(ms), ctypes.byref(n)) == -2
    assert L.ple_timing_read(0, None, ctypes.byref(n)) == -1
    assert capi.timing_read(capi.TIMER_FORWARD) == (0.0, 0)
    assert capi.timing_read(capi.TIMER_BACKWARD) == (0.0, 0)


def test_tuning_knobs_round_trip():
    """Planner overrides: set, read back as the previous value, restored;
    unknown knobs rejected."""
    from piecewiselinearembeddings_optimized_amd import capi

    L = capi.lib()
    assert set(capi.TUNE.values()) == set(range(len(capi.TUNE)))
    header = open(HEADER).read()
    for name, code in capi.TUNE.items():
        assert re.search(rf"PLE_TUNE_{name}\s*=\s*{code}\b", header), name
    for name in capi.TUNE:
        assert capi.set_tuning(name, 3) == 0
        assert capi.set_tuning(name, 0) == 3
    assert L.ple_set_tuning(len(capi.TUNE), 1) == -2
    assert L.ple_set_tuning(-1, 1) == -2


def test_operator_schemas_match_reference():
    ops = torch.ops.rtdl_num_embeddings_cuda
    for name, schema in REFERENCE_SCHEMAS.items():
        assert str(getattr(ops, name).default._schema) == schema
    assert hasattr(ops, "forward_with_bias") and hasattr(ops, "backward_with_bias")


@pytest.mark.parametrize("bmax,idx_dtype", [(5, torch.uint8), (256, torch.uint8), (300, torch.int16), (40000, torch.int32)])
def test_fake_tensor_contract(bmax, idx_dtype):
    from torch._subclasses.fake_tensor import FakeTensorMode

    ops = torch.ops.rtdl_num_embeddings_cuda
    with FakeTensorMode(allow_non_fake_inputs=False):
        x = torch.empty(7, 3, device="cuda")
        e = torch.empty(3, bmax + 1, device="cuda")
        iw = torch.empty(3, bmax, device="cuda")
        nb = torch.empty(3, dtype=torch.int32, device="cuda")
        w = torch.empty(3, bmax, 5, device="cuda")
        b = torch.empty(3, 5, device="cuda")
        out, idx = ops.forward(x, e, iw, nb, w, torch.bfloat16)
        assert out.shape == (7, 3, 5) and out.dtype == torch.bfloat16
        assert idx.shape == (7, 3) and idx.dtype == idx_dtype
        out2, _ = ops.forward_with_bias(x, e, iw, nb, w, b, torch.bfloat16)
        assert out2.dtype == torch.float32
        g = torch.empty(7, 3, 5, device="cuda")
        gx, gw = ops.backward(g, x, e, iw, nb, w, idx, True, False)
        assert gx.shape == x.shape and gw.shape == (0,)
        gx, gw, gb = ops.backward_with_bias(g, x, e, iw, nb, w, idx, torch.float32, False, True, True)
        assert gx.shape == (0,) and gw.shape == w.shape and gb.shape == (3, 5)
        with pytest.raises(Exception):
            ops.forward(x.double(), e, iw, nb, w, torch.float32)


def test_package_surface():
    import rtdl_num_embeddings_cuda as r

    assert r.__all__ == ["CudaPiecewiseLinearEmbeddings"]
    assert r.__version__ == "0.2.0.dev0"
    assert r._C is pkg._C
    import rtdl_num_embeddings_cuda._C  # noqa: F401


def _module(case, d, activation, version, seed=0):
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings

    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        m = CudaPiecewiseLinearEmbeddings(make_bins(case), d, activation=activation, version=version)
    init_parameters_(m, seed=seed)
    return m


def test_module_parameters_and_state_dict():
    a = _module("ragged", 10, False, "A")
    b = _module("ragged", 10, True, "B")
    assert set(dict(a.named_parameters())) == {"linear.weight", "linear.bias"}
    assert set(dict(b.named_parameters())) == {"linear.weight", "linear0.weight", "linear0.bias"}
    sd = a.state_dict()
    assert not any(k.startswith("_cuda") for k in sd)
    assert set(sd) == {"impl.weight", "impl.bias", "impl.mask", "linear.weight", "linear.bias"}
    assert a.get_output_shape() == torch.Size((4, 10))
    assert a.linear.weight.shape == (4, 5, 10)
    c = _module("single_bin", 4, False, "A")
    assert "impl.single_bin_mask" in c.state_dict()
    # strict round trip of the trainable state
    a2 = _module("ragged", 10, False, "A", seed=3)
    a2.linear.load_state_dict(a.linear.state_dict(), strict=True)
    assert torch.equal(a2.linear.weight, a.linear.weight)


def test_module_buffers_follow_reference_layout():
    m = _module("ragged", 6, False, "A")
    bins = [b.numpy() for b in make_bins("ragged")]
    edges, iw, nb = po.pad_bins(bins)
    np.testing.assert_array_equal(m._cuda_bin_edges.numpy(), edges)
    np.testing.assert_array_equal(m._cuda_inv_bin_widths.numpy(), iw)
    np.testing.assert_array_equal(m._cuda_n_bins.numpy(), nb)
    assert m._cuda_n_bins.dtype == torch.int32


def test_module_constructor_validation():
    from rtdl_num_embeddings_cuda import CudaPiecewiseLinearEmbeddings

    with pytest.raises(AssertionError):
        CudaPiecewiseLinearEmbeddings(make_bins("equal"), 65, activation=False, version="A")
    with pytest.raises(ValueError):
        CudaPiecewiseLinearEmbeddings([], 8, activation=False, version="A")
    with pytest.raises(ValueError):
        CudaPiecewiseLinearEmbeddings([torch.tensor([1.0, 0.0])], 8, activation=False, version="A")
    with pytest.raises(ValueError):
        CudaPiecewiseLinearEmbeddings([torch.tensor([0.0, float("nan")])], 8, activation=False, version="A")
    with pytest.warns(UserWarning):
        CudaPiecewiseLinearEmbeddings(make_bins("equal"), 8, activation=False)


@pytest.mark.parametrize("case", BIN_CASE_NAMES)
@pytest.mark.parametrize("version", ("A", "B"))
@pytest.mark.parametrize("activation", (False, True))
def test_module_cpu_path_matches_oracle(case, version, activation):
    m = _module(case, 10, activation, version, seed=5)
    bins = make_bins(case)
    x = sample_features(bins, batch_size=128, seed=7).requires_grad_(True)
    out = m(x)
    tables = po.pad_bins([b.numpy() for b in bins])
    lin0 = None if m.linear0 is None else (m.linear0.weight.detach().numpy(), m.linear0.bias.detach().numpy())
    bias = None if m.linear.bias is None else m.linear.bias.detach().numpy()
    ref, _, _ = po.module_forward(x.detach().numpy(), tables, m.linear.weight.detach().numpy(), bias=bias,
                                  linear0=lin0, activation=activation)
    torch.testing.assert_close(out.detach().double(), torch.from_numpy(ref), rtol=FORWARD_RTOL, atol=FORWARD_ATOL)
    if not activation:
        g = torch.randn_like(out)
        out.backward(g)
        edges, iw, nb = tables
        idx = po.bin_indices(x.detach().numpy(), edges, nb)
        r = po.backward(g.numpy(), x.detach().numpy(), edges, iw, nb, m.linear.weight.detach().numpy(), idx)
        dx = r["dx"] + (0.0 if m.linear0 is None else (g.numpy() * m.linear0.weight.detach().numpy()[None]).sum(-1))
        torch.testing.assert_close(x.grad.double(), torch.from_numpy(dx), rtol=GRAD_RTOL, atol=GRAD_ATOL)
        torch.testing.assert_close(m.linear.weight.grad.double(), torch.from_numpy(r["dw"]), rtol=GRAD_RTOL, atol=GRAD_ATOL)


def test_module_rejects_bad_shapes_on_cpu():
    m = _module("equal", 4, False, "A")
    with pytest.raises(ValueError):
        m(torch.zeros(4, 3, 1))
    with pytest.raises(ValueError):
        m(torch.zeros(4, 2))


@pytest.mark.parametrize("case_name", ["equal", "ragged", "single_bin", "all_single_bin"])
def test_encoding_module_cpu_path_is_the_upstream_dense_encoding(case_name):
    import numpy as np

    from oracle import ple_oracle as po
    from piecewiselinearembeddings_optimized_amd import CudaPiecewiseLinearEncoding
    from tests.ple_cases import make_bins, sample_features

    bins = make_bins(case_name)
    m = CudaPiecewiseLinearEncoding(bins)
    total = sum(len(b) - 1 for b in bins)
    assert m.get_output_shape() == torch.Size((total,))
    assert list(m.state_dict()) == [k for k in ("impl.weight", "impl.bias", "impl.single_bin_mask", "impl.mask")
                                   if getattr(m.impl, k.split(".")[1]) is not None]
    x = sample_features(bins, batch_size=64, seed=3)
    out = m(x)
    assert out.shape == (64, total) and out.dtype == torch.float32
    edges, iw, nb = po.pad_bins([b.numpy() for b in bins])
    np.testing.assert_allclose(out.numpy(), po.encoding_closed_form(x.numpy(), edges, iw, nb), rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        m(x[:, :1])
