"""The CPU provider (m3.c_amd/csrc/host/m3_cpu_provider.c) against the
oracle, on the host backend (CPU only).

The CPU provider runs the sessions that disable the GPU provider
(allow_metal = false) and the nodes a GPU session leaves to the CPU. Its
cases are the GPU parity cases (tests/test_gpu_parity.py), run with the
host backend in place of the HIP backend: every binary layout class, op
and dtype mix, strided and aliased views; all cast pairs, every 16-bit
source and an F32 bit sweep; softmax over widths, dtypes, zero tails,
subnormal ties, strided, transposed and in-place rows; Snake1d, TANH and
GATED_SILU layouts, NaN-heavy operands and aliases. Every output byte must
equal the oracle's, status included. The list semantics are the
reference host provider's (src/m3_op_execute_host.c:5-60): each command's
data check runs right before it, so a failing check stops the list with
the commands before it done.
"""
import numpy as np
import pytest

import test_gpu_parity as gp
from conftest import m3
from harness import HostFixture, ViewSpec, as_bytes


@pytest.fixture(scope="module")
def host():
    fixture = HostFixture()
    yield fixture
    fixture.close()


def test_host_backend_reports_the_cpu_provider(host):
    info = m3.BackendInfo()
    error = m3.Error()
    assert host.lib.m3_backend_get_info(host.backend, info,
                                        error) == m3.OK
    assert info.kind == m3.BACKEND_HOST and info.unified_memory


@pytest.mark.parametrize("op", [m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV])
@pytest.mark.parametrize("layout", range(len(gp.BINARY_LAYOUTS)))
def test_binary_f32_layouts(host, op, layout):
    gp.test_binary_f32_layouts(host, op, layout)


@pytest.mark.parametrize("dtypes", [(m3.F16, m3.F16, m3.F16),
                                    (m3.F32, m3.BF16, m3.F16),
                                    (m3.BF16, m3.F16, m3.F32)])
@pytest.mark.parametrize("layout", [0, 4, 8])
def test_binary_mixed_dtypes(host, dtypes, layout):
    gp.test_binary_mixed_dtypes(host, dtypes, layout)


def test_binary_strided_offset_and_alias(host):
    gp.test_binary_strided_and_offset_views(host)
    gp.test_binary_exact_alias_in_place(host)


@pytest.mark.parametrize("src", gp.DTYPES)
@pytest.mark.parametrize("dst", gp.DTYPES)
def test_cast_all_pairs(host, src, dst):
    for count in (1, 3, 1021):
        gp.test_cast_all_pairs(host, src, dst, count)


def test_cast_exhaustive_sources_sweep_and_strides(host):
    gp.test_cast_exhaustive_16bit_sources(host)
    gp.test_cast_f32_dense_bit_sweep(host)
    gp.test_cast_strided_input(host)


@pytest.mark.parametrize("width", [1, 3, 12, 260, 1024, 3000])
def test_softmax_widths(host, width):
    gp.test_softmax_widths(host, width)


@pytest.mark.parametrize("dtypes", [(m3.F16, m3.F16), (m3.BF16, m3.F32)])
def test_softmax_dtypes(host, dtypes):
    gp.test_softmax_dtypes(host, dtypes, 256)


def test_softmax_tails_ties_strides(host):
    gp.test_softmax_zero_tails(host, 200)
    gp.test_softmax_subnormal_ties(host, 128)
    gp.test_softmax_strided_and_in_place(host)


@pytest.mark.parametrize("shape", [(1, 3, 5), (3, 7, 12), (2, 16, 1024)])
def test_snake1d_layouts(host, shape):
    gp.test_snake1d_layouts(host, shape)


def test_snake1d_strided_and_alias(host):
    gp.test_snake1d_strided_input_and_alias(host)


@pytest.mark.parametrize("shape", [(1,), (4, 1001), (2, 3, 4, 5, 6, 7, 2, 3)])
def test_tanh_layouts(host, shape):
    gp.test_tanh_layouts(host, shape)


def test_tanh_strided_offset_and_in_place(host):
    gp.test_tanh_strided_offset_and_in_place(host)


@pytest.mark.parametrize("dtypes", [(g, u, o) for g in gp.FLOAT_DTYPES
                                    for u in gp.FLOAT_DTYPES
                                    for o in gp.FLOAT_DTYPES])
def test_gated_silu_dtypes(host, dtypes):
    gp.test_gated_silu_dtypes(host, dtypes, 4099)


def test_gated_silu_nan_strided_and_aliases(host):
    gp.test_gated_silu_nan_operands(host, 4003)
    gp.test_gated_silu_strided_and_aliases(host)


def test_data_check_runs_right_before_each_command(host):
    """[MUL, SOFTMAX over a NaN row, ADD]: the MUL has run, the SOFTMAX
    fails with OUT_OF_RANGE and writes nothing, the ADD does not run."""
    a = np.arange(8, dtype=np.float32)
    logits = np.array([[1.0, np.nan, 2.0, 3.0]], np.float32)
    handles = host.upload([as_bytes(a), as_bytes(a),
                           np.zeros(32, np.uint8), as_bytes(logits),
                           np.zeros(16, np.uint8), np.zeros(32, np.uint8)])
    specs = [ViewSpec(0, m3.F32, (8,)), ViewSpec(1, m3.F32, (8,)),
             ViewSpec(2, m3.F32, (8,)), ViewSpec(3, m3.F32, (1, 4)),
             ViewSpec(4, m3.F32, (1, 4)), ViewSpec(5, m3.F32, (8,))]
    v = host.views(handles, specs)
    status, message = host.execute([(m3.OP_MUL, [v[0], v[1], v[2]]),
                                    (m3.OP_SOFTMAX, [v[3], v[4]]),
                                    (m3.OP_ADD, [v[0], v[1], v[5]])])
    assert status == m3.OUT_OF_RANGE and "NaN" in message
    mul, soft, add = host.download([handles[2], handles[4], handles[5]],
                                   [np.zeros(8, np.float32),
                                    np.zeros(4, np.float32),
                                    np.zeros(8, np.float32)])
    assert np.array_equal(mul, a * a)
    assert not soft.any() and not add.any()


def test_cast_to_i32_checks_its_values(host):
    """An out-of-range float to I32 cast fails with OUT_OF_RANGE and leaves
    its output untouched; in-range values truncate toward zero."""
    good = np.array([-2.5, 2.5, 2147483520.0, -2147483648.0], np.float32)
    bad = np.array([1.0, 2147483648.0, 0.0, 0.0], np.float32)
    for values, expected in ((good, m3.OK), (bad, m3.OUT_OF_RANGE)):
        status, out, _ = host.run(
            m3.OP_CAST, [as_bytes(values), np.zeros(16, np.uint8)],
            [ViewSpec(0, m3.F32, (4,)), ViewSpec(1, m3.I32, (4,))])
        assert status == expected
        result = out[1].view(np.int32)
        if expected == m3.OK:
            assert list(result) == [-2, 2, 2147483520, -2147483648]
        else:
            assert not result.any()
