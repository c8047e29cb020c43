"""Known-answer cases taken from the reference's own tests.

Each case is one command (kind, storages, views) plus a check of the
expected result, with the reference test it comes from. The same cases run
on the oracle (CPU), the compiled reference and the HIP provider (GPU).
"""
import math
from dataclasses import dataclass
from typing import Callable, List

import numpy as np

from conftest import m3
from harness import ViewSpec, as_bytes, bits_f32, f32_bits


@dataclass
class Case:
    name: str
    source: str
    kind: int
    storages: List[np.ndarray]
    views: List[ViewSpec]
    check: Callable  # (status, storages) -> None (asserts)


def u16(values):
    return np.asarray(values, dtype=np.uint16)


def f32(values):
    return np.asarray(values, dtype=np.float32)


def out_f32(storages, index, count, offset=0):
    return storages[index][offset:offset + 4 * count].view(np.float32)


def out_u16(storages, index, count):
    return storages[index][:2 * count].view(np.uint16)


def out_i32(storages, index, count):
    return storages[index][:4 * count].view(np.int32)


def _expect_ok(status):
    assert status == m3.OK, m3.status_name(status)


CASES = []


def case(name, source, kind, storages, views):
    def register(check):
        CASES.append(Case(name, source, kind, storages, views, check))
        return check
    return register


# ---- CAST -----------------------------------------------------------------

F16_SOURCE = f32([1.00048828125, 1.00146484375, math.inf, -math.inf,
                  math.nan, 2.0 ** -24, 2.0 ** -25])


@case("cast_f32_f16_rounding", "tests/test_op_basic.c:16-86",
      m3.OP_CAST, [as_bytes(F16_SOURCE), as_bytes(np.zeros(7, np.uint16))],
      [ViewSpec(0, m3.F32, (7,)), ViewSpec(1, m3.F16, (7,))])
def _(status, s):
    _expect_ok(status)
    assert list(out_u16(s, 1, 7)) == [0x3c00, 0x3c02, 0x7c00, 0xfc00, 0x7e00,
                                      0x0001, 0x0000]


@case("cast_f16_f32_roundtrip", "tests/test_op_basic.c:87-101",
      m3.OP_CAST,
      [as_bytes(u16([0x3c00, 0x3c02, 0x7c00, 0xfc00, 0x7e00, 0x0001,
                     0x0000])), as_bytes(F16_SOURCE)],
      [ViewSpec(0, m3.F16, (7,)), ViewSpec(1, m3.F32, (7,))])
def _(status, s):
    _expect_ok(status)
    v = out_f32(s, 1, 7)
    assert v[0] == 1.0 and v[1] == 1.001953125
    assert math.isinf(v[2]) and v[2] > 0 and math.isinf(v[3]) and v[3] < 0
    assert math.isnan(v[4]) and v[5] == 2.0 ** -24 and v[6] == 0.0


@case("cast_f32_bf16_rounding", "tests/test_metal_cast.c:173-223",
      m3.OP_CAST,
      [as_bytes(f32([1.00390625, 1.01171875, math.inf, math.nan])),
       as_bytes(np.zeros(4, np.uint16))],
      [ViewSpec(0, m3.F32, (4,)), ViewSpec(1, m3.BF16, (4,))])
def _(status, s):
    _expect_ok(status)
    assert list(out_u16(s, 1, 4)) == [0x3f80, 0x3f82, 0x7f80, 0x7fc0]


@case("cast_f32_i32_truncates", "tests/test_op_basic.c:124-137",
      m3.OP_CAST, [as_bytes(f32([2.9, -2.9])),
                   as_bytes(np.zeros(2, np.int32))],
      [ViewSpec(0, m3.F32, (2,)), ViewSpec(1, m3.I32, (2,))])
def _(status, s):
    _expect_ok(status)
    assert list(out_i32(s, 1, 2)) == [2, -2]


@case("cast_f32_i32_invalid_is_atomic", "tests/test_op_basic.c:138-158",
      m3.OP_CAST,
      [as_bytes(f32([math.nan, math.inf, -math.inf, 2147483648.0])),
       as_bytes(np.full(4, 77, np.int32))],
      [ViewSpec(0, m3.F32, (4,)), ViewSpec(1, m3.I32, (4,))])
def _(status, s):
    assert status == m3.OUT_OF_RANGE
    assert list(out_i32(s, 1, 4)) == [77, 77, 77, 77]


@case("cast_f32_i32_in_place", "tests/test_metal_cast.c:248-269",
      m3.OP_CAST, [as_bytes(f32([2.9, -2.9]))],
      [ViewSpec(0, m3.F32, (2,)), ViewSpec(0, m3.I32, (2,))])
def _(status, s):
    _expect_ok(status)
    assert list(out_i32(s, 0, 2)) == [2, -2]


@case("cast_f16_bf16_in_place", "tests/test_metal_cast.c:270-290",
      m3.OP_CAST, [as_bytes(u16([0x3c00, 0x7c01, 0x0001]))],
      [ViewSpec(0, m3.F16, (3,)), ViewSpec(0, m3.BF16, (3,))])
def _(status, s):
    _expect_ok(status)
    assert list(out_u16(s, 0, 3)) == [0x3f80, 0x7fc0, 0x3380]


# ---- ADD / MUL --------------------------------------------------------------

@case("add_strided_broadcast", "tests/test_op_basic.c:164-247",
      m3.OP_ADD,
      [as_bytes(f32([1, 4, 2, 5, 3, 6])), as_bytes(f32([10, 20, 30])),
       as_bytes(np.zeros(6, np.float32))],
      [ViewSpec(0, m3.F32, (2, 3), (4, 8)), ViewSpec(1, m3.F32, (3,)),
       ViewSpec(2, m3.F32, (2, 3))])
def _(status, s):
    _expect_ok(status)
    assert list(out_f32(s, 2, 6)) == [11, 22, 33, 14, 25, 36]


@case("mul_scalar_exact_alias", "tests/test_op_basic.c:248-260",
      m3.OP_MUL,
      [as_bytes(f32([11, 22, 33, 14, 25, 36])), as_bytes(f32([2]))],
      [ViewSpec(0, m3.F32, (2, 3)), ViewSpec(1, m3.F32, (1,)),
       ViewSpec(0, m3.F32, (2, 3))])
def _(status, s):
    _expect_ok(status)
    v = out_f32(s, 0, 6)
    assert v[0] == 22.0 and v[5] == 72.0


@case("add_f32_strided_rounding", "tests/test_metal_basic_arithmetic.c:"
      "123-173", m3.OP_ADD,
      [as_bytes(f32([16777216.0, -16777216.0, 1.00000011920928955078125,
                     2.0 ** -149, -3.5, 8.0])),
       as_bytes(f32([1.0, 2.0 ** -24, 0.25])),
       as_bytes(np.zeros(6, np.float32))],
      [ViewSpec(0, m3.F32, (2, 3), (4, 8)), ViewSpec(1, m3.F32, (3,)),
       ViewSpec(2, m3.F32, (2, 3))])
def _(status, s):
    _expect_ok(status)
    out = out_f32(s, 2, 6)
    assert int(out.view(np.uint32)[0]) == 0x4b800000
    left = f32([16777216.0, -16777216.0, 1.00000011920928955078125,
                2.0 ** -149, -3.5, 8.0]).reshape(3, 2).T
    right = f32([1.0, 2.0 ** -24, 0.25])
    assert np.array_equal((left + right).reshape(-1).view(np.uint32),
                          out.view(np.uint32))


def _f16_mul_expected():
    left = u16([0x3c00, 0x4000, 0xc200, 0x3800]).view(np.float16)
    right = u16([0x3e00, 0x3555]).view(np.float16)
    product = (left.astype(np.float32).reshape(2, 2) *
               right.astype(np.float32)).astype(np.float16)
    return product.reshape(-1).view(np.uint16)


@case("mul_f16_strided_broadcast", "tests/test_metal_basic_arithmetic.c:"
      "175-218", m3.OP_MUL,
      [as_bytes(u16([0x3c00, 0x4000, 0xc200, 0x3800])),
       as_bytes(u16([0x3e00, 0x7e00, 0x3555])),
       as_bytes(np.zeros(4, np.uint16))],
      [ViewSpec(0, m3.F16, (2, 2)), ViewSpec(1, m3.F16, (2,), (4,)),
       ViewSpec(2, m3.F16, (2, 2))])
def _(status, s):
    _expect_ok(status)
    assert np.array_equal(out_u16(s, 2, 4), _f16_mul_expected())


@case("add_bf16_left_alias", "tests/test_metal_basic_arithmetic.c:220-262",
      m3.OP_ADD,
      [as_bytes(u16([0x3f80, 0x3f81, 0xbf80, 0x7f7f])),
       as_bytes(u16([0x3b80, 0x3b80, 0x3f00, 0xff7f]))],
      [ViewSpec(0, m3.BF16, (4,)), ViewSpec(1, m3.BF16, (4,)),
       ViewSpec(0, m3.BF16, (4,))])
def _(status, s):
    _expect_ok(status)
    assert list(out_u16(s, 0, 4)) == [0x3f80, 0x3f82, 0xbf00, 0x0000]


@case("mul_mixed_right_alias", "tests/test_metal_basic_arithmetic.c:264-313",
      m3.OP_MUL,
      [as_bytes(f32([2.0, -2.0, 0.5, 4.0])),
       as_bytes(u16([0x3fc0, 0xc000, 0x3f00, 0x3e80]))],
      [ViewSpec(0, m3.F32, (4,)), ViewSpec(1, m3.BF16, (4,)),
       ViewSpec(1, m3.F16, (4,))])
def _(status, s):
    _expect_ok(status)
    assert list(out_u16(s, 1, 4)) == [0x4200, 0x4400, 0x3400, 0x3c00]


@case("add_rank_zero", "tests/test_metal_basic_arithmetic.c:350-378",
      m3.OP_ADD,
      [as_bytes(f32([1.5])), as_bytes(f32([2.25])), as_bytes(f32([0.0]))],
      [ViewSpec(0, m3.F32, ()), ViewSpec(1, m3.F32, ()),
       ViewSpec(2, m3.F32, ())])
def _(status, s):
    _expect_ok(status)
    assert out_f32(s, 2, 1)[0] == 3.75


@case("add_empty_broadcast", "tests/test_metal_basic_arithmetic.c:315-349",
      m3.OP_ADD,
      [np.zeros(0, np.uint8), as_bytes(f32([1.0, 2.0, 3.0])),
       np.zeros(0, np.uint8)],
      [ViewSpec(0, m3.F32, (0, 3)), ViewSpec(1, m3.F32, (1, 3)),
       ViewSpec(2, m3.F32, (0, 3))])
def _(status, s):
    _expect_ok(status)


# ---- SOFTMAX ----------------------------------------------------------------

@case("softmax_shifted_in_place", "tests/test_op_sampling.c:36-53",
      m3.OP_SOFTMAX, [as_bytes(f32([1000, 1001]))],
      [ViewSpec(0, m3.F32, (2,)), ViewSpec(0, m3.F32, (2,))])
def _(status, s):
    _expect_ok(status)
    v = out_f32(s, 0, 2)
    assert abs(v[0] - 0.268941432) <= 1e-6 and abs(v[1] - 0.731058598) <= 1e-6


@case("softmax_all_negative_infinity", "tests/test_op_sampling.c:54-67",
      m3.OP_SOFTMAX,
      [as_bytes(f32([-math.inf, -math.inf])), as_bytes(f32([7, 7]))],
      [ViewSpec(0, m3.F32, (2,)), ViewSpec(1, m3.F32, (2,))])
def _(status, s):
    _expect_ok(status)
    assert list(out_f32(s, 1, 2)) == [0.0, 0.0]


@case("softmax_positive_infinity_split", "tests/test_op_sampling.c:68-81",
      m3.OP_SOFTMAX,
      [as_bytes(f32([math.inf, 1, math.inf])), as_bytes(f32([7, 7, 7]))],
      [ViewSpec(0, m3.F32, (3,)), ViewSpec(1, m3.F32, (3,))])
def _(status, s):
    _expect_ok(status)
    assert list(out_f32(s, 1, 3)) == [0.5, 0.0, 0.5]


@case("softmax_nan_rejected_atomically", "tests/test_op_sampling.c:82-96",
      m3.OP_SOFTMAX,
      [as_bytes(f32([0, math.nan])), as_bytes(f32([-7, -7]))],
      [ViewSpec(0, m3.F32, (2,)), ViewSpec(1, m3.F32, (2,))])
def _(status, s):
    assert status == m3.OUT_OF_RANGE
    assert list(out_f32(s, 1, 2)) == [-7.0, -7.0]


@case("softmax_f32_strided_rows", "tests/test_metal_basic_softmax.c:110-158",
      m3.OP_SOFTMAX,
      [as_bytes(f32([1, 2, 3, 4, 91, -3, -1, 0, 2, 92])),
       as_bytes(np.zeros(8, np.float32))],
      [ViewSpec(0, m3.F32, (2, 4), (20, 4)), ViewSpec(1, m3.F32, (2, 4))])
def _(status, s):
    _expect_ok(status)
    v = out_f32(s, 1, 8).astype(np.float64)
    rows = np.array([[1, 2, 3, 4], [-3, -1, 0, 2]], np.float64)
    exact = np.exp(rows - rows.max(1, keepdims=True))
    exact /= exact.sum(1, keepdims=True)
    assert np.all(np.abs(v - exact.reshape(-1)) <=
                  2e-7 + 2e-6 * np.abs(exact.reshape(-1)))
    assert abs(float(np.float32(v[0]) + np.float32(v[1]) + np.float32(v[2]) +
                     np.float32(v[3])) - 1.0) <= 2e-7


@case("softmax_bf16_special_rows", "tests/test_metal_basic_softmax.c:194-240",
      m3.OP_SOFTMAX,
      [as_bytes(u16([0xff80, 0xff80, 0xff80, 0xff80,
                     0x7f80, 0x3f80, 0x7f80, 0xff80])),
       as_bytes(np.full(8, 0xdead, np.uint16))],
      [ViewSpec(0, m3.BF16, (2, 4)), ViewSpec(1, m3.BF16, (2, 4))])
def _(status, s):
    _expect_ok(status)
    assert list(out_u16(s, 1, 8)) == [0, 0, 0, 0, 0x3f00, 0, 0x3f00, 0]


@case("softmax_width_one", "tests/test_metal_basic_softmax.c:359-412",
      m3.OP_SOFTMAX,
      [as_bytes(f32([-math.inf, math.inf, 2.0])), as_bytes(f32([0, 0, 0]))],
      [ViewSpec(0, m3.F32, (3, 1)), ViewSpec(1, m3.F32, (3, 1))])
def _(status, s):
    _expect_ok(status)
    assert list(out_f32(s, 1, 3)) == [0.0, 1.0, 1.0]


@case("softmax_empty_rows", "tests/test_metal_basic_softmax.c:370-385",
      m3.OP_SOFTMAX, [np.zeros(0, np.uint8), np.zeros(0, np.uint8)],
      [ViewSpec(0, m3.F32, (0, 3)), ViewSpec(1, m3.F32, (0, 3))])
def _(status, s):
    _expect_ok(status)


# ---- SNAKE1D ----------------------------------------------------------------

def _bits(value):
    return int(np.float32(value).view(np.uint32))


@case("snake1d_statement_order", "tests/test_vocoder_activations.c:64-136",
      m3.OP_SNAKE1D,
      [as_bytes(bits_f32([0x3e1d90cd, _bits(1.0)])),
       as_bytes(bits_f32([0x3e0b9eef, 0xb089705f])),
       as_bytes(np.zeros(2, np.float32))],
      [ViewSpec(0, m3.F32, (1, 2, 1)), ViewSpec(1, m3.F32, (1, 2, 1)),
       ViewSpec(2, m3.F32, (1, 2, 1))])
def _(status, s):
    _expect_ok(status)
    bits = out_f32(s, 2, 2).view(np.uint32)
    assert int(bits[0]) == 0x3e20def4 and int(bits[1]) == 0x7f800000


@case("snake1d_strided_alpha", "tests/test_vocoder_activations.c:87-168",
      m3.OP_SNAKE1D,
      [as_bytes(f32([0.25, -99, -2, -99, 4, -99, 0.5, -99, 1, -99, 2])),
       as_bytes(np.concatenate([f32([0.0, -99.0]),
                                bits_f32([0xb089705f])])),
       as_bytes(np.zeros(6, np.float32))],
      [ViewSpec(0, m3.F32, (1, 2, 3), (48, 24, 8)),
       ViewSpec(1, m3.F32, (1, 2, 1), (16, 8, 4)),
       ViewSpec(2, m3.F32, (1, 2, 3))])
def _(status, s):
    _expect_ok(status)
    out = out_f32(s, 2, 6)
    assert list(out[:3]) == [0.25, -2.0, 4.0]
    assert [int(b) for b in out[3:].view(np.uint32)] == [0x7f800000] * 3


@case("snake1d_exact_alias", "tests/test_vocoder_activations.c:169-185",
      m3.OP_SNAKE1D,
      [as_bytes(f32([1.0, -2.0, 3.0])), as_bytes(f32([0.0]))],
      [ViewSpec(0, m3.F32, (1, 1, 3)), ViewSpec(1, m3.F32, (1, 1, 1)),
       ViewSpec(0, m3.F32, (1, 1, 3))])
def _(status, s):
    _expect_ok(status)
    assert list(out_f32(s, 0, 3)) == [1.0, -2.0, 3.0]


# ---- TANH -------------------------------------------------------------------

_TANH_IN = bits_f32([0x00000000, 0x80000000, _bits(1.0), _bits(-1.0),
                     0x7f800000, 0xff800000, 0x7fc12345, _bits(0.5)])


@case("tanh_special_bits", "tests/test_vocoder_activations.c:188-236",
      m3.OP_TANH,
      [as_bytes(_TANH_IN), as_bytes(np.zeros(8, np.float32))],
      [ViewSpec(0, m3.F32, (8,)), ViewSpec(1, m3.F32, (8,))])
def _(status, s):
    _expect_ok(status)
    bits = [int(b) for b in out_f32(s, 1, 8).view(np.uint32)]
    assert bits[:6] == [0x00000000, 0x80000000, 0x3f42f7d6, 0xbf42f7d6,
                        0x3f800000, 0xbf800000]
    assert (bits[6] & 0x7f800000) == 0x7f800000 and (bits[6] & 0x7fffff)
    assert bits[7] == 0x3eec9a9f


@case("tanh_exact_in_place", "tests/test_vocoder_activations.c:237-243",
      m3.OP_TANH, [as_bytes(_TANH_IN)],
      [ViewSpec(0, m3.F32, (8,)), ViewSpec(0, m3.F32, (8,))])
def _(status, s):
    _expect_ok(status)
    bits = [int(b) for b in out_f32(s, 0, 8).view(np.uint32)]
    assert bits[1] == 0x80000000 and bits[2] == 0x3f42f7d6


@case("tanh_empty_rank8", "tests/test_vocoder_activations.c:313-340",
      m3.OP_TANH, [np.zeros(0, np.uint8), np.zeros(0, np.uint8)],
      [ViewSpec(0, m3.F32, (0, 1 << 32, 1, 1, 1, 1, 1, 1)),
       ViewSpec(1, m3.F32, (0, 1 << 32, 1, 1, 1, 1, 1, 1))])
def _(status, s):
    _expect_ok(status)


# ---- GATED_SILU -------------------------------------------------------------

@case("gated_silu_strided_f32", "tests/test_metal_dense_norm.c:304-356",
      m3.OP_GATED_SILU,
      [as_bytes(f32([0.0, 91.0, 1.0])), as_bytes(f32([2.0, 92.0, 2.0])),
       as_bytes(np.zeros(2, np.float32))],
      [ViewSpec(0, m3.F32, (2,), (8,)), ViewSpec(1, m3.F32, (2,), (8,)),
       ViewSpec(2, m3.F32, (2,))])
def _(status, s):
    _expect_ok(status)
    out = out_f32(s, 2, 2)
    assert int(out.view(np.uint32)[0]) == 0
    # 2 / (1 + e^-1), within the reference test's 1e-7 tolerance
    assert abs(float(out[1]) - 2.0 / (1.0 + math.exp(-1.0))) <= 2.0e-7


@case("gated_silu_bf16_rounds_activation",
      "tests/test_metal_dense_norm.c:357-377", m3.OP_GATED_SILU,
      [as_bytes(u16([0x3f00])), as_bytes(u16([0x3f40])),
       as_bytes(u16([0]))],
      [ViewSpec(0, m3.BF16, (1,)), ViewSpec(1, m3.BF16, (1,)),
       ViewSpec(2, m3.BF16, (1,))])
def _(status, s):
    _expect_ok(status)
    assert int(out_u16(s, 2, 1)[0]) == 0x3e6e


@case("gated_silu_gate_alias", "tests/test_metal_dense_norm.c:400-409",
      m3.OP_GATED_SILU,
      [as_bytes(u16([0x3f00])), as_bytes(u16([0x3f40]))],
      [ViewSpec(0, m3.BF16, (1,)), ViewSpec(1, m3.BF16, (1,)),
       ViewSpec(0, m3.BF16, (1,))])
def _(status, s):
    _expect_ok(status)
    assert int(out_u16(s, 0, 1)[0]) == 0x3e6e


@case("gated_silu_up_alias_f16", "tests/test_metal_dense_norm.c:378-418",
      m3.OP_GATED_SILU,
      [as_bytes(u16([0x3800])), as_bytes(u16([0x3a00]))],
      [ViewSpec(0, m3.F16, (1,)), ViewSpec(1, m3.F16, (1,)),
       ViewSpec(1, m3.F16, (1,))])
def _(status, s):
    _expect_ok(status)
    # silu(0.5) = 0.31122 rounds to the F16 0x34fb (0.311279296875);
    # times 0.75 = 0.23345947265625 rounds to 0x3378
    assert int(out_u16(s, 1, 1)[0]) == 0x3378


CASE_IDS = [c.name for c in CASES]
