"""SUB and DIV of the oracle pinned to their closed form (CPU).

The reference has no SUB or DIV operation; this library adds them as the
same loop as ADD/MUL (src/m3_op_execute_basic.c:61-77) with the other two
IEEE operations: out = round_o(float(l) - float(r)) and
round_o(float(l) / float(r)), one correctly rounded F32 operation. The
checks below hold the oracle to that form independently of its code:

* non-NaN results equal numpy's float32 subtraction and division, which are
  IEEE-754 correctly rounded with round-to-nearest-even and gradual
  underflow (signed zeros, infinities and subnormals included);
* NaN results follow the stated payload rule: a NaN left operand gives its
  own quieted bits (payload and sign kept, bit 22 set); otherwise a NaN
  right operand gives its quieted bits; an invalid operation on non-NaN
  operands (inf - inf, 0 / 0, inf / inf) gives 0xffc00000.
* F16 outputs of non-NaN results equal numpy's float32 -> float16
  conversion (IEEE round-to-nearest-even) of the F32 result.

Two planted mistakes show that the checks bite: the oracle run with its
operands swapped (b - a, b / a, and the right operand's NaN preferred)
must fail them.
"""
import numpy as np
import pytest

from conftest import m3
from harness import ViewSpec, as_bytes, run_oracle

QUIET = np.uint32(0x00400000)
INVALID = np.uint32(0xffc00000)

EDGES = np.array([
    0x00000000, 0x80000000,              # +-0
    0x7f800000, 0xff800000,              # +-inf
    0x00000001, 0x80000001,              # smallest subnormals
    0x007fffff, 0x807fffff,              # largest subnormals
    0x00800000, 0x80800000,              # smallest normals
    0x3f800000, 0xbf800000,              # +-1
    0x7f7fffff, 0xff7fffff,              # +-max
    0x34000000, 0x33800000,              # 2^-23, 2^-24
    0x4b800000, 0x4b800001,              # 2^24, 2^24 + 2
    0x7fc00000, 0xffc00000,              # quiet NaNs
    0x7f800001, 0xff800001,              # signalling NaNs
    0x7fa5a5a5, 0xffdeadbe,              # NaN payloads
], np.uint32)


def operands(seed, count):
    """Random F32 pairs: wide-range normals, subnormals, near-equal pairs
    (cancellation), and every pair of the edge values."""
    rng = np.random.default_rng(seed)
    a = (rng.standard_normal(count) *
         np.exp2(rng.integers(-140, 120, count))).astype(np.float32)
    b = (rng.standard_normal(count) *
         np.exp2(rng.integers(-140, 120, count))).astype(np.float32)
    near = rng.random(count) < 0.1
    b[near] = np.nextafter(a[near], rng.choice([-np.inf, np.inf],
                                               near.sum())).astype(np.float32)
    ab = a.view(np.uint32).copy()
    bb = b.view(np.uint32).copy()
    pick = rng.random(count) < 0.1
    ab[pick] = rng.choice(EDGES, pick.sum())
    pick = rng.random(count) < 0.1
    bb[pick] = rng.choice(EDGES, pick.sum())
    ea, eb = np.meshgrid(EDGES, EDGES, indexing="ij")
    ab = np.concatenate([ab, ea.reshape(-1)])
    bb = np.concatenate([bb, eb.reshape(-1)])
    return ab, bb


def oracle_op(kind, left_bits, right_bits, out_dtype=m3.F32):
    n = left_bits.size
    out_size = m3.DTYPE_SIZES[out_dtype]
    status, storages = run_oracle(
        kind, [as_bytes(left_bits), as_bytes(right_bits),
               np.zeros(n * out_size, np.uint8)],
        [ViewSpec(0, m3.F32, (n,)), ViewSpec(1, m3.F32, (n,)),
         ViewSpec(2, out_dtype, (n,))])
    assert status == m3.OK
    return storages[2].view(np.uint32 if out_size == 4 else np.uint16)


def closed_form_f32(kind, a_bits, b_bits):
    """The F32 result bits that IEEE-754 and the NaN payload rule fix."""
    a = a_bits.view(np.float32)
    b = b_bits.view(np.float32)
    with np.errstate(all="ignore"):
        r = (a - b) if kind == m3.OP_SUB else (a / b)
    bits = r.view(np.uint32).copy()
    a_nan = np.isnan(a)
    b_nan = np.isnan(b) & ~a_nan
    invalid = np.isnan(r) & ~np.isnan(a) & ~np.isnan(b)
    bits[a_nan] = a_bits[a_nan] | QUIET
    bits[b_nan] = b_bits[b_nan] | QUIET
    bits[invalid] = INVALID
    return bits


def mismatches(kind, a_bits, b_bits, got):
    return int(np.count_nonzero(closed_form_f32(kind, a_bits, b_bits) != got))


@pytest.mark.parametrize("kind", [m3.OP_SUB, m3.OP_DIV], ids=["sub", "div"])
def test_oracle_f32_matches_ieee_and_nan_rule(kind):
    a, b = operands(11 + kind, 200_000)
    got = oracle_op(kind, a, b)
    assert mismatches(kind, a, b, got) == 0
    # the edge table holds every class: subnormal results, overflow to
    # infinity, signed zeros and invalid operations all occur
    r = got.view(np.float32)
    assert np.any(np.isinf(r)) and np.any(r == 0) and np.any(np.isnan(r))
    assert np.any((np.abs(r) < np.float32(1.1754944e-38)) & (r != 0))
    assert np.any(got == INVALID)


@pytest.mark.parametrize("kind", [m3.OP_SUB, m3.OP_DIV], ids=["sub", "div"])
def test_oracle_f16_output_rounds_the_f32_result(kind):
    rng = np.random.default_rng(5 + kind)
    a = (rng.standard_normal(50_000) * 300).astype(np.float32)
    b = (rng.standard_normal(50_000) * 3).astype(np.float32)
    b[::97] = 0.0
    got = oracle_op(kind, a.view(np.uint32), b.view(np.uint32), m3.F16)
    with np.errstate(all="ignore"):
        r = (a - b) if kind == m3.OP_SUB else (a / b)
        expected = r.astype(np.float16).view(np.uint16)
    finite = ~np.isnan(r)
    assert np.array_equal(got[finite], expected[finite])


@pytest.mark.parametrize("kind", [m3.OP_SUB, m3.OP_DIV], ids=["sub", "div"])
def test_planted_operand_swap_fails_the_checks(kind):
    """The oracle run as b - a (b / a) must fail the closed form, both on
    ordinary values and on the both-NaN payload rule."""
    a, b = operands(23 + kind, 20_000)
    swapped = oracle_op(kind, b, a)
    assert mismatches(kind, a, b, swapped) > 1000
    both = np.isnan(a.view(np.float32)) & np.isnan(b.view(np.float32)) & \
        ((a | QUIET) != (b | QUIET))
    assert both.sum() > 10
    right_rule = swapped[both]  # what preferring the right NaN would give
    assert np.all(right_rule == (b[both] | QUIET))
    assert np.all(closed_form_f32(kind, a, b)[both] != right_rule)
