"""Checked inputs produced inside a command list, gated on the device (GPU).

A softmax input, or the input of a float-to-I32 cast, that an earlier
command of the same list writes is checked as the reference CPU provider
checks it, right before its command (src/m3_op_execute_host.c:5-60): the
commands before it run, it and every later command do not, and the list
fails with OUT_OF_RANGE. The HIP provider queues the check on the device
after the producers and lets a failed check close the list's gate, so the
list waits for the host once, at its end. These tests hold the order
semantics (every earlier output written, every later one untouched, the
first failing check decides) and the single wait per run.
"""
import math
import os
import sys

import numpy as np
import pytest

from conftest import m3
from harness import HipFixture, ViewSpec, as_bytes, run_oracle

pytestmark = pytest.mark.gpu


def f32(values):
    return np.asarray(values, dtype=np.float32)


@pytest.fixture()
def hip(gpu):
    fixture = HipFixture()
    yield fixture
    fixture.close()


def values(hip, handle, count, dtype=np.float32):
    return hip.download([handle], [np.empty(count, dtype=dtype)])[0]


def softmax_oracle(row):
    views = [ViewSpec(0, m3.F32, (row.size,)),
             ViewSpec(1, m3.F32, (row.size,))]
    status, out = run_oracle(m3.OP_SOFTMAX, [as_bytes(row),
                                             np.zeros(row.nbytes, np.uint8)],
                             views)
    assert status == m3.OK
    return out[1].view(np.float32)


def test_nan_produced_mid_list_stops_the_rest(hip):
    print("gpu case gate nan_produced_mid_list", file=sys.stderr, flush=True)
    sentinel = f32([-9, -9, -9])
    arrays = [f32([3, 4, 5]), f32([2, 2, 2]), f32([1, math.nan, 1])] + \
        [sentinel.copy() for _ in range(6)]
    h = hip.upload(arrays)
    a, b, c, t1, y1, t2, u, y2, z = hip.views(
        h, [ViewSpec(i, m3.F32, (3,)) for i in range(9)])
    commands = [(m3.OP_ADD, [a, b, t1]),       # produces a clean input
                (m3.OP_SOFTMAX, [t1, y1]),     # its check passes
                (m3.OP_MUL, [c, b, t2]),       # produces a NaN
                (m3.OP_ADD, [a, a, u]),        # before the failing check
                (m3.OP_SOFTMAX, [t2, y2]),     # its check fails
                (m3.OP_MUL, [a, b, z])]        # after it: must not run
    status, message = hip.execute(commands)
    assert status == m3.OUT_OF_RANGE and "NaN" in message, message
    assert list(values(hip, h[3], 3)) == [5, 6, 7]
    assert np.array_equal(values(hip, h[4], 3).view(np.uint32),
                          softmax_oracle(f32([5, 6, 7])).view(np.uint32))
    got = values(hip, h[5], 3)
    assert got[0] == 2 and math.isnan(got[1]) and got[2] == 2
    assert list(values(hip, h[6], 3)) == [6, 8, 10]
    assert list(values(hip, h[7], 3)) == [-9, -9, -9]
    assert list(values(hip, h[8], 3)) == [-9, -9, -9]
    # The next list on the same device is not gated by the failed one.
    status, message = hip.execute([(m3.OP_MUL, [a, b, z])])
    assert status == m3.OK, message
    assert list(values(hip, h[8], 3)) == [6, 8, 10]


def test_first_failing_check_decides(hip):
    """Two produced checks that both fail: the first one in list order is
    reported (a NaN softmax input before an invalid I32 cast input), and
    the command between them does not run."""
    print("gpu case gate first_failing_check", file=sys.stderr, flush=True)
    arrays = [f32([1, math.nan, 2, 3]), f32([1, 1, 1, 1]),
              f32([7, 7, 7, 7]), f32([7, 7, 7, 7]), f32([7, 7, 7, 7]),
              np.array([5, 5, 5, 5], np.int32)]
    h = hip.upload(arrays)
    x, one, t, y, w = hip.views(h[:5], [ViewSpec(i, m3.F32, (4,))
                                        for i in range(5)])
    (i32,) = hip.views([h[5]], [ViewSpec(0, m3.I32, (4,))])
    status, message = hip.execute([(m3.OP_MUL, [x, one, t]),
                                   (m3.OP_SOFTMAX, [t, y]),
                                   (m3.OP_COPY, [x, w]),
                                   (m3.OP_CAST, [w, i32])])
    assert status == m3.OUT_OF_RANGE and "NaN" in message, message
    assert list(values(hip, h[3], 4)) == [7, 7, 7, 7]
    assert list(values(hip, h[4], 4)) == [7, 7, 7, 7]
    assert list(values(hip, h[5], 4, np.int32)) == [5, 5, 5, 5]
    # Only the cast's input is produced and invalid: the cast is reported.
    status, message = hip.execute([(m3.OP_COPY, [x, w]),
                                   (m3.OP_CAST, [w, i32]),
                                   (m3.OP_MUL, [one, one, y])])
    assert status == m3.OUT_OF_RANGE and "I32" in message, message
    got = values(hip, h[4], 4)
    assert got[0] == 1 and math.isnan(got[1])
    assert list(values(hip, h[5], 4, np.int32)) == [5, 5, 5, 5]
    assert list(values(hip, h[3], 4)) == [7, 7, 7, 7]


def attention_graph(shape):
    """scores * scale + mask -> SOFTMAX: the scaled, causally masked scores
    of attention, produced and checked inside one run."""
    rows, width = shape[-2], shape[-1]
    g = m3.Graph()
    scores = g.add_value(m3.INPUT, m3.F32, shape)
    scale = g.add_value(m3.CONSTANT, m3.F32, (1,))
    mask = g.add_value(m3.CONSTANT, m3.F32, (rows, width))
    g.set_constant(scale, np.array([0.125], np.float32))
    causal = np.where(np.triu(np.ones((rows, width), bool), 1), -np.inf,
                      0.0).astype(np.float32)
    g.set_constant(mask, causal)
    t0 = g.add_inferred(m3.OP_MUL, [scores, scale], m3.TEMPORARY, m3.F32)
    g.add_node(m3.OP_MUL, [scores, scale], [t0])
    t1 = g.add_inferred(m3.OP_ADD, [t0, mask], m3.TEMPORARY, m3.F32)
    g.add_node(m3.OP_ADD, [t0, mask], [t1])
    y = g.add_inferred(m3.OP_SOFTMAX, [t1], m3.OUTPUT, m3.F32)
    g.add_node(m3.OP_SOFTMAX, [t1], [y])
    return g, scores, y, causal


def attention_oracle(scores, causal):
    shape = scores.shape
    f = np.float32
    logits = ((scores * f(0.125)).astype(f) + causal).astype(f)
    views = [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, shape)]
    status, out = run_oracle(m3.OP_SOFTMAX, [as_bytes(logits),
                                             np.zeros(logits.nbytes,
                                                      np.uint8)], views)
    assert status == m3.OK
    return out[1].view(np.float32).reshape(shape)


def test_attention_pattern_waits_once_per_run(gpu):
    """The fused scale-and-mask program produces the softmax input; the
    run waits for the host once, the result equals the oracle bit for bit
    (MUL and ADD are single IEEE operations, which numpy float32 fixes), and
    a NaN made by the program (inf * 0 is not reachable with a fixed scale,
    so an inf score plus a -inf mask entry) fails the run with OUT_OF_RANGE
    and leaves the output as it was."""
    print("gpu case gate attention_waits_once", file=sys.stderr, flush=True)
    shape = (2, 64, 96)
    rng = np.random.default_rng(3)
    scores = rng.standard_normal(shape).astype(np.float32) * 3
    g, vin, vout, causal = attention_graph(shape)
    session = m3.Session(g)
    g.free()
    assert all(session.provider(i) == m3.PROVIDER_HIP for i in range(3))
    session.write(vin, scores)
    session.run()
    before = session.host_waits()
    for _ in range(3):
        session.run()
    assert session.host_waits() - before == 3
    out = session.read(vout, np.zeros(shape, np.float32))
    assert np.array_equal(out.view(np.uint32),
                          attention_oracle(scores, causal).view(np.uint32))
    bad = scores.copy()
    bad[1, 5, 70] = np.inf  # column 70 > row 5: the mask adds -inf there
    session.write(vin, bad)
    with pytest.raises(m3.M3Error) as failure:
        session.run()
    assert failure.value.status == m3.OUT_OF_RANGE
    assert "NaN" in failure.value.message
    again = session.read(vout, np.zeros(shape, np.float32))
    assert np.array_equal(again.view(np.uint32), out.view(np.uint32))
    # a clean input afterwards runs again
    session.write(vin, scores)
    session.run()
    out2 = session.read(vout, np.zeros(shape, np.float32))
    assert np.array_equal(out2.view(np.uint32), out.view(np.uint32))
    session.free()


def test_attention_pattern_full_size(gpu):
    """[16, 1024, 1024] causal attention scores through the same graph,
    every element against the oracle."""
    print("gpu case gate attention_full_size", file=sys.stderr, flush=True)
    shape = (16, 1024, 1024)
    scores = m3.rng_fill("normal", int(np.prod(shape)), seed=4,
                         a=3.0).reshape(shape)
    g, vin, vout, causal = attention_graph(shape)
    session = m3.Session(g)
    g.free()
    session.write(vin, scores)
    session.run()
    out = session.read(vout, np.zeros(shape, np.float32))
    session.free()
    expected = attention_oracle(scores, causal)
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))


class environment:
    """Sets environment variables for the sessions created inside."""

    def __init__(self, **values):
        self.values = values
        self.saved = {}

    def __enter__(self):
        for key, value in self.values.items():
            self.saved[key] = os.environ.get(key)
            os.environ[key] = value

    def __exit__(self, *exc):
        for key, value in self.saved.items():
            if value is None:
                del os.environ[key]
            else:
                os.environ[key] = value


def scaled_graph(shape, op, f16):
    """t = (x (op) w) + z, or CAST(x (op) w) to F16 with `f16`, then
    SOFTMAX(t): the two elementwise nodes fuse into one program that writes
    t (a graph output), and the program checks the values it stores for NaN
    in place of a scan of t."""
    g = m3.Graph()
    x = g.add_value(m3.INPUT, m3.F32, shape)
    w = g.add_value(m3.INPUT, m3.F32, shape)
    z = g.add_value(m3.INPUT, m3.F32, shape)
    t0 = g.add_inferred(op, [x, w], m3.TEMPORARY, m3.F32)
    g.add_node(op, [x, w], [t0])
    if f16:
        t = g.add_value(m3.OUTPUT, m3.F16, shape)
        g.add_node(m3.OP_CAST, [t0], [t])
    else:
        t = g.add_inferred(m3.OP_ADD, [t0, z], m3.OUTPUT, m3.F32)
        g.add_node(m3.OP_ADD, [t0, z], [t])
    y = g.add_inferred(m3.OP_SOFTMAX, [t], m3.OUTPUT, m3.F32)
    g.add_node(m3.OP_SOFTMAX, [t], [y])
    return g, x, w, z, t, y


def run_scaled(shape, op, runs, timing=False, generated=True, f16=False):
    """Runs the graph once per (x, w) pair of `runs`, with z = 0, the
    program generated or interpreted; returns, per run, the failure (or
    None), t (as float32), the softmax output and the kernels timed (when
    `timing`)."""
    with environment(M3_HIP_PROGRAM_JIT="1" if generated else "0"):
        return _run_scaled(shape, op, runs, timing, f16)


def _run_scaled(shape, op, runs, timing, f16):
    g, x, w, z, t, y = scaled_graph(shape, op, f16)
    session = m3.Session(g)
    g.free()
    session.write(z, np.zeros(shape, np.float32))
    out_type = np.uint16 if f16 else np.float32
    results = []
    for xs, ws in runs:
        session.write(x, xs)
        session.write(w, ws)
        if timing:
            session.timing_enable(True)
            session.timing_reset()
        try:
            session.run()
            failure = None
        except m3.M3Error as e:
            failure = e
        kernels = session.timing_read() if timing else {}
        if timing:
            session.timing_enable(False)
        traw = session.read(t, np.zeros(shape, out_type))
        tout = traw.view(np.float16).astype(np.float32) if f16 else traw
        yout = session.read(y, np.zeros(shape, np.float32))
        results.append((failure, tout, yout, kernels))
    session.free()
    return results


@pytest.mark.parametrize("generated", [True, False])
def test_fused_check_passes_with_a_tail_lane_that_would_be_nan(gpu,
                                                               generated):
    """15 elements: the program's last group has one lane past the end,
    whose loads are not data; 0 / 0 there is not a stored value and must
    not fail the check. The run passes, makes no separate scan, and both
    outputs equal the oracle."""
    print("gpu case gate fused_tail_clean", generated, file=sys.stderr,
          flush=True)
    shape = (3, 5)
    rng = np.random.default_rng(11)
    xs = (rng.random(shape) + 0.5).astype(np.float32)
    ws = (rng.random(shape) + 0.5).astype(np.float32)
    ((failure, tout, yout, kernels),) = run_scaled(
        shape, m3.OP_DIV, [(xs, ws)], timing=True, generated=generated)
    assert failure is None, failure
    assert not any(name.startswith("m3_scan_f32") or
                   name.startswith("m3_scan_strided") for name in kernels), \
        kernels
    assert ("m3_program" if generated else "m3_program_interpreted") in \
        kernels, kernels
    expected_t = (xs / ws).astype(np.float32) + np.float32(0.0)
    assert np.array_equal(tout.view(np.uint32), expected_t.view(np.uint32))
    for r in range(shape[0]):
        assert np.array_equal(yout[r].view(np.uint32),
                              softmax_oracle(expected_t[r]).view(np.uint32))


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("generated", [True, False])
@pytest.mark.parametrize("where", [0, 7, 14])
def test_fused_check_fails_on_a_stored_nan(gpu, where, generated, f16):
    """A NaN the program stores (0 / 0 at element `where`, the last one of
    the partial group included; F32, or cast to F16 in the program) fails
    the run with OUT_OF_RANGE: the program's output is written in full, the
    softmax output keeps what the clean run before it wrote."""
    print("gpu case gate fused_nan at", where, generated, f16,
          file=sys.stderr, flush=True)
    shape = (3, 5)
    xs = np.ones(shape, np.float32)
    ws = np.full(shape, 2.0, np.float32)
    bad_x = xs.copy()
    bad_w = ws.copy()
    bad_x.reshape(-1)[where] = 0.0
    bad_w.reshape(-1)[where] = 0.0
    clean, bad = run_scaled(shape, m3.OP_DIV, [(xs, ws), (bad_x, bad_w)],
                            generated=generated, f16=f16)
    assert clean[0] is None, clean[0]
    failure, tout, yout, _ = bad
    assert failure is not None and failure.status == m3.OUT_OF_RANGE
    assert "NaN" in failure.message
    flat = tout.reshape(-1)
    assert math.isnan(flat[where])
    assert np.all(np.delete(flat, where) == np.float32(0.5))
    assert np.array_equal(yout.view(np.uint8), clean[2].view(np.uint8))


@pytest.mark.parametrize("generated", [True, False])
def test_fused_check_large_program_output_written_in_full(gpu, generated):
    """A NaN early in a [64, 4096] program output: every group of the
    program is still stored (its waves do not stop at the check), and the
    softmax does not run."""
    print("gpu case gate fused_large", generated, file=sys.stderr,
          flush=True)
    shape = (64, 4096)
    rng = np.random.default_rng(12)
    xs = rng.standard_normal(shape).astype(np.float32)
    ws = rng.standard_normal(shape).astype(np.float32)
    bad_x = xs.copy()
    bad_w = ws.copy()
    bad_x[0, 3] = np.inf
    bad_w[0, 3] = 0.0  # inf * 0 = NaN
    clean, bad = run_scaled(shape, m3.OP_MUL, [(xs, ws), (bad_x, bad_w)],
                            generated=generated)
    assert clean[0] is None, clean[0]
    failure, tout, yout, _ = bad
    assert failure is not None and failure.status == m3.OUT_OF_RANGE
    with np.errstate(invalid="ignore"):
        expected = (bad_x * bad_w).astype(np.float32) + np.float32(0.0)
    assert math.isnan(tout[0, 3])
    mask = ~np.isnan(expected)
    assert np.array_equal(tout[mask].view(np.uint32),
                          expected[mask].view(np.uint32))
    assert np.array_equal(yout.view(np.uint32), clean[2].view(np.uint32))
