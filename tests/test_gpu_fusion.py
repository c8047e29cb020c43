"""Fused elementwise runs on the HIP provider (GPU).

The session compiler fuses runs of F32 ADD/SUB/MUL/DIV nodes into
elementwise programs (m3_hip_launch_program), which run as kernels
generated from the program at first use (timed as m3_program) or, with
M3_HIP_PROGRAM_JIT=0, in the interpreter kernel (m3_program_interpreted).
Each test runs the same graph with fusion on and off (M3_HIP_FUSION=0 at
session creation) and requires every OUTPUT to be identical bit for bit,
NaN payloads included; the unfused path is the per-node kernels that the
parity tests pin to the oracle. The CFG + Euler graph is also checked
against the same float32 operations in numpy and must run as one program
launch.
"""
import ctypes
import os

import numpy as np
import pytest

from conftest import m3

pytestmark = pytest.mark.gpu


class environment:
    """Sets environment variables for a block and restores them."""

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


def run_session(build, fusion, generated=True):
    with environment(M3_HIP_FUSION="1" if fusion else "0",
                     M3_HIP_PROGRAM_JIT="1" if generated else "0"):
        g, feeds, outputs = build()
        session = m3.Session(g)
        return _run(session, g, feeds, outputs)


def _run(session, g, feeds, outputs):
    g.free()
    plan = session.plan()
    for node in range(plan.node_count):
        assert session.provider(node) == m3.PROVIDER_HIP
    for vid, data in feeds:
        session.write(vid, data)
    session.timing_reset()
    session.timing_enable(True)
    session.run()
    kernels = session.timing_read()
    session.timing_enable(False)
    results = [session.read(vid, np.zeros(shape, np.float32))
               for vid, shape in outputs]
    # a second run on the same inputs gives the same bits
    session.run()
    again = [session.read(vid, np.zeros(shape, np.float32))
             for vid, shape in outputs]
    for a, b in zip(results, again):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    session.free()
    return results, (plan.storage_slot_count, plan.allocated_bytes), kernels


def specials(rng, shape):
    data = rng.standard_normal(shape).astype(np.float32)
    bits = data.view(np.uint32)
    pick = rng.random(shape)
    payload = rng.integers(1, 1 << 22, shape, dtype=np.uint32)
    sign = rng.integers(0, 2, shape, dtype=np.uint32) << np.uint32(31)
    nan = pick < 0.03
    bits[nan] = (sign | 0x7f800000 | payload)[nan]
    bits[(pick >= 0.03) & (pick < 0.05)] = 0xff800000
    bits[(pick >= 0.05) & (pick < 0.06)] = 0
    bits[(pick >= 0.06) & (pick < 0.07)] = (payload & 0x7fffff)[
        (pick >= 0.06) & (pick < 0.07)]
    return data


def chain_graph(seed, shape, nodes=40):
    """Random elementwise DAG: array and scalar operands, OUTPUT values read
    again, COPY barriers and temporaries read by several nodes."""
    def build():
        rng = np.random.default_rng(seed)
        g = m3.Graph()
        values, feeds, outputs = [], [], []
        for _ in range(3):
            vid = g.add_value(m3.INPUT, m3.F32, shape)
            feeds.append((vid, specials(rng, shape)))
            values.append((vid, shape))
        for _ in range(2):
            vid = g.add_value(m3.CONSTANT, m3.F32, (1,))
            g.set_constant(vid, (rng.standard_normal(1) + 2.0)
                           .astype(np.float32))
            values.append((vid, (1,)))
        kinds = [m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV]
        for n in range(nodes):
            role = m3.OUTPUT if n == nodes - 1 or rng.random() < 0.2 \
                else m3.TEMPORARY
            a = values[rng.integers(len(values))]
            if rng.random() < 0.1:
                out_shape = a[1]
                vid = g.add_value(role, m3.F32, out_shape)
                g.add_node(m3.OP_COPY, [a[0]], [vid])
            else:
                b = values[rng.integers(len(values))]
                out_shape = shape if shape in (a[1], b[1]) else (1,)
                vid = g.add_value(role, m3.F32, out_shape)
                g.add_node(kinds[rng.integers(4)], [a[0], b[0]], [vid])
            values.append((vid, out_shape))
            if role == m3.OUTPUT:
                outputs.append((vid, out_shape))
        return g, feeds, outputs
    return build


@pytest.mark.parametrize("generated", [True, False])
@pytest.mark.parametrize("seed,shape", [(0, (3, 5, 7)), (1, (3, 5, 7)),
                                        (2, (2, 33, 129)),
                                        (3, (4, 1000, 37)),
                                        (4, (1, 1, 4096)), (5, (1,))])
def test_fused_equals_unfused(gpu, seed, shape, generated):
    print("fusion chain graph seed", seed, "shape", shape, "generated",
          generated, flush=True)
    build = chain_graph(2000 + seed, shape)
    fused, plan_on, kernels_on = run_session(build, True, generated)
    plain, plan_off, kernels_off = run_session(build, False)
    assert plan_on == plan_off
    assert "m3_program" not in kernels_off
    assert "m3_program_interpreted" not in kernels_off
    for a, b in zip(fused, plain):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ran = "m3_program" if generated else "m3_program_interpreted"
    other = "m3_program_interpreted" if generated else "m3_program"
    assert other not in kernels_on
    if shape != (1,):
        assert kernels_on.get(ran, (0, 0.0))[0] >= 1


def euler_graph(steps, shape):
    def build():
        rng = m3.rng_new(0, 0)
        count = int(np.prod(shape))
        x0 = m3.rng_fill("normal", count, seed=0, a=1.0,
                         rng=rng).reshape(shape)
        g = m3.Graph()
        vx = g.add_value(m3.INPUT, m3.F32, shape)
        consts = {}
        for name, value in (("m1", -1.0), ("s", 3.0), ("dt", 1.0 / 30.0)):
            vid = g.add_value(m3.CONSTANT, m3.F32, (1,))
            g.set_constant(vid, np.array([value], np.float32))
            consts[name] = vid
        current = vx
        expected = x0.copy()
        for k in range(steps):
            vu_data = m3.rng_fill("normal", count, seed=0, a=1.0,
                                  rng=rng).reshape(shape)
            vc_data = m3.rng_fill("normal", count, seed=0, a=1.0,
                                  rng=rng).reshape(shape)
            vu = g.add_value(m3.CONSTANT, m3.F32, shape)
            vc = g.add_value(m3.CONSTANT, m3.F32, shape)
            g.set_constant(vu, vu_data)
            g.set_constant(vc, vc_data)
            t = [g.add_value(m3.TEMPORARY, m3.F32, shape) for _ in range(5)]
            nxt = g.add_value(m3.OUTPUT if k == steps - 1 else m3.TEMPORARY,
                              m3.F32, shape)
            g.add_node(m3.OP_MUL, [vu, consts["m1"]], [t[0]])
            g.add_node(m3.OP_ADD, [vc, t[0]], [t[1]])
            g.add_node(m3.OP_MUL, [t[1], consts["s"]], [t[2]])
            g.add_node(m3.OP_ADD, [vu, t[2]], [t[3]])
            g.add_node(m3.OP_MUL, [t[3], consts["dt"]], [t[4]])
            g.add_node(m3.OP_ADD, [current, t[4]], [nxt])
            current = nxt
            a = (vu_data * np.float32(-1.0)).astype(np.float32)
            a = (vc_data + a).astype(np.float32)
            a = (a * np.float32(3.0)).astype(np.float32)
            v = (vu_data + a).astype(np.float32)
            b = (v * np.float32(1.0 / 30.0)).astype(np.float32)
            expected = (expected + b).astype(np.float32)
        euler_graph.expected = expected
        return g, [(vx, x0)], [(current, shape)]
    return build


@pytest.mark.parametrize("generated", [True, False])
def test_euler_graph_is_one_program(gpu, generated):
    """30 CFG + Euler steps (src/m3_flow_solver_math.c:36-135) at reduced
    size: one program launch per run, the numpy float32 result bit for bit,
    and the unfused plan's slots and bytes."""
    shape = (2, 64, 96)
    build = euler_graph(30, shape)
    fused, plan_on, kernels = run_session(build, True, generated)
    expected = euler_graph.expected
    plain, plan_off, _ = run_session(build, False)
    name = "m3_program" if generated else "m3_program_interpreted"
    assert plan_on == plan_off
    assert kernels[name][0] == 1
    assert set(kernels) == {name}
    assert np.array_equal(fused[0].view(np.uint32), expected.view(np.uint32))
    assert np.array_equal(plain[0].view(np.uint32), expected.view(np.uint32))


def test_program_words_are_checked_before_launch(gpu):
    """m3_hip_launch_program rejects malformed words on the host (nothing
    is launched): bad magic, operand index out of range, a scalar fetched,
    unknown opcode, and a word count that does not match the header."""
    _, lib = m3.load()
    handle = ctypes.c_void_p()
    msg = ctypes.create_string_buffer(256)
    assert lib.m3_hip_device_open(0, ctypes.byref(handle), msg, 256) == 0
    try:
        def words(operands, code, count=8):
            header = [0x4d335031, len(operands) // 2, len(code),
                      count, 0, 0, 0, 0]
            return np.array(header + operands + code, np.uint32)

        # one array operand at a 16-byte aligned fake address, one scalar
        operands = [0x10000, 0, 0x20001, 0]
        good = words(operands, [0x00000000 | (0 << 2), 0x00,
                                0x1 | (0 << 2) | (0 << 4) | (4 << 8) |
                                (8 << 12) | (1 << 16),
                                0x2 | (0 << 4) | (0 << 8)])
        bad = []
        b = good.copy()
        b[0] = 0
        bad.append(b)
        b = good.copy()
        b[9 + 4] = 0x05  # FETCH operand 5 of 2
        bad.append(b)
        b = good.copy()
        b[9 + 4] = 0x01  # FETCH the scalar
        bad.append(b)
        b = good.copy()
        b[-1] = 0x3  # opcode 3
        bad.append(b)
        for w in bad:
            code = lib.m3_hip_launch_program(
                handle, w.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                ctypes.c_void_p(0x1000), w.size, msg, 256)
            assert code == 1, msg.value  # M3_HIP_INVALID
        code = lib.m3_hip_launch_program(
            handle, good.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
            ctypes.c_void_p(0x1000), good.size - 1, msg, 256)
        assert code == 1
    finally:
        lib.m3_hip_device_close(handle)
