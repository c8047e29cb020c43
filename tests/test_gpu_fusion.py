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


NUMPY_OF = {m3.F32: np.float32, m3.F16: np.uint16, m3.BF16: np.uint16}


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
    results = [session.read(vid, np.zeros(entry[0], entry[1] if len(entry)
                                          > 1 else np.float32))
               for vid, *entry in outputs]
    # a second run on the same inputs gives the same bits
    session.run()
    again = [session.read(vid, np.zeros(entry[0], entry[1] if len(entry)
                                        > 1 else np.float32))
             for vid, *entry in outputs]
    for a, b in zip(results, again):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
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


def narrow(rng, shape, dtype):
    """Random 16-bit patterns: values near 1, NaN payloads (signalling and
    quiet), infinities, zeros and subnormals."""
    data = specials(rng, shape)
    if dtype == m3.BF16:
        return (data.view(np.uint32) >> np.uint32(16)).astype(np.uint16)
    half = data.astype(np.float16).view(np.uint16)
    pick = rng.random(shape)
    half[pick < 0.05] = rng.integers(0x7c01, 0x8000, shape)[pick < 0.05]
    half[(pick >= 0.05) & (pick < 0.07)] = 0x0001
    return half


def mixed_graph(seed, shape, nodes=40):
    """Random elementwise DAG over F32, F16 and BF16 values: binary nodes
    with any float output dtype, CASTs between float dtypes, COPYs, scalar
    operands (F32 and BF16), OUTPUT values read again."""
    def build():
        rng = np.random.default_rng(seed)
        floats = [m3.F32, m3.F16, m3.BF16]
        g = m3.Graph()
        values, feeds, outputs = [], [], []
        for dtype in (m3.F32, m3.F16, m3.BF16, m3.F32):
            vid = g.add_value(m3.INPUT, dtype, shape)
            feeds.append((vid, specials(rng, shape) if dtype == m3.F32
                          else narrow(rng, shape, dtype)))
            values.append((vid, shape, dtype))
        for dtype in (m3.F32, m3.BF16):
            vid = g.add_value(m3.CONSTANT, dtype, (1,))
            constant = (rng.standard_normal(1) + 2.0).astype(np.float32)
            g.set_constant(vid, constant if dtype == m3.F32 else
                           (constant.view(np.uint32) >> np.uint32(16))
                           .astype(np.uint16))
            values.append((vid, (1,), dtype))
        kinds = [m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV]
        for n in range(nodes):
            role = m3.OUTPUT if n == nodes - 1 or rng.random() < 0.2 \
                else m3.TEMPORARY
            a = values[rng.integers(len(values))]
            pick = rng.random()
            if pick < 0.1:
                vid = g.add_value(role, a[2], a[1])
                g.add_node(m3.OP_COPY, [a[0]], [vid])
                entry = (vid, a[1], a[2])
            elif pick < 0.3:
                dtype = floats[rng.integers(3)]
                vid = g.add_value(role, dtype, a[1])
                g.add_node(m3.OP_CAST, [a[0]], [vid])
                entry = (vid, a[1], dtype)
            else:
                b = values[rng.integers(len(values))]
                out_shape = shape if shape in (a[1], b[1]) else (1,)
                dtype = floats[rng.integers(3)]
                vid = g.add_value(role, dtype, out_shape)
                g.add_node(kinds[rng.integers(4)], [a[0], b[0]], [vid])
                entry = (vid, out_shape, dtype)
            values.append(entry)
            if role == m3.OUTPUT:
                outputs.append((entry[0], entry[1], NUMPY_OF[entry[2]]))
        return g, feeds, outputs
    return build


@pytest.mark.parametrize("generated", [True, False])
@pytest.mark.parametrize("seed,shape", [(0, (3, 5, 7)), (1, (2, 33, 129)),
                                        (2, (4, 1000, 37)), (3, (1, 4099)),
                                        (4, (1,))])
def test_fused_mixed_dtypes_equal_unfused(gpu, seed, shape, generated):
    """F16/BF16 loads, stores and scalars, rounding through the output
    dtype and fused CASTs: every OUTPUT byte for byte equal to the per-node
    kernels, NaN payloads included."""
    print("fusion mixed graph seed", seed, "shape", shape, "generated",
          generated, flush=True)
    build = mixed_graph(4000 + seed, shape)
    fused, plan_on, kernels_on = run_session(build, True, generated)
    plain, plan_off, kernels_off = run_session(build, False)
    assert plan_on == plan_off
    for a, b in zip(fused, plain):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    ran = "m3_program" if generated else "m3_program_interpreted"
    if shape != (1,):
        assert kernels_on.get(ran, (0, 0.0))[0] >= 1


def broadcast_graph(seed, full, nodes=40):
    """Random elementwise DAG over `full` = (A, B, C) whose operands are
    broadcast from smaller tensors: along trailing axes ((C,), (1, C),
    (B, C), (1, B, C)), which programs read periodically, and along others
    ((A, 1, C), (A, B, 1), (B, 1)), which stay per-node kernels; F16 and
    BF16 values and scalars among them."""
    a_, b_, c_ = full
    shapes = [full, (c_,), (1, c_), (b_, c_), (1, b_, c_), (a_, 1, c_),
              (a_, b_, 1), (b_, 1), (1,)]

    def build():
        rng = np.random.default_rng(seed)
        floats = [m3.F32, m3.F16, m3.BF16]
        g = m3.Graph()
        values, feeds, outputs = [], [], []
        for shape in shapes:
            for dtype in (m3.F32, floats[1 + rng.integers(2)]):
                vid = g.add_value(m3.INPUT, dtype, shape)
                feeds.append((vid, specials(rng, shape) if dtype == m3.F32
                              else narrow(rng, shape, dtype)))
                values.append((vid, shape, dtype))
        kinds = [m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV]
        for n in range(nodes):
            role = m3.OUTPUT if n == nodes - 1 or rng.random() < 0.2 \
                else m3.TEMPORARY
            produced = [v for v in values[2 * len(shapes):] if v[1] == full]
            pool = produced if produced and rng.random() < 0.7 else values
            a = pool[rng.integers(len(pool))]
            b = values[rng.integers(len(values))]
            if rng.random() < 0.5:
                a, b = b, a
            out_shape = tuple(np.broadcast_shapes(a[1], b[1]))
            dtype = floats[rng.integers(3)] if rng.random() < 0.3 \
                else m3.F32
            vid = g.add_value(role, dtype, out_shape)
            g.add_node(kinds[rng.integers(4)], [a[0], b[0]], [vid])
            entry = (vid, out_shape, dtype)
            values.append(entry)
            if role == m3.OUTPUT:
                outputs.append((vid, out_shape, NUMPY_OF[dtype]))
        return g, feeds, outputs
    return build


@pytest.mark.parametrize("generated", [True, False])
@pytest.mark.parametrize("seed,full", [(0, (3, 4, 8)), (1, (2, 33, 132)),
                                       (2, (4, 96, 1536))])
def test_fused_broadcasts_equal_unfused(gpu, seed, full, generated):
    """Operands broadcast along trailing axes, read periodically inside
    programs, give every OUTPUT byte for byte equal to the per-node
    kernels, NaN payloads included."""
    print("fusion broadcast graph seed", seed, "shape", full, "generated",
          generated, flush=True)
    build = broadcast_graph(6000 + seed, full)
    fused, plan_on, kernels_on = run_session(build, True, generated)
    plain, plan_off, _ = run_session(build, False)
    assert plan_on == plan_off
    for a, b in zip(fused, plain):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    ran = "m3_program" if generated else "m3_program_interpreted"
    assert kernels_on.get(ran, (0, 0.0))[0] >= 1


def scale_shift_graph(shape):
    """y = bf16((x * scale + shift) * gate) with per-channel scale and
    shift [C] and a per-position gate [L, C] over x [N, L, C]."""
    def build():
        rng = np.random.default_rng(11)
        n, length, channels = shape
        x = specials(rng, shape)
        scale = rng.standard_normal(channels).astype(np.float32)
        shift = rng.standard_normal((1, channels)).astype(np.float32)
        gate = rng.standard_normal((length, channels)).astype(np.float32)
        g = m3.Graph()
        vx = g.add_value(m3.INPUT, m3.F32, shape)
        vs = g.add_value(m3.CONSTANT, m3.F32, (channels,))
        vb = g.add_value(m3.CONSTANT, m3.F32, (1, channels))
        vg = g.add_value(m3.INPUT, m3.F32, (length, channels))
        g.set_constant(vs, scale)
        g.set_constant(vb, shift)
        t0 = g.add_value(m3.TEMPORARY, m3.F32, shape)
        t1 = g.add_value(m3.TEMPORARY, m3.F32, shape)
        t2 = g.add_value(m3.TEMPORARY, m3.F32, shape)
        vy = g.add_value(m3.OUTPUT, m3.BF16, shape)
        g.add_node(m3.OP_MUL, [vx, vs], [t0])
        g.add_node(m3.OP_ADD, [t0, vb], [t1])
        g.add_node(m3.OP_MUL, [t1, vg], [t2])
        g.add_node(m3.OP_CAST, [t2], [vy])
        f = np.float32
        with np.errstate(invalid="ignore", over="ignore"):
            y = ((x * scale).astype(f) + shift).astype(f)
            y = (y * gate).astype(f)
        scale_shift_graph.expected = y
        return g, [(vx, x), (vg, gate)], [(vy, shape, np.uint16)]
    return build


def bf16_bits(values):
    """float32 -> bfloat16 bits, round to nearest even, NaNs quieted (the
    CAST's conversion)."""
    bits = values.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7fff + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(values)
    rounded[nan] = ((bits[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


@pytest.mark.parametrize("generated", [True, False])
def test_scale_shift_gate_is_one_program(gpu, generated):
    """A per-channel scale and shift and a per-position gate read
    periodically: the four nodes run as one program launch whose output
    equals the float32 numpy operations rounded to bfloat16."""
    shape = (4, 256, 1536)
    print("fusion scale/shift/gate", shape, "generated", generated,
          flush=True)
    build = scale_shift_graph(shape)
    fused, plan_on, kernels = run_session(build, True, generated)
    plain, plan_off, _ = run_session(build, False)
    name = "m3_program" if generated else "m3_program_interpreted"
    assert plan_on == plan_off
    assert kernels[name][0] == 1 and set(kernels) == {name}
    expected = bf16_bits(scale_shift_graph.expected)
    assert np.array_equal(fused[0], expected)
    assert np.array_equal(plain[0], expected)


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
    a rounding dtype out of range in OP and in ROUND, an operand dtype out
    of range, a misaligned 16-bit array, a word count that does not match
    the header, and period tables that break the rules (more entries than
    operands, a period that is zero, not a multiple of 4 or does not
    divide the count, an index out of range, a scalar or STORE target made
    periodic, indices not increasing). Every address in the words, and the device copy of
    the words, is real device memory, so a case the check missed would
    still only touch memory of this test; the valid words run once."""
    _, lib = m3.load()
    vp, sz, cp = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_char_p
    lib.m3_hip_arena_reserve.argtypes = [vp, sz, ctypes.POINTER(vp), cp, sz]
    lib.m3_hip_arena_release.argtypes = [vp, vp]
    lib.m3_hip_fill_zero.argtypes = [vp, vp, sz, cp, sz]
    lib.m3_hip_copy_h2d.argtypes = [vp, vp, vp, sz, cp, sz]
    handle = ctypes.c_void_p()
    base = ctypes.c_void_p()
    msg = ctypes.create_string_buffer(256)
    assert lib.m3_hip_device_open(0, ctypes.byref(handle), msg, 256) == 0
    try:
        assert lib.m3_hip_arena_reserve(handle, 65536, ctypes.byref(base),
                                        msg, 256) == 0, msg.value
        assert lib.m3_hip_fill_zero(handle, base, 65536, msg, 256) == 0
        array = base.value + 4096      # 8 F32 elements
        scalar = base.value + 8192     # one F32
        device_words = ctypes.c_void_p(base.value + 16384)

        def words(operands, code, count=8, periods=()):
            header = [0x4d335031, len(operands) // 2, len(code),
                      count, 0, len(periods) // 2, 0, 0]
            return np.array(header + operands + list(periods) + code,
                            np.uint32)

        def address(at, flags=0, dtype=0):
            return [(at & 0xffffffff) | flags, (at >> 32) | (dtype << 30)]

        # R0 = F0 * scalar, stored back to the array
        operands = address(array) + address(scalar, flags=1)
        good = words(operands, [0x00000000 | (0 << 2), 0x00,
                                0x1 | (1 << 2) | (0 << 4) | (4 << 8) |
                                (8 << 12) | (1 << 16),
                                0x2 | (0 << 4) | (0 << 8)])
        assert lib.m3_hip_copy_h2d(
            handle, device_words, good.ctypes.data_as(ctypes.c_void_p),
            good.nbytes, msg, 256) == 0
        bad = []
        b = good.copy()
        b[0] = 0
        bad.append(b)
        b = good.copy()
        b[13] = 0x05  # FETCH operand 5 of 2
        bad.append(b)
        b = good.copy()
        b[13] = 0x01  # FETCH the scalar
        bad.append(b)
        b = good.copy()
        b[14] |= 3 << 24  # OP rounding dtype 3
        bad.append(b)
        b = good.copy()
        b[15] = 0x3 | (3 << 24)  # ROUND with dtype 3
        bad.append(b)
        b = good.copy()
        b[9] |= 3 << 30  # operand dtype 3
        bad.append(b)
        b = good.copy()
        b[8:10] = address(array + 4, dtype=1)  # F16 array not 8-aligned
        bad.append(b)
        for index, w in enumerate(bad):
            code = lib.m3_hip_launch_program(
                handle, w.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                device_words, w.size, msg, 256)
            assert code == 1, (index, msg.value)  # M3_HIP_INVALID
        code = lib.m3_hip_launch_program(
            handle, good.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
            device_words, good.size - 1, msg, 256)
        assert code == 1
        code = lib.m3_hip_launch_program(
            handle, good.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
            device_words, good.size, msg, 256)
        assert code == 0, msg.value
        assert lib.m3_hip_synchronize(handle, msg, 256) == 0, msg.value

        # periodic operand: array[e] = array[e] * period4[e mod 4]
        period4 = base.value + 6144    # 4 F32 elements
        operands = address(array) + address(period4)
        periodic = words(operands, [0x0 | (1 << 2), 0x0100,
                                    0x1 | (1 << 2) | (0 << 4) | (4 << 8) |
                                    (5 << 12),
                                    0x2 | (0 << 4) | (0 << 8)],
                         periods=[1, 4])
        assert lib.m3_hip_copy_h2d(
            handle, device_words, periodic.ctypes.data_as(ctypes.c_void_p),
            periodic.nbytes, msg, 256) == 0
        bad = []
        for at, value in ((5, 3),          # more periodic operands than P
                          (13, 6),         # period not a multiple of 4
                          (13, 16),        # period does not divide count
                          (13, 0),         # period zero
                          (12, 2),         # operand index out of range
                          (17, 0x2 | (1 << 8))):  # STORE to the periodic
            b = periodic.copy()
            b[at] = value
            bad.append(b)
        b = periodic.copy()
        b[10] |= 1  # the periodic operand flagged scalar
        bad.append(b)
        bad.append(words(operands + address(period4),
                         [0x0 | (1 << 2), 0x0100, 0x1 | (4 << 8) | (5 << 12),
                          0x2], periods=[2, 4, 1, 4]))  # not increasing
        for index, w in enumerate(bad):
            code = lib.m3_hip_launch_program(
                handle, w.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                device_words, w.size, msg, 256)
            assert code == 1, ("periodic", index, msg.value)
        x = np.arange(1, 9, dtype=np.float32)
        p = np.array([2.0, -1.0, 0.5, 3.0], np.float32)
        for data, at in ((x, array), (p, period4)):
            assert lib.m3_hip_copy_h2d(
                handle, ctypes.c_void_p(at),
                data.ctypes.data_as(ctypes.c_void_p), data.nbytes, msg,
                256) == 0
        code = lib.m3_hip_launch_program(
            handle, periodic.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
            device_words, periodic.size, msg, 256)
        assert code == 0, msg.value
        got = np.zeros(8, np.float32)
        lib.m3_hip_copy_d2h.argtypes = [vp, vp, vp, sz, cp, sz]
        assert lib.m3_hip_copy_d2h(
            handle, got.ctypes.data_as(ctypes.c_void_p),
            ctypes.c_void_p(array), got.nbytes, msg, 256) == 0, msg.value
        assert np.array_equal(got, x * np.tile(p, 2))
    finally:
        if base.value:
            lib.m3_hip_arena_release(handle, base)
        lib.m3_hip_device_close(handle)


def consumer_graph(consumer, shape):
    """x * scale + bias feeding a node that never fuses (the scale + mask
    -> softmax and x * w + b -> tanh patterns; Snake1d and GATED_SILU read
    two values)."""
    def build():
        rng = np.random.default_rng(17)
        g = m3.Graph()
        x = g.add_value(m3.INPUT, m3.F32, shape)
        x_data = rng.standard_normal(shape).astype(np.float32)
        scale = g.add_value(m3.CONSTANT, m3.F32, (1,))
        g.set_constant(scale, np.array([0.125], np.float32))
        bias = g.add_value(m3.CONSTANT, m3.F32, shape[-1:])
        g.set_constant(bias, rng.standard_normal(shape[-1:])
                       .astype(np.float32))
        t0 = g.add_value(m3.TEMPORARY, m3.F32, shape)
        t1 = g.add_value(m3.TEMPORARY, m3.F32, shape)
        g.add_node(m3.OP_MUL, [x, scale], [t0])
        g.add_node(m3.OP_ADD, [t0, bias], [t1])
        y = g.add_value(m3.OUTPUT, m3.F32, shape)
        if consumer == m3.OP_SNAKE1D:
            alpha = g.add_value(m3.CONSTANT, m3.F32, (1, shape[1], 1))
            g.set_constant(alpha, rng.uniform(0.1, 2.0, (1, shape[1], 1))
                           .astype(np.float32))
            g.add_node(m3.OP_SNAKE1D, [t1, alpha], [y])
        elif consumer == m3.OP_GATED_SILU:
            g.add_node(m3.OP_GATED_SILU, [t1, x], [y])
        else:
            g.add_node(consumer, [t1], [y])
        return g, [(x, x_data)], [(y, shape)]
    return build


@pytest.mark.parametrize("generated", [True, False])
@pytest.mark.parametrize("consumer", ["SOFTMAX", "TANH", "SNAKE1D",
                                      "GATED_SILU"])
def test_value_read_by_an_unfused_kind_is_stored(gpu, consumer, generated):
    """The fused MUL + ADD program stores the temporary that its
    non-fusing reader needs: fused equals unfused bit for bit, as one
    program launch plus the reader's kernel."""
    kind = getattr(m3, "OP_" + consumer)
    shape = (4, 96, 1024) if kind == m3.OP_SNAKE1D else (384, 1024)
    build = consumer_graph(kind, shape)
    fused, plan_on, kernels = run_session(build, True, generated)
    plain, plan_off, _ = run_session(build, False)
    assert plan_on == plan_off
    assert sum(launches for name, (launches, _) in kernels.items()
               if name.startswith("m3_program")) == 1, kernels
    assert np.array_equal(fused[0].view(np.uint32),
                          plain[0].view(np.uint32))


def periodic_slot_graph(rows):
    """x = c + d ([4]) takes the 16 * rows-byte slot a finished [rows, 4]
    value left; z = y + x reads x as a trailing broadcast and t = z * a is
    planned into the same slot once x is dead. A program storing t there
    would overwrite x while other lanes still read x[e mod 4]."""
    def build():
        rng = np.random.default_rng(3)
        shape = (rows, 4)
        g = m3.Graph()
        a, b, y = (g.add_value(m3.INPUT, m3.F32, shape) for _ in range(3))
        c = g.add_value(m3.CONSTANT, m3.F32, (4,))
        d = g.add_value(m3.CONSTANT, m3.F32, (4,))
        g.set_constant(c, rng.standard_normal(4).astype(np.float32))
        g.set_constant(d, rng.standard_normal(4).astype(np.float32))
        p = g.add_value(m3.TEMPORARY, m3.F32, shape)
        q = g.add_value(m3.OUTPUT, m3.F32, shape)
        x = g.add_value(m3.TEMPORARY, m3.F32, (4,))
        z = g.add_value(m3.TEMPORARY, m3.F32, shape)
        t = g.add_value(m3.TEMPORARY, m3.F32, shape)
        out = g.add_value(m3.OUTPUT, m3.F32, shape)
        g.add_node(m3.OP_MUL, [a, b], [p])
        g.add_node(m3.OP_SOFTMAX, [p], [q])
        g.add_node(m3.OP_ADD, [c, d], [x])
        g.add_node(m3.OP_ADD, [y, x], [z])
        g.add_node(m3.OP_MUL, [z, a], [t])
        g.add_node(m3.OP_TANH, [t], [out])
        feeds = [(v, rng.standard_normal(shape).astype(np.float32))
                 for v in (a, b, y)]
        return g, feeds, [(q, shape), (out, shape)]
    return build


def narrow_slot_graph(rows, width):
    """A softmax output s (F32) is read by a fused MUL + CAST whose F16
    result h is planned into s's slot once s is dead: lane e's store of h
    covers bytes of s[e / 2], which another lane reads."""
    def build():
        rng = np.random.default_rng(4)
        shape = (rows, width)
        g = m3.Graph()
        x = g.add_value(m3.INPUT, m3.F32, shape)
        w = g.add_value(m3.INPUT, m3.F32, shape)
        s = g.add_value(m3.TEMPORARY, m3.F32, shape)
        u = g.add_value(m3.TEMPORARY, m3.F32, shape)
        h = g.add_value(m3.TEMPORARY, m3.F16, shape)
        out = g.add_value(m3.OUTPUT, m3.F32, shape)
        g.add_node(m3.OP_SOFTMAX, [x], [s])
        g.add_node(m3.OP_MUL, [s, w], [u])
        g.add_node(m3.OP_CAST, [u], [h])
        g.add_node(m3.OP_SOFTMAX, [h], [out])
        feeds = [(x, rng.standard_normal(shape).astype(np.float32)),
                 (w, rng.standard_normal(shape).astype(np.float32))]
        return g, feeds, [(out, shape)]
    return build


@pytest.mark.parametrize("generated", [True, False])
@pytest.mark.parametrize("graph", ["periodic", "narrow"])
def test_fused_stores_never_land_on_operands_other_lanes_read(gpu, graph,
                                                              generated):
    """Slots shared by liveness never put a program's store on an operand
    that other lanes still read: such runs stay unfused, and the results
    equal the unfused run's bit for bit."""
    build = periodic_slot_graph(1 << 16) if graph == "periodic" \
        else narrow_slot_graph(512, 1024)
    fused, plan_on, kernels = run_session(build, True, generated)
    plain, plan_off, _ = run_session(build, False)
    assert plan_on == plan_off
    assert not any(k.startswith("m3_program") for k in kernels), kernels
    for a, b in zip(fused, plain):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
