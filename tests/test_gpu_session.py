"""The public m3_graph / m3_session API on the HIP provider (GPU).

Graph -> compiler (liveness slots carved from one device arena) ->
write_input (host to device) -> m3_session_run (every node on the session
stream) -> read_output (device to host), checked bit for bit against the
oracle or against numpy where a float32 IEEE operation is the definition.
Each benchmark configuration runs here at a reduced size.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

from conftest import m3
from harness import ViewSpec, as_bytes, run_oracle

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype.itemsize == 4
                                        else np.uint16)


def run_graph(graph, feeds, outputs, **options):
    session = m3.Session(graph, **options)
    graph.free()
    for node in range(session.plan().node_count):
        assert session.provider(node) == m3.PROVIDER_HIP
    for value, array in feeds:
        session.write(value, array)
    session.run()
    results = [session.read(value, np.zeros(shape, dtype))
               for value, shape, dtype in outputs]
    session.free()
    return results


_LIBM = ctypes.CDLL(ctypes.util.find_library("m"))
_LIBM.tanhf.restype = ctypes.c_float
_LIBM.tanhf.argtypes = [ctypes.c_float]


def c_tanhf(values):
    """The C library's tanhf, which the reference calls."""
    return np.array([_LIBM.tanhf(float(v)) for v in values], np.float32)


def test_reference_graph_plan_and_result(gpu):
    """tests/test_graph_runtime.c:87-160 on the GPU: x + c -> tanh -> * c
    -> + x with inferred values; 6 values, 4 nodes, 5 slots, 80 bytes;
    every node on the HIP provider; the C library's tanhf, tolerance
    zero."""
    g = m3.Graph()
    x = g.add_value(m3.INPUT, m3.F32, (4,))
    c = g.add_value(m3.CONSTANT, m3.F32, (4,))
    constant = np.array([0.5, -1.0, 2.0, 3.0], np.float32)
    g.set_constant(c, constant)
    t0 = g.add_inferred(m3.OP_ADD, [x, c], m3.TEMPORARY, m3.F32)
    g.add_node(m3.OP_ADD, [x, c], [t0])
    t1 = g.add_inferred(m3.OP_TANH, [t0], m3.TEMPORARY, m3.F32)
    g.add_node(m3.OP_TANH, [t0], [t1])
    t2 = g.add_inferred(m3.OP_MUL, [t1, c], m3.TEMPORARY, m3.F32)
    g.add_node(m3.OP_MUL, [t1, c], [t2])
    y = g.add_inferred(m3.OP_ADD, [t2, x], m3.OUTPUT, m3.F32)
    g.add_node(m3.OP_ADD, [t2, x], [y])
    session = m3.Session(g)
    g.free()
    plan = session.plan()
    assert (plan.value_count, plan.node_count, plan.storage_slot_count,
            plan.allocated_bytes) == (6, 4, 5, 80)
    assert [session.provider(i) for i in range(4)] == [m3.PROVIDER_HIP] * 4
    data = np.array([1.0, 2.0, -3.0, 0.25], np.float32)
    session.write(x, data)
    session.run()
    out = session.read(y, np.zeros(4, np.float32))
    expected = ((c_tanhf(data + constant) * constant).astype(np.float32)
                + data).astype(np.float32)
    assert np.array_equal(bits(out), bits(expected))
    # repeated runs on unchanged inputs give the same bits
    session.run()
    again = session.read(y, np.zeros(4, np.float32))
    assert np.array_equal(bits(again), bits(expected))
    session.free()


def _random_graph(rng, nodes, shape):
    """A random DAG of ADD/MUL/SUB/DIV over F32 values of `shape` with
    broadcast operands of the trailing size and of size 1."""
    g = m3.Graph()
    values = []
    feeds = []
    for _ in range(3):
        vid = g.add_value(m3.INPUT, m3.F32, shape)
        data = rng.standard_normal(shape).astype(np.float32)
        feeds.append((vid, data))
        values.append((vid, shape, data))
    for cshape in ((shape[-1],), (1,)):
        vid = g.add_value(m3.CONSTANT, m3.F32, cshape)
        data = (rng.standard_normal(cshape) + 3.0).astype(np.float32)
        g.set_constant(vid, data)
        values.append((vid, cshape, data))
    ops = [(m3.OP_ADD, np.add), (m3.OP_MUL, np.multiply),
           (m3.OP_SUB, np.subtract), (m3.OP_DIV, np.divide)]
    outputs = []
    for n in range(nodes):
        kind, fn = ops[rng.integers(len(ops))]
        a = values[rng.integers(len(values))]
        b = values[rng.integers(len(values))]
        out_shape = np.broadcast_shapes(a[1], b[1])
        role = m3.OUTPUT if n == nodes - 1 or rng.random() < 0.15 \
            else m3.TEMPORARY
        vid = g.add_value(role, m3.F32, out_shape)
        with np.errstate(all="ignore"):
            result = fn(np.broadcast_to(a[2], out_shape),
                        np.broadcast_to(b[2], out_shape)).astype(np.float32)
        g.add_node(kind, [a[0], b[0]], [vid])
        values.append((vid, out_shape, result))
        if role == m3.OUTPUT:
            outputs.append((vid, out_shape, result))
    return g, feeds, outputs


@pytest.mark.parametrize("seed", range(6))
def test_random_graphs_reuse_slots_on_device(gpu, seed):
    """Temporaries share arena slots by liveness; no live value is
    overwritten (every output matches numpy's float32 IEEE result)."""
    rng = np.random.default_rng(100 + seed)
    g, feeds, outputs = _random_graph(rng, 40, (6, 37, 40))
    session = m3.Session(g)
    g.free()
    plan = session.plan()
    assert plan.storage_slot_count < plan.value_count
    for vid, data in feeds:
        session.write(vid, data)
    session.run()
    for vid, shape, expected in outputs:
        got = session.read(vid, np.zeros(shape, np.float32))
        finite = np.isfinite(expected)
        assert np.array_equal(bits(got)[finite], bits(expected)[finite]), vid
        assert np.array_equal(np.isnan(got), np.isnan(expected)), vid
    session.free()


def test_mul_broadcast_config(gpu):
    """Broadcast MUL x[8,1024,1536] * c[1536] at reduced size: x ~ U(-1,1)
    times a constant c ~ N(0,1) broadcast over the last axis."""
    shape = (2, 64, 1536)
    x = m3.rng_fill("uniform", int(np.prod(shape)), seed=0, a=-1.0,
                    b=1.0).reshape(shape)
    c = m3.rng_fill("normal", shape[-1], seed=0, sequence=1, a=1.0)
    g = m3.Graph()
    vx = g.add_value(m3.INPUT, m3.F32, shape)
    vc = g.add_value(m3.CONSTANT, m3.F32, shape[-1:])
    vy = g.add_value(m3.OUTPUT, m3.F32, shape)
    g.set_constant(vc, c)
    g.add_node(m3.OP_MUL, [vx, vc], [vy])
    (y,) = run_graph(g, [(vx, x)], [(vy, shape, np.float32)])
    assert np.array_equal(bits(y), bits((x * c).astype(np.float32)))


def _oracle_unary(kind, src, src_dtype, dst_shape, dst_dtype, np_out):
    out = np.zeros(int(np.prod(dst_shape)) * m3.DTYPE_SIZES[dst_dtype],
                   np.uint8)
    status, storages = run_oracle(kind, [as_bytes(src), out],
                                  [ViewSpec(0, src_dtype, src.shape),
                                   ViewSpec(1, dst_dtype, dst_shape)])
    assert status == m3.OK
    return storages[1].view(np_out).reshape(dst_shape)


def test_softmax_causal_config(gpu):
    """Causal softmax of [16,1024,1024] scores at reduced size: logits ~
    N(0,3), strict upper triangle -inf, bit-exact with the oracle (the C
    library's expf)."""
    n = 256
    s = m3.rng_fill("normal", 3 * n * n, seed=0, a=3.0).reshape(3, n, n)
    s[:, np.triu(np.ones((n, n), bool), k=1)] = -np.inf
    g = m3.Graph()
    vi = g.add_value(m3.INPUT, m3.F32, s.shape)
    vo = g.add_value(m3.OUTPUT, m3.F32, s.shape)
    g.add_node(m3.OP_SOFTMAX, [vi], [vo])
    (p,) = run_graph(g, [(vi, s)], [(vo, s.shape, np.float32)])
    expected = _oracle_unary(m3.OP_SOFTMAX, s, m3.F32, s.shape, m3.F32,
                             np.float32)
    assert np.array_equal(bits(p), bits(expected))


def test_softmax_nan_input_is_rejected_until_rewritten(gpu):
    """A NaN in the input makes the run OUT_OF_RANGE and leaves the output
    untouched; a clean rewrite is accepted, and a NaN written later is
    seen again (the device scan result does not outlive a host write)."""
    shape = (8, 64)
    clean = m3.rng_fill("normal", 8 * 64, seed=3, a=2.0).reshape(shape)
    dirty = clean.copy()
    dirty[5, 17] = np.nan
    g = m3.Graph()
    vi = g.add_value(m3.INPUT, m3.F32, shape)
    vo = g.add_value(m3.OUTPUT, m3.F32, shape)
    g.add_node(m3.OP_SOFTMAX, [vi], [vo])
    session = m3.Session(g)
    g.free()
    lib, _ = m3.load()
    session.write(vi, dirty)
    assert lib.m3_session_run(session.handle, None) == m3.OUT_OF_RANGE
    assert not session.read(vo, np.ones(shape, np.float32)).any()
    session.write(vi, clean)
    session.run()
    good = session.read(vo, np.zeros(shape, np.float32))
    expected = _oracle_unary(m3.OP_SOFTMAX, clean, m3.F32, shape, m3.F32,
                             np.float32)
    assert np.array_equal(bits(good), bits(expected))
    session.write(vi, dirty)
    assert lib.m3_session_run(session.handle, None) == m3.OUT_OF_RANGE
    assert np.array_equal(bits(session.read(vo, np.zeros(shape, np.float32))),
                          bits(expected))
    session.free()


@pytest.mark.parametrize("pair", [(m3.F32, m3.F16), (m3.F16, m3.F32),
                                  (m3.F32, m3.BF16), (m3.BF16, m3.F32)])
def test_cast_config(gpu, pair):
    """The F32<->F16/BF16 casts of [4096,4096] at reduced size: normals ~ N(0,
    1e3) with 5% specials (subnormal, signed zeros, infinities, NaN payloads),
    bit-exact."""
    src_dtype, dst_dtype = pair
    n = 256 * 256
    rng = np.random.default_rng(7)
    values = (rng.standard_normal(n) * 1000).astype(np.float32)
    raw = values.view(np.uint32).copy()
    pick = rng.random(n) < 0.05
    specials = np.array([0x00000001, 0x007fffff, 0x80000000, 0x00000000,
                         0x7f800000, 0xff800000, 0x7fc00001, 0x7f800123,
                         0xffa00000], np.uint32)
    raw[pick] = specials[rng.integers(len(specials), size=int(pick.sum()))]
    f32 = raw.view(np.float32).reshape(256, 256)
    if src_dtype == m3.F16:
        src = f32.astype(np.float16).view(np.uint16)
    elif src_dtype == m3.BF16:
        src = (f32.view(np.uint32) >> 16).astype(np.uint16)
    else:
        src = f32
    out_np = np.float32 if dst_dtype == m3.F32 else np.uint16
    g = m3.Graph()
    vi = g.add_value(m3.INPUT, src_dtype, src.shape)
    vo = g.add_value(m3.OUTPUT, dst_dtype, src.shape)
    g.add_node(m3.OP_CAST, [vi], [vo])
    (got,) = run_graph(g, [(vi, src)], [(vo, src.shape, out_np)])
    expected = _oracle_unary(m3.OP_CAST, src, src_dtype, src.shape,
                             dst_dtype, out_np)
    assert np.array_equal(bits(got), bits(expected))


def test_snake_config(gpu):
    """Snake1d of x[2,1536,65536] at reduced size: x ~ N(0,1), alpha ~ U(0.1,
    2) per channel."""
    shape = (2, 48, 4096)
    x = m3.rng_fill("normal", int(np.prod(shape)), seed=0,
                    a=1.0).reshape(shape)
    alpha = m3.rng_fill("uniform", shape[1], seed=0, sequence=1, a=0.1,
                        b=2.0).reshape(1, shape[1], 1)
    g = m3.Graph()
    vx = g.add_value(m3.INPUT, m3.F32, shape)
    va = g.add_value(m3.CONSTANT, m3.F32, alpha.shape)
    vy = g.add_value(m3.OUTPUT, m3.F32, shape)
    g.set_constant(va, alpha)
    g.add_node(m3.OP_SNAKE1D, [vx, va], [vy])
    (y,) = run_graph(g, [(vx, x)], [(vy, shape, np.float32)])
    out = np.zeros(x.nbytes, np.uint8)
    status, storages = run_oracle(
        m3.OP_SNAKE1D, [as_bytes(x), as_bytes(alpha), out],
        [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, alpha.shape),
         ViewSpec(2, m3.F32, shape)])
    assert status == m3.OK
    assert np.array_equal(bits(y), storages[2].view(np.uint32)
                          .reshape(shape))


def test_euler_cfg_graph(gpu):
    """The 30-step Euler CFG graph at reduced size: 4 steps in the reference's
    op order (src/m3_flow_solver_math.c:36-135), constants per step,
    temporaries reusing slots; checked against the same float32 operations in
    numpy."""
    shape = (2, 64, 96)
    count = int(np.prod(shape))
    steps = 4
    rng = m3.rng_new(0, 0)
    x0 = m3.rng_fill("normal", count, seed=0, a=1.0, rng=rng).reshape(shape)
    vus = [m3.rng_fill("normal", count, seed=0, a=1.0, rng=rng)
           .reshape(shape) for _ in range(steps)]
    vcs = [m3.rng_fill("normal", count, seed=0, a=1.0, rng=rng)
           .reshape(shape) for _ in range(steps)]
    scale = np.float32(3.0)
    dt = np.float32(1.0 / 30.0)
    g = m3.Graph()
    vx = g.add_value(m3.INPUT, m3.F32, shape)
    consts = {}
    for name, value in (("minus_one", -1.0), ("scale", scale), ("dt", dt)):
        vid = g.add_value(m3.CONSTANT, m3.F32, (1,))
        g.set_constant(vid, np.array([value], np.float32))
        consts[name] = vid
    current = vx
    expected = x0.copy()
    for k in range(steps):
        vu = g.add_value(m3.CONSTANT, m3.F32, shape)
        vc = g.add_value(m3.CONSTANT, m3.F32, shape)
        g.set_constant(vu, vus[k])
        g.set_constant(vc, vcs[k])
        t = [g.add_value(m3.TEMPORARY, m3.F32, shape) for _ in range(5)]
        nxt = g.add_value(m3.OUTPUT if k == steps - 1 else m3.TEMPORARY,
                          m3.F32, shape)
        g.add_node(m3.OP_MUL, [vu, consts["minus_one"]], [t[0]])
        g.add_node(m3.OP_ADD, [vc, t[0]], [t[1]])
        g.add_node(m3.OP_MUL, [t[1], consts["scale"]], [t[2]])
        g.add_node(m3.OP_ADD, [vu, t[2]], [t[3]])
        g.add_node(m3.OP_MUL, [t[3], consts["dt"]], [t[4]])
        g.add_node(m3.OP_ADD, [current, t[4]], [nxt])
        current = nxt
        a = (vus[k] * np.float32(-1.0)).astype(np.float32)
        a = (vcs[k] + a).astype(np.float32)
        a = (a * scale).astype(np.float32)
        v = (vus[k] + a).astype(np.float32)
        b = (v * dt).astype(np.float32)
        expected = (expected + b).astype(np.float32)
    session = m3.Session(g)
    g.free()
    plan = session.plan()
    assert plan.storage_slot_count < plan.value_count
    session.write(vx, x0)
    session.run()
    y = session.read(current, np.zeros(shape, np.float32))
    assert np.array_equal(bits(y), bits(expected))
    session.free()


def test_gpu_provider_disabled_runs_on_the_cpu_provider(gpu):
    """With the GPU provider disallowed the session keeps host storage and
    runs every node on the CPU provider, as the reference does
    (src/m3_provider.c:35-99); the result is the oracle's, bit for bit,
    and the GPU-provider session of the same graph gives the same bits."""
    rng = np.random.default_rng(77)
    shape = (64, 300)
    logits = (rng.standard_normal(shape) * 3).astype(np.float32)
    outs = []
    for allow_metal in (False, True):
        g = m3.Graph()
        vi = g.add_value(m3.INPUT, m3.F32, shape)
        vo = g.add_value(m3.OUTPUT, m3.F32, shape)
        g.add_node(m3.OP_SOFTMAX, [vi], [vo])
        session = m3.Session(g, allow_metal=allow_metal,
                             allow_neural_engine=False)
        g.free()
        assert session.provider(0) == (m3.PROVIDER_HIP if allow_metal
                                       else m3.PROVIDER_CPU)
        session.write(vi, logits)
        session.run()
        outs.append(session.read(vo, np.zeros(shape, np.float32)))
        session.free()
    status, storages = run_oracle(
        m3.OP_SOFTMAX, [as_bytes(logits), as_bytes(np.zeros_like(logits))],
        [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, shape)])
    assert status == m3.OK
    expected = storages[1].view(np.float32).reshape(shape)
    for out in outs:
        assert np.array_equal(bits(out), bits(expected))


def _mixed_session_outputs(cpu_kinds, shape, seed):
    """x * c -> SOFTMAX -> + x -> TANH -> * c = y, and SOFTMAX(x) = z, with
    the kinds in `cpu_kinds` left to the CPU provider."""
    rng = np.random.default_rng(seed)
    import os
    previous = os.environ.get("M3_HIP_CPU_KINDS")
    if cpu_kinds:
        os.environ["M3_HIP_CPU_KINDS"] = cpu_kinds
    try:
        g = m3.Graph()
        x = g.add_value(m3.INPUT, m3.F32, shape)
        c = g.add_value(m3.CONSTANT, m3.F32, shape[-1:])
        g.set_constant(c, rng.standard_normal(shape[-1:]).astype(np.float32))
        t = [g.add_value(m3.TEMPORARY, m3.F32, shape) for _ in range(4)]
        y = g.add_value(m3.OUTPUT, m3.F32, shape)
        z = g.add_value(m3.OUTPUT, m3.F32, shape)
        g.add_node(m3.OP_MUL, [x, c], [t[0]])
        g.add_node(m3.OP_SOFTMAX, [t[0]], [t[1]])
        g.add_node(m3.OP_ADD, [t[1], x], [t[2]])
        g.add_node(m3.OP_TANH, [t[2]], [t[3]])
        g.add_node(m3.OP_MUL, [t[3], c], [y])
        g.add_node(m3.OP_SOFTMAX, [x], [z])
        session = m3.Session(g)
    finally:
        if previous is None:
            os.environ.pop("M3_HIP_CPU_KINDS", None)
        else:
            os.environ["M3_HIP_CPU_KINDS"] = previous
    g.free()
    providers = [session.provider(n) for n in range(6)]
    results = []
    for _ in range(2):
        session.write(x, (rng.standard_normal(shape) * 2).astype(np.float32))
        session.run()
        results.append([session.read(v, np.zeros(shape, np.float32))
                        for v in (y, z)])
    session.free()
    return providers, results


def test_mixed_gpu_and_cpu_session(gpu):
    """SOFTMAX and TANH on the CPU provider between GPU nodes of one HIP
    session: the CPU nodes run on host mirrors of the device values, with
    one device -> host copy per value they read and one host -> device
    copy per value a GPU node or the caller reads next. Two runs on fresh
    inputs equal the all-GPU session's bits."""
    shape = (96, 1024)
    gpu_providers, expected = _mixed_session_outputs(None, shape, 5)
    providers, results = _mixed_session_outputs("SOFTMAX,TANH", shape, 5)
    assert gpu_providers == [m3.PROVIDER_HIP] * 6
    assert providers == [m3.PROVIDER_HIP, m3.PROVIDER_CPU, m3.PROVIDER_HIP,
                         m3.PROVIDER_CPU, m3.PROVIDER_HIP, m3.PROVIDER_CPU]
    for run, want in zip(results, expected):
        for a, b in zip(run, want):
            assert np.array_equal(bits(a), bits(b))
    assert not np.array_equal(results[0][0], results[1][0])


def test_two_sessions_interleave(gpu):
    """Two sessions (two backends, two streams) alternate runs; each keeps
    its own arena and results."""
    shape = (16, 96)
    graphs = []
    for seed in (11, 12):
        x = m3.rng_fill("normal", 16 * 96, seed=seed, a=2.0).reshape(shape)
        g = m3.Graph()
        vi = g.add_value(m3.INPUT, m3.F32, shape)
        vo = g.add_value(m3.OUTPUT, m3.F32, shape)
        g.add_node(m3.OP_SOFTMAX, [vi], [vo])
        session = m3.Session(g)
        g.free()
        session.write(vi, x)
        graphs.append((session, vi, vo, x))
    for _ in range(3):
        for session, _, _, _ in graphs:
            session.run()
    for session, vi, vo, x in graphs:
        got = session.read(vo, np.zeros(shape, np.float32))
        expected = _oracle_unary(m3.OP_SOFTMAX, x, m3.F32, shape, m3.F32,
                                 np.float32)
        assert np.array_equal(bits(got), bits(expected))
        session.free()


def test_scaled_scores_then_softmax(gpu):
    """A softmax whose input a MUL produces in the same run (attention
    scores times a scale): the MUL runs, its output is scanned on the
    device, and the softmax runs on it, equal to the oracle's MUL then
    softmax bit for bit. With a producer that makes a NaN (inf * 0) the run
    fails with OUT_OF_RANGE and the softmax output keeps its old bits."""
    from harness import ViewSpec, as_bytes, run_oracle
    rng = np.random.default_rng(77)
    shape = (64, 200)
    scores = (rng.standard_normal(shape) * 4).astype(np.float32)
    scale = np.array([0.125], np.float32)
    g = m3.Graph()
    x = g.add_value(m3.INPUT, m3.F32, shape)
    c = g.add_value(m3.INPUT, m3.F32, (1,))
    t = g.add_inferred(m3.OP_MUL, [x, c], m3.TEMPORARY, m3.F32)
    g.add_node(m3.OP_MUL, [x, c], [t])
    y = g.add_inferred(m3.OP_SOFTMAX, [t], m3.OUTPUT, m3.F32)
    g.add_node(m3.OP_SOFTMAX, [t], [y])
    session = m3.Session(g)
    g.free()
    assert [session.provider(i) for i in range(2)] == [m3.PROVIDER_HIP] * 2
    session.write(x, scores)
    session.write(c, scale)
    session.run()
    out = session.read(y, np.zeros(shape, np.float32))
    views = [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, (1,)),
             ViewSpec(2, m3.F32, shape)]
    _, mul = run_oracle(m3.OP_MUL, [as_bytes(scores), as_bytes(scale),
                                    np.zeros(scores.nbytes, np.uint8)], views)
    views = [ViewSpec(0, m3.F32, shape), ViewSpec(1, m3.F32, shape)]
    status, soft = run_oracle(m3.OP_SOFTMAX, [mul[2], np.zeros(
        scores.nbytes, np.uint8)], views)
    assert status == m3.OK
    assert np.array_equal(out.view(np.uint32).reshape(-1),
                          soft[1].view(np.uint32))
    # inf * 0 = NaN reaches the softmax input: the run stops there
    bad = scores.copy()
    bad[3, 7] = np.inf
    session.write(x, bad)
    session.write(c, np.zeros(1, np.float32))
    with pytest.raises(m3.M3Error) as failure:
        session.run()
    assert failure.value.status == m3.OUT_OF_RANGE
    assert "NaN" in failure.value.message
    again = session.read(y, np.zeros(shape, np.float32))
    assert np.array_equal(again.view(np.uint32), out.view(np.uint32))
    session.free()


def test_timing_samples_follow_the_launches(gpu):
    """m3_hip_timing_samples gives one positive duration per launch of a
    kernel, in launch order, and their sum is m3_hip_timing_read's total;
    a reset empties both."""
    shape = (4, 1024, 256)
    x = m3.rng_fill("normal", int(np.prod(shape)), seed=3,
                    a=1.0).reshape(shape)
    g = m3.Graph()
    vx = g.add_value(m3.INPUT, m3.F32, shape)
    vy = g.add_value(m3.OUTPUT, m3.F32, shape)
    g.add_node(m3.OP_TANH, [vx], [vy])
    session = m3.Session(g)
    g.free()
    try:
        session.write(vx, x)
        session.run()
        session.timing_reset()
        session.timing_enable(True)
        for _ in range(3):
            session.run()
        totals = session.timing_read()
        samples = session.timing_samples("m3_tanh")
        session.timing_enable(False)
        assert totals["m3_tanh"][0] == 3
        assert len(samples) == 3 and min(samples) > 0.0
        assert abs(sum(samples) - totals["m3_tanh"][1]) <= \
            1e-6 * max(1.0, totals["m3_tanh"][1])
        assert session.timing_samples("no such kernel") == []
        session.timing_reset()
        assert session.timing_samples("m3_tanh") == []
    finally:
        session.free()


def test_started_scans_of_two_inputs(gpu):
    """Two softmax inputs in separate storages: a write to one starts its
    scan, a write to the other settles that scan and starts its own, and
    every run sees the data it reads; a session freed with a scan still
    started frees cleanly."""
    shape = (16, 256)
    rng_a = m3.rng_fill("normal", 16 * 256, seed=5, a=2.0).reshape(shape)
    rng_b = m3.rng_fill("normal", 16 * 256, seed=6, a=2.0).reshape(shape)
    dirty_a = rng_a.copy()
    dirty_a[3, 100] = np.nan
    g = m3.Graph()
    va = g.add_value(m3.INPUT, m3.F32, shape)
    vb = g.add_value(m3.INPUT, m3.F32, shape)
    oa = g.add_value(m3.OUTPUT, m3.F32, shape)
    ob = g.add_value(m3.OUTPUT, m3.F32, shape)
    g.add_node(m3.OP_SOFTMAX, [va], [oa])
    g.add_node(m3.OP_SOFTMAX, [vb], [ob])
    session = m3.Session(g)
    g.free()
    lib, _ = m3.load()
    want_a = _oracle_unary(m3.OP_SOFTMAX, rng_a, m3.F32, shape, m3.F32,
                           np.float32)
    want_b = _oracle_unary(m3.OP_SOFTMAX, rng_b, m3.F32, shape, m3.F32,
                           np.float32)
    try:
        session.write(va, rng_a)
        session.write(vb, rng_b)
        session.run()  # the first run scans; both views are now watched
        for _ in range(2):
            session.write(va, rng_a)  # starts the scan of a
            session.write(vb, rng_b)  # settles a's, starts b's
            session.run()
            assert np.array_equal(bits(session.read(oa, np.zeros(
                shape, np.float32))), bits(want_a))
            assert np.array_equal(bits(session.read(ob, np.zeros(
                shape, np.float32))), bits(want_b))
        session.write(va, dirty_a)
        session.write(vb, rng_b)
        assert lib.m3_session_run(session.handle, None) == m3.OUT_OF_RANGE
        session.write(va, rng_a)
        session.run()
        assert np.array_equal(bits(session.read(oa, np.zeros(
            shape, np.float32))), bits(want_a))
        session.write(vb, rng_b)  # left started
    finally:
        session.free()
