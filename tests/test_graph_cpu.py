"""Graph builder, session compiler, liveness planner and scheduler (CPU).

libm3.so runs unchanged; the scheduler's GPU backend constructor is
replaced (m3_provider_set_gpu_factory) by a test backend over host memory
that evaluates commands with the oracle (tests/csrc/oracle_backend.c).
Restates the reference's graph tests (tests/test_graph_runtime.c:87-248)
and adds brute-force checks of the liveness plan on random graphs.
"""
import ctypes
import ctypes.util
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT, m3

BUILD = os.path.join(ROOT, "tests", "_build")
# The sanitizer run (tests/test_sanitize_cpu.py) links the test backend
# with the same sanitizers against the sanitized host layer.
SANITIZE = os.environ.get("M3_SANITIZE") == "1"
LIB_DIR = os.environ.get("M3_LIBRARY_DIR", os.path.join(ROOT, "m3.c_amd"))
LIB = os.path.join(BUILD, "liboracle_backend%s.so" %
                   ("_sanitize" if SANITIZE else ""))


def _build_backend():
    os.makedirs(BUILD, exist_ok=True)
    sources = [os.path.join(ROOT, "tests", "csrc", "oracle_backend.c"),
               os.path.join(ROOT, "oracle", "m3_oracle.c")]
    flags = (["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
              "-fno-omit-frame-pointer", "-g"] if SANITIZE else [])
    subprocess.run(["gcc", "-std=c11", "-O2", "-fPIC", "-shared",
                    "-ffp-contract=off", "-mfma", "-D_POSIX_C_SOURCE=200809L",
                    "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "oracle")] + flags + sources +
                   ["-L", LIB_DIR, "-lm3", "-Wl,-rpath," + LIB_DIR, "-lm",
                    "-o", LIB], check=True)


@pytest.fixture(scope="module")
def backend_lib():
    lib, _ = m3.load()
    _build_backend()
    fake = ctypes.CDLL(LIB)
    fake.oracle_backend_log.restype = ctypes.c_size_t
    fake.oracle_backend_log.argtypes = [ctypes.POINTER(ctypes.c_int),
                                        ctypes.POINTER(ctypes.c_int),
                                        ctypes.c_size_t]
    fake.oracle_backend_lists.restype = ctypes.c_size_t
    fake.oracle_backend_reserved.restype = ctypes.c_size_t
    fake.oracle_backend_fail_allocation_at.argtypes = [ctypes.c_size_t]
    fake.oracle_backend_programs.restype = ctypes.c_size_t
    fake.oracle_backend_periodic.restype = ctypes.c_size_t
    fake.oracle_backend_set_program_order.argtypes = [ctypes.c_int]
    fake.oracle_backend_set_create_status.argtypes = [ctypes.c_int]
    fake.oracle_backend_fail_list_at.argtypes = [ctypes.c_size_t,
                                                 ctypes.c_int]
    factory = ctypes.cast(fake.oracle_backend_create, ctypes.c_void_p)
    lib.m3_provider_set_gpu_factory.argtypes = [ctypes.c_void_p]
    lib.m3_provider_set_gpu_factory(factory)
    yield fake
    lib.m3_provider_set_gpu_factory(None)


@pytest.fixture()
def fake(backend_lib):
    backend_lib.oracle_backend_reset()
    return backend_lib


def log_of(fake):
    kinds = (ctypes.c_int * 4096)()
    lists = (ctypes.c_int * 4096)()
    count = fake.oracle_backend_log(kinds, lists, 4096)
    return list(kinds[:count]), list(lists[:count])


def reference_graph():
    """tests/test_graph_runtime.c:30-85: x + c -> tanh -> * c -> + x, every
    later value added by shape inference."""
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
    return g, x, y, constant


_LIBM = ctypes.CDLL(ctypes.util.find_library("m"))
_LIBM.tanhf.restype = ctypes.c_float
_LIBM.tanhf.argtypes = [ctypes.c_float]


def c_tanhf(values):
    """The C library's tanhf, which the reference calls."""
    return np.array([_LIBM.tanhf(float(v)) for v in values], np.float32)


def test_liveness_plan_kat_and_execution(fake):
    g, x, y, constant = reference_graph()
    session = m3.Session(g, allow_neural_engine=False)
    g.free()
    plan = session.plan()
    assert (plan.value_count, plan.node_count, plan.storage_slot_count,
            plan.allocated_bytes) == (6, 4, 5, 80)
    assert fake.oracle_backend_reserved() == 5 * 256
    assert [session.provider(i) for i in range(4)] == [m3.PROVIDER_HIP] * 4
    data = np.array([1.0, 2.0, -3.0, 0.25], np.float32)
    session.write(x, data)
    session.run()
    out = session.read(y, np.zeros(4, np.float32))
    # tests/test_graph_runtime.c:139-146, tolerance zero
    expected = ((c_tanhf(data + constant) * constant).astype(np.float32)
                + data).astype(np.float32)
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))
    kinds, lists = log_of(fake)
    assert kinds == [m3.OP_ADD, m3.OP_TANH, m3.OP_MUL, m3.OP_ADD]
    assert lists == [0, 0, 0, 0]  # one partition, one list per run
    session.free()


def test_session_io_contracts(fake):
    g, x, y, _ = reference_graph()
    session = m3.Session(g)
    data = np.zeros(4, np.float32)
    lib, _ = m3.load()
    ptr = data.ctypes.data_as(ctypes.c_void_p)
    assert lib.m3_session_write_input(session.handle, y, ptr, 16,
                                      None) == m3.INVALID_ARGUMENT
    assert lib.m3_session_read_output(session.handle, x, ptr, 16,
                                      None) == m3.INVALID_ARGUMENT
    assert lib.m3_session_write_input(session.handle, x, ptr, 15,
                                      None) == m3.INVALID_ARGUMENT
    assert lib.m3_session_write_input(session.handle, 99, ptr, 16,
                                      None) == m3.OUT_OF_RANGE
    error = m3.Error()
    node = ctypes.c_int()
    assert lib.m3_session_get_node_provider(session.handle, 4,
                                            ctypes.byref(node),
                                            ctypes.byref(error)) == \
        m3.OUT_OF_RANGE
    session.free()


def _session_status(graph, options=None):
    lib, _ = m3.load()
    handle = ctypes.c_void_p()
    error = m3.Error()
    opts = None
    if options is not None:
        opts = ctypes.byref(m3.SessionOptions(*options))
    status = lib.m3_session_create(ctypes.byref(handle), graph.handle, opts,
                                   ctypes.byref(error))
    if handle:
        lib.m3_session_free(handle)
    return status, bool(handle.value), error.text()


def test_graph_validation_rejects_atomically(fake):
    g = m3.Graph()
    x = g.add_value(m3.INPUT, m3.F32, (2,))
    t = g.add_value(m3.TEMPORARY, m3.F32, (2,))
    y = g.add_value(m3.OUTPUT, m3.F32, (2,))
    g.add_node(m3.OP_ADD, [t, x], [y])
    status, made, _ = _session_status(g)
    assert status == m3.INVALID_ARGUMENT and not made
    lib, _ = m3.load()
    node = m3.NodeDesc()
    lib.m3_graph_node_desc_init(ctypes.byref(node), m3.OP_ADD)
    node.inputs[1] = x
    inferred = ctypes.c_uint32(m3.VALUE_NONE)
    assert lib.m3_graph_add_inferred_value(
        g.handle, ctypes.byref(node), 0, m3.TEMPORARY, m3.F32,
        ctypes.byref(inferred), None) == m3.OUT_OF_RANGE
    assert inferred.value == m3.VALUE_NONE
    node.kind = 999
    node.inputs[0] = x
    assert lib.m3_graph_add_inferred_value(
        g.handle, ctypes.byref(node), 0, m3.TEMPORARY, m3.F32,
        ctypes.byref(inferred), None) == m3.UNSUPPORTED
    g.free()

    g = m3.Graph()
    c = g.add_value(m3.CONSTANT, m3.F32, (2,))
    y = g.add_value(m3.OUTPUT, m3.F32, (2,))
    g.add_node(m3.OP_COPY, [c], [y])
    status, made, _ = _session_status(g)
    assert status == m3.INVALID_ARGUMENT and not made  # unset constant
    g.free()


def test_topology_errors(fake):
    def graph_with(nodes, roles):
        g = m3.Graph()
        ids = [g.add_value(role, m3.F32, (3,)) for role in roles]
        for kind, ins, outs in nodes:
            g.add_node(kind, [ids[i] for i in ins], [ids[o] for o in outs])
        return g

    cases = [
        # writes an input
        ([(m3.OP_COPY, [0], [0])], [m3.INPUT]),
        # two producers
        ([(m3.OP_COPY, [0], [1]), (m3.OP_COPY, [0], [1])],
         [m3.INPUT, m3.OUTPUT]),
        # no producer for an output
        ([(m3.OP_COPY, [0], [1])], [m3.INPUT, m3.OUTPUT, m3.OUTPUT]),
    ]
    for nodes, roles in cases:
        g = graph_with(nodes, roles)
        status, made, _ = _session_status(g)
        assert status == m3.INVALID_ARGUMENT and not made
        g.free()


def test_extra_and_out_of_range_node_operands(fake):
    lib, _ = m3.load()
    g = m3.Graph()
    x = g.add_value(m3.INPUT, m3.F32, (3,))
    y = g.add_value(m3.OUTPUT, m3.F32, (3,))
    node = m3.NodeDesc()
    lib.m3_graph_node_desc_init(ctypes.byref(node), m3.OP_COPY)
    node.inputs[0] = x
    node.inputs[1] = x  # COPY takes one input
    node.outputs[0] = y
    assert lib.m3_graph_add_node(g.handle, ctypes.byref(node), None) == m3.OK
    assert _session_status(g)[0] == m3.INVALID_ARGUMENT
    g.free()
    g = m3.Graph()
    x = g.add_value(m3.INPUT, m3.F32, (3,))
    y = g.add_value(m3.OUTPUT, m3.F32, (3,))
    g.add_node(m3.OP_COPY, [x + 7], [y])
    assert _session_status(g)[0] == m3.OUT_OF_RANGE
    g.free()


def test_provider_options(fake):
    g, _, _, _ = reference_graph()
    assert _session_status(g, (False, False, False))[0] == \
        m3.INVALID_ARGUMENT
    # the CPU provider alone: host storage, no GPU backend made
    status, made, text = _session_status(g, (False, False, True))
    assert status == m3.OK and made, text
    assert fake.oracle_backend_reserved() == 0
    assert _session_status(g, (False, True, False))[0] == m3.OK
    # Neural Engine alone gives GPU storage but no provider for regular
    # nodes, as in the reference (src/m3_provider.c:62-99).
    assert _session_status(g, (True, False, False))[0] == m3.UNSUPPORTED
    g.free()


def test_no_gpu_falls_back_to_the_cpu_provider(fake):
    """src/m3_provider.c:46-58 of the reference: when the GPU backend cannot
    be made (UNSUPPORTED, no device) and the CPU provider is allowed, the
    session gets host storage and every node runs on the CPU provider. The
    default options (NULL) take this path. Without the CPU provider the
    session is UNSUPPORTED; any other constructor failure is returned as it
    is, whatever the options."""
    fake.oracle_backend_set_create_status(m3.UNSUPPORTED)
    g, x, y, constant = reference_graph()
    for options in (None, (True, True, True), (False, True, True),
                    (True, False, True)):
        status, made, text = _session_status(g, options)
        assert status == m3.OK and made, (options, text)
    assert fake.oracle_backend_reserved() == 0
    session = m3.Session(g)
    assert [session.provider(i) for i in range(4)] == [m3.PROVIDER_CPU] * 4
    data = np.array([1.0, 2.0, -3.0, 0.25], np.float32)
    session.write(x, data)
    session.run()
    out = session.read(y, np.zeros(4, np.float32))
    session.free()
    # tests/test_graph_runtime.c:139-146 of the reference, tolerance zero
    expected = ((c_tanhf(data + constant) * constant).astype(np.float32)
                + data).astype(np.float32)
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))
    assert log_of(fake) == ([], [])
    status, made, text = _session_status(g, (False, True, False))
    assert status == m3.UNSUPPORTED and not made, text
    assert "test backend: made to fail" in text
    # The Neural Engine option allows host storage (src/m3_graph_compile.c
    # :506-507 of the reference) but not the CPU provider for regular
    # nodes (:412-413), so the list finds no provider.
    status, made, text = _session_status(g, (True, True, False))
    assert status == m3.UNSUPPORTED and not made, text
    fake.oracle_backend_set_create_status(m3.INTERNAL)
    for options in (None, (False, True, True), (False, True, False)):
        status, made, text = _session_status(g, options)
        assert status == m3.INTERNAL and not made, (options, text)
    fake.oracle_backend_set_create_status(0)
    assert _session_status(g)[0] == m3.OK
    g.free()


def test_device_error_reported_by_its_run(fake):
    """An error the device reports when a list's completion is awaited (the
    HIP provider's stream wait or completion poll returns it from the
    list's execute call, as M3_STATUS_INTERNAL with the runtime's text)
    fails the m3_session_run that queued the list, with that status and
    message, and leaves the session usable: the next run succeeds and gives
    the exact result. This is the host side of the path; on the device an
    error the stream records without stopping its work is seen by the
    completion-word poll at most 63 completions later, and one that stops
    the queue after the 1 ms poll limit, by the stream wait."""
    g, x, y, constant = reference_graph()
    session = m3.Session(g)
    g.free()
    data = np.array([1.0, 2.0, -3.0, 0.25], np.float32)
    session.write(x, data)
    session.run()
    good = session.read(y, np.zeros(4, np.float32))
    lists = fake.oracle_backend_lists()
    fake.oracle_backend_fail_list_at(lists + 1, m3.INTERNAL)
    with pytest.raises(m3.M3Error) as failure:
        session.run()
    assert failure.value.status == m3.INTERNAL
    assert "the device reported an error" in failure.value.message
    assert fake.oracle_backend_lists() == lists + 1
    session.run()
    out = session.read(y, np.zeros(4, np.float32))
    assert np.array_equal(out.view(np.uint32), good.view(np.uint32))
    expected = ((c_tanhf(data + constant) * constant).astype(np.float32)
                + data).astype(np.float32)
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))
    session.free()


def test_reference_graph_kat_on_the_cpu_provider(fake):
    """tests/test_graph_runtime.c:87-160 of the reference: with the Neural
    Engine and GPU providers disabled the session compiles to host storage,
    every node runs on the CPU provider, the plan is 6 values, 4 nodes,
    5 slots, 80 bytes, the result equals tanhf(x + c) * c + x exactly, and
    I/O keeps roles and exact byte counts. Nothing reaches the GPU
    backend."""
    g, x, y, constant = reference_graph()
    session = m3.Session(g, allow_neural_engine=False, allow_metal=False)
    g.free()
    plan = session.plan()
    assert (plan.value_count, plan.node_count, plan.storage_slot_count,
            plan.allocated_bytes) == (6, 4, 5, 80)
    assert [session.provider(i) for i in range(4)] == [m3.PROVIDER_CPU] * 4
    data = np.array([1.0, 2.0, -3.0, 0.25], np.float32)
    session.write(x, data)
    session.run()
    out = session.read(y, np.zeros(4, np.float32))
    expected = ((c_tanhf(data + constant) * constant).astype(np.float32)
                + data).astype(np.float32)
    assert np.array_equal(out.view(np.uint32), expected.view(np.uint32))
    assert log_of(fake) == ([], [])
    assert fake.oracle_backend_reserved() == 0
    with pytest.raises(m3.M3Error) as failure:
        session.write(y, data)
    assert failure.value.status == m3.INVALID_ARGUMENT
    with pytest.raises(m3.M3Error) as failure:
        session.read(x, np.zeros(4, np.float32))
    assert failure.value.status == m3.INVALID_ARGUMENT
    session.free()


def test_out_of_scope_operation_is_unsupported(fake):
    g = m3.Graph()
    x = g.add_value(m3.INPUT, m3.F32, (3,))
    y = g.add_value(m3.OUTPUT, m3.F32, (3,))
    g.add_node(m3.OP_NEAREST_RESIZE1D, [x], [y])
    status, made, _ = _session_status(g)
    assert status == m3.UNSUPPORTED and not made
    g.free()
    lib, _ = m3.load()
    g = m3.Graph()
    assert lib.m3_graph_add_coreml_partition(g.handle, None,
                                             None) == m3.UNSUPPORTED
    g.free()


def test_allocation_failure_leaves_no_session(fake):
    g, _, _, _ = reference_graph()
    for index in range(1, 6):
        fake.oracle_backend_fail_allocation_at(index)
        status, made, _ = _session_status(g)
        assert status == m3.OUT_OF_MEMORY and not made
    fake.oracle_backend_fail_allocation_at(0)
    assert _session_status(g)[0] == m3.OK
    g.free()


def _random_graph(rng, nodes):
    """A random DAG of elementwise nodes over [5, 7] F32 values with mixed
    sizes (broadcast [7] and [1] operands)."""
    g = m3.Graph()
    shape = (5, 7)
    values = []  # (id, shape, numpy value)
    inputs = []
    for i in range(3):
        vid = g.add_value(m3.INPUT, m3.F32, shape)
        data = rng.standard_normal(shape).astype(np.float32)
        inputs.append((vid, data))
        values.append((vid, shape, data))
    c = g.add_value(m3.CONSTANT, m3.F32, (7,))
    cdata = rng.standard_normal(7).astype(np.float32)
    g.set_constant(c, cdata)
    values.append((c, (7,), cdata))
    produced = []
    ops = [(m3.OP_ADD, np.add), (m3.OP_MUL, np.multiply),
           (m3.OP_SUB, np.subtract)]
    for n in range(nodes):
        kind, fn = ops[rng.integers(len(ops))]
        a = values[rng.integers(len(values))]
        b = values[rng.integers(len(values))]
        out_shape = np.broadcast_shapes(a[1], b[1])
        role = m3.OUTPUT if n == nodes - 1 or rng.random() < 0.15 \
            else m3.TEMPORARY
        vid = g.add_value(role, m3.F32, out_shape)
        result = fn(np.broadcast_to(a[2], out_shape),
                    np.broadcast_to(b[2], out_shape)).astype(np.float32)
        g.add_node(kind, [a[0], b[0]], [vid])
        values.append((vid, out_shape, result))
        if role == m3.OUTPUT:
            produced.append((vid, result))
    return g, inputs, produced


@pytest.mark.parametrize("seed", range(12))
def test_random_graphs_reuse_slots_without_clobbering(fake, seed):
    rng = np.random.default_rng(seed)
    g, inputs, outputs = _random_graph(rng, 40)
    session = m3.Session(g)
    g.free()
    plan = session.plan()
    assert plan.storage_slot_count < plan.value_count  # reuse happened
    for vid, data in inputs:
        session.write(vid, data)
    session.run()
    for vid, expected in outputs:
        got = session.read(vid, np.zeros(expected.shape, np.float32))
        assert np.array_equal(got.view(np.uint32),
                              expected.view(np.uint32)), vid
    session.free()


def test_command_executor_runs_flow_math(fake, backend_lib):
    """The non-graph caller (src/m3_command_executor.c:55-92) used by the
    flow CFG/Euler math: one list per op through the scheduler."""
    lib, _ = m3.load()
    backend = ctypes.c_void_p()
    error = m3.Error()
    assert backend_lib.oracle_backend_create(ctypes.byref(backend),
                                             ctypes.byref(error)) == m3.OK
    executor = (ctypes.c_uint8 * 64)()
    lib.m3_command_executor_init(executor, backend)
    storages = []
    views = []
    arrays = [np.arange(6, dtype=np.float32), np.full(1, 2.0, np.float32),
              np.zeros(6, np.float32)]
    for array in arrays:
        storage = ctypes.c_void_p()
        lib.m3_storage_allocate(backend, array.nbytes, 64,
                                ctypes.byref(storage), None)
        lib.m3_storage_write(storage, 0, array.ctypes.data_as(
            ctypes.c_void_p), array.nbytes, None)
        view = m3.TensorView()
        shape = (ctypes.c_uint64 * 8)(*array.shape)
        assert lib.m3_tensor_view_contiguous(ctypes.byref(view), storage,
                                             m3.F32, 1, shape, 0,
                                             None) == m3.OK
        storages.append(storage)
        views.append(view)
    command = m3.Command()
    command.kind = m3.OP_MUL
    for i in range(3):
        command.descriptor.views[i] = ctypes.pointer(views[i])
    lib.m3_command_executor_execute.argtypes = [ctypes.c_void_p,
                                                ctypes.POINTER(m3.Command),
                                                ctypes.c_size_t,
                                                ctypes.POINTER(m3.Error)]
    assert lib.m3_command_executor_execute(executor, ctypes.byref(command), 1,
                                           ctypes.byref(error)) == m3.OK
    out = np.zeros(6, np.float32)
    lib.m3_storage_read(storages[2], 0, out.ctypes.data_as(ctypes.c_void_p),
                        24, None)
    assert list(out) == [0, 2, 4, 6, 8, 10]
    lib.m3_command_executor_dispose(executor)
    for storage in storages:
        lib.m3_storage_free(storage)
    lib.m3_backend_free(backend)


# ---- fused elementwise runs ------------------------------------------------

def _session_outputs(graph_builder, fusion, fake):
    """Builds, runs and reads a graph with fusion on or off; returns the
    outputs, the plan and the number of programs the backend ran."""
    previous = os.environ.get("M3_HIP_FUSION")
    os.environ["M3_HIP_FUSION"] = "1" if fusion else "0"
    try:
        g, feeds, outputs = graph_builder()
        fake.oracle_backend_reset()
        session = m3.Session(g)
    finally:
        if previous is None:
            del os.environ["M3_HIP_FUSION"]
        else:
            os.environ["M3_HIP_FUSION"] = previous
    g.free()
    plan = session.plan()
    for vid, data in feeds:
        session.write(vid, data)
    session.run()
    results = [session.read(vid, np.zeros(entry[0], entry[1] if len(entry)
                                          > 1 else np.float32))
               for vid, *entry in outputs]
    programs = fake.oracle_backend_programs()
    kinds, _ = log_of(fake)
    session.free()
    return results, (plan.storage_slot_count, plan.allocated_bytes), \
        programs, kinds


def _specials(rng, shape):
    data = rng.standard_normal(shape).astype(np.float32)
    bits = data.view(np.uint32)
    pick = rng.random(shape)
    payload = rng.integers(1, 1 << 22, shape, dtype=np.uint32)
    bits[pick < 0.03] = (0x7f800000 | payload)[pick < 0.03]
    bits[(pick >= 0.03) & (pick < 0.05)] = 0xff800000
    bits[(pick >= 0.05) & (pick < 0.06)] = 0
    return data


def _random_chain_graph(seed):
    """Elementwise DAGs with scalar operands, OUTPUT values read again,
    COPY barriers and temporaries read by several nodes."""
    def build():
        rng = np.random.default_rng(seed)
        shape = (3, 5, 7)
        g = m3.Graph()
        values = []
        feeds = []
        outputs = []
        for _ in range(3):
            vid = g.add_value(m3.INPUT, m3.F32, shape)
            feeds.append((vid, _specials(rng, shape)))
            values.append((vid, shape))
        for _ in range(2):
            vid = g.add_value(m3.CONSTANT, m3.F32, (1,))
            g.set_constant(vid, (rng.standard_normal(1) + 2.0)
                           .astype(np.float32))
            values.append((vid, (1,)))
        kinds = [m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV]
        for n in range(30):
            role = m3.OUTPUT if n == 29 or rng.random() < 0.2 \
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


_NUMPY_OF = {m3.F32: np.float32, m3.F16: np.uint16, m3.BF16: np.uint16}


def _narrow(rng, shape, dtype):
    """Random 16-bit patterns of `dtype`: normal values near 1 with NaN
    payloads (signalling and quiet), infinities, zeros and subnormals."""
    data = _specials(rng, shape)
    bits = data.view(np.uint32)
    if dtype == m3.BF16:
        return (bits >> np.uint32(16)).astype(np.uint16)
    half = data.astype(np.float16).view(np.uint16)
    pick = rng.random(shape)
    half[pick < 0.05] = rng.integers(0x7c01, 0x8000, shape)[pick < 0.05]
    half[(pick >= 0.05) & (pick < 0.07)] = 0x0001
    return half


def _mixed_chain_graph(seed):
    """Elementwise DAGs over F32, F16 and BF16 values: binary nodes with
    any float output dtype, CASTs between float dtypes, COPYs, scalar
    operands, OUTPUT values read again."""
    def build():
        rng = np.random.default_rng(seed)
        shape = (3, 5, 7)
        floats = [m3.F32, m3.F16, m3.BF16]
        g = m3.Graph()
        values = []
        feeds = []
        outputs = []
        for dtype in (m3.F32, m3.F16, m3.BF16, m3.F32):
            vid = g.add_value(m3.INPUT, dtype, shape)
            feeds.append((vid, _specials(rng, shape) if dtype == m3.F32
                          else _narrow(rng, shape, dtype)))
            values.append((vid, shape, dtype))
        for dtype in (m3.F32, m3.BF16):
            vid = g.add_value(m3.CONSTANT, dtype, (1,))
            constant = (rng.standard_normal(1) + 2.0).astype(np.float32)
            g.set_constant(vid, constant if dtype == m3.F32 else
                           (constant.view(np.uint32) >> np.uint32(16))
                           .astype(np.uint16))
            values.append((vid, (1,), dtype))
        kinds = [m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV]
        for n in range(40):
            role = m3.OUTPUT if n == 39 or rng.random() < 0.2 \
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
                outputs.append((entry[0], entry[1], _NUMPY_OF[entry[2]]))
        return g, feeds, outputs
    return build


@pytest.mark.parametrize("seed", range(8))
def test_fused_mixed_dtype_runs_equal_unfused_runs(fake, seed):
    """F16/BF16 values, CAST and COPY inside programs: every OUTPUT is
    identical byte for byte with and without fusion."""
    build = _mixed_chain_graph(3000 + seed)
    fused, plan_on, programs_on, kinds_on = _session_outputs(build, True,
                                                             fake)
    plain, plan_off, programs_off, kinds_off = _session_outputs(build, False,
                                                                fake)
    assert plan_on == plan_off
    assert programs_off == 0
    assert kinds_on == kinds_off
    for a, b in zip(fused, plain):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


def test_mixed_dtype_graphs_fuse_casts(fake):
    """The planner does fuse CAST nodes and 16-bit values (the backend logs
    the constituents of every program it runs)."""
    programs = 0
    for seed in range(8):
        build = _mixed_chain_graph(3000 + seed)
        programs += _session_outputs(build, True, fake)[2]
    assert programs >= 8


@pytest.mark.parametrize("seed", range(8))
def test_fused_runs_equal_unfused_runs(fake, seed):
    """Every OUTPUT, NaN payloads included, is identical with and without
    fusion; the slot plan does not change; fused runs do execute."""
    build = _random_chain_graph(1000 + seed)
    fused, plan_on, programs_on, kinds_on = _session_outputs(build, True,
                                                             fake)
    plain, plan_off, programs_off, kinds_off = _session_outputs(build, False,
                                                                fake)
    assert plan_on == plan_off
    assert programs_off == 0
    assert kinds_on == kinds_off
    for a, b in zip(fused, plain):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_fusion_happens_on_random_graphs(fake):
    total = 0
    for seed in range(8):
        build = _random_chain_graph(1000 + seed)
        total += _session_outputs(build, True, fake)[2]
    assert total >= 8


def _broadcast_chain_graph(seed):
    """Elementwise DAGs over [3, 4, 8] whose operands are broadcast from
    smaller tensors: trailing ones ([8], [1, 8], [4, 8], [1, 4, 8], which
    programs read periodically), others ([3, 1, 8], [3, 4, 1], [4, 1],
    which stay unfused nodes), scalars, F16 and BF16 values among them."""
    full = (3, 4, 8)
    shapes = [full, (8,), (1, 8), (4, 8), (1, 4, 8), (3, 1, 8), (3, 4, 1),
              (4, 1), (1,)]

    def build():
        rng = np.random.default_rng(seed)
        floats = [m3.F32, m3.F16, m3.BF16]
        g = m3.Graph()
        values = []
        feeds = []
        outputs = []
        for shape in shapes:
            for dtype in (m3.F32, floats[1 + rng.integers(2)]):
                vid = g.add_value(m3.INPUT, dtype, shape)
                feeds.append((vid, _specials(rng, shape) if dtype == m3.F32
                              else _narrow(rng, shape, dtype)))
                values.append((vid, shape, dtype))
        kinds = [m3.OP_ADD, m3.OP_MUL, m3.OP_SUB, m3.OP_DIV]
        for n in range(40):
            role = m3.OUTPUT if n == 39 or rng.random() < 0.2 \
                else m3.TEMPORARY
            # mostly a full-size operand beside a broadcast one
            produced = [v for v in values[2 * len(shapes):]
                        if v[1] == full]
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
                outputs.append((vid, out_shape, _NUMPY_OF[dtype]))
        return g, feeds, outputs
    return build


@pytest.mark.parametrize("seed", range(8))
def test_fused_broadcast_runs_equal_unfused_runs(fake, seed):
    """Operands broadcast along trailing axes are read periodically inside
    programs; every OUTPUT is identical byte for byte with and without
    fusion."""
    build = _broadcast_chain_graph(5000 + seed)
    fused, plan_on, _, kinds_on = _session_outputs(build, True, fake)
    plain, plan_off, programs_off, kinds_off = _session_outputs(build, False,
                                                                fake)
    assert plan_on == plan_off
    assert programs_off == 0
    assert kinds_on == kinds_off
    for a, b in zip(fused, plain):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


def test_broadcast_graphs_fuse_periodic_operands(fake):
    """The planner does read trailing-broadcast operands inside programs
    (the backend counts the periodic operands of the programs it runs)."""
    periodic = 0
    for seed in range(8):
        _session_outputs(_broadcast_chain_graph(5000 + seed), True, fake)
        periodic += fake.oracle_backend_periodic()
    assert periodic >= 40


def _euler_graph(steps, shape):
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
        for k in range(steps):
            vu = g.add_value(m3.CONSTANT, m3.F32, shape)
            vc = g.add_value(m3.CONSTANT, m3.F32, shape)
            g.set_constant(vu, m3.rng_fill("normal", count, seed=0, a=1.0,
                                           rng=rng).reshape(shape))
            g.set_constant(vc, m3.rng_fill("normal", count, seed=0, a=1.0,
                                           rng=rng).reshape(shape))
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
        return g, [(vx, x0)], [(current, shape)]
    return build


def test_euler_graph_runs_as_one_program(fake):
    """The 6-step CFG + Euler graph becomes one program (every node in it,
    in order), with the unfused slot plan and result."""
    build = _euler_graph(6, (2, 8, 12))
    fused, plan_on, programs, kinds = _session_outputs(build, True, fake)
    plain, plan_off, _, kinds_off = _session_outputs(build, False, fake)
    assert programs == 1
    assert kinds == kinds_off and len(kinds) == 36
    assert plan_on == plan_off
    assert np.array_equal(fused[0].view(np.uint32), plain[0].view(np.uint32))


# ---- fused runs next to nodes that never fuse, and shared slots ------------

def _both_orders(fake, build):
    """Fused outputs with programs run over increasing and decreasing
    elements, and the unfused outputs."""
    results = []
    try:
        for decreasing in (0, 1):
            fake.oracle_backend_set_program_order(decreasing)
            results.append(_session_outputs(build, True, fake))
    finally:
        fake.oracle_backend_set_program_order(0)
    return results, _session_outputs(build, False, fake)


def _consumer_graph(consumer):
    """A fused run whose last temporary is read only by a node that never
    fuses (the scale + mask -> softmax and x * w + b -> tanh patterns, and
    the two-input Snake1d and GATED_SILU)."""
    def build():
        rng = np.random.default_rng(17)
        shape = (4, 8, 64) if consumer == m3.OP_SNAKE1D else (4, 64)
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


@pytest.mark.parametrize("consumer", ["SOFTMAX", "TANH", "SNAKE1D",
                                      "GATED_SILU"])
def test_value_read_by_an_unfused_kind_is_stored(fake, consumer):
    """The fused MUL + ADD run stores the temporary its non-fusing reader
    needs; the result equals the unfused run's, and the run is fused."""
    build = _consumer_graph(getattr(m3, "OP_" + consumer))
    fused_runs, plain = _both_orders(fake, build)
    for fused in fused_runs:
        assert fused[2] == 1
        assert fused[1] == plain[1]
        assert np.array_equal(fused[0][0].view(np.uint32),
                              plain[0][0].view(np.uint32))


def _periodic_slot_graph():
    """x = c + d ([4]) takes the free 128-byte slot a finished [8, 4] value
    left; z = y + x reads x periodically (a trailing broadcast) and
    t = z * a is planned into the same slot once x is dead. Fused, t's
    stores would overwrite x while other elements still read x[e mod 4]."""
    def build():
        rng = np.random.default_rng(3)
        shape = (8, 4)
        g = m3.Graph()
        a = g.add_value(m3.INPUT, m3.F32, shape)
        b = g.add_value(m3.INPUT, m3.F32, shape)
        y = g.add_value(m3.INPUT, m3.F32, shape)
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


def _narrow_slot_graph():
    """A softmax output s (F32) is read by a fused run whose F16 result h
    is planned into s's slot once s is dead; element e of h covers bytes of
    element e / 2 of s, which another element reads."""
    def build():
        rng = np.random.default_rng(4)
        g = m3.Graph()
        x = g.add_value(m3.INPUT, m3.F32, (8, 16))
        w = g.add_value(m3.INPUT, m3.F32, (8, 16))
        s = g.add_value(m3.TEMPORARY, m3.F32, (8, 16))
        u = g.add_value(m3.TEMPORARY, m3.F32, (8, 16))
        h = g.add_value(m3.TEMPORARY, m3.F16, (8, 16))
        out = g.add_value(m3.OUTPUT, m3.F32, (8, 16))
        g.add_node(m3.OP_SOFTMAX, [x], [s])
        g.add_node(m3.OP_MUL, [s, w], [u])
        g.add_node(m3.OP_CAST, [u], [h])
        g.add_node(m3.OP_SOFTMAX, [h], [out])
        feeds = [(x, rng.standard_normal((8, 16)).astype(np.float32)),
                 (w, rng.standard_normal((8, 16)).astype(np.float32))]
        return g, feeds, [(out, (8, 16))]
    return build


@pytest.mark.parametrize("graph", ["periodic", "narrow"])
def test_fused_stores_never_land_on_operands_other_elements_read(fake,
                                                                 graph):
    """With slots shared by liveness, the planner does not fuse a run whose
    store would overwrite an operand other elements still read: fused
    results equal unfused ones in either element order, the slot plan is
    unchanged."""
    build = _periodic_slot_graph() if graph == "periodic" \
        else _narrow_slot_graph()
    fused_runs, plain = _both_orders(fake, build)
    for fused in fused_runs:
        assert fused[1] == plain[1]
        for a, b in zip(fused[0], plain[0]):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- sessions that mix the GPU and CPU providers ----------------------------

def _mixed_graph(seed):
    """MUL (GPU) -> SOFTMAX (CPU) -> ADD (GPU) -> TANH (CPU) -> MUL (GPU),
    and a CPU-only branch from the input and a constant to an OUTPUT:
    x * c -> softmax -> + x -> tanh -> * c = y; softmax(x + 0) read only by
    the CPU = z."""
    def build():
        rng = np.random.default_rng(seed)
        shape = (4, 64)
        g = m3.Graph()
        x = g.add_value(m3.INPUT, m3.F32, shape)
        c = g.add_value(m3.CONSTANT, m3.F32, (64,))
        g.set_constant(c, rng.standard_normal(64).astype(np.float32))
        t = [g.add_value(m3.TEMPORARY, m3.F32, shape) for _ in range(4)]
        y = g.add_value(m3.OUTPUT, m3.F32, shape)
        z = g.add_value(m3.OUTPUT, m3.F32, shape)
        g.add_node(m3.OP_MUL, [x, c], [t[0]])
        g.add_node(m3.OP_SOFTMAX, [t[0]], [t[1]])
        g.add_node(m3.OP_ADD, [t[1], x], [t[2]])
        g.add_node(m3.OP_TANH, [t[2]], [t[3]])
        g.add_node(m3.OP_MUL, [t[3], c], [y])
        g.add_node(m3.OP_SOFTMAX, [x], [z])
        return g, x, (y, z), shape, rng
    return build


def _run_mixed(fake, build, cpu_kinds, device_memory):
    previous = os.environ.get("M3_HIP_CPU_KINDS")
    if cpu_kinds:
        os.environ["M3_HIP_CPU_KINDS"] = cpu_kinds
    fake.oracle_backend_set_device_memory(1 if device_memory else 0)
    try:
        g, x, outputs, shape, rng = build()
        session = m3.Session(g)
    finally:
        fake.oracle_backend_set_device_memory(0)
        if previous is None:
            os.environ.pop("M3_HIP_CPU_KINDS", None)
        else:
            os.environ["M3_HIP_CPU_KINDS"] = previous
    g.free()
    providers = [session.provider(n) for n in range(6)]
    runs = []
    for _ in range(2):
        session.write(x, rng.standard_normal(shape).astype(np.float32))
        before = (fake.oracle_backend_transfers(1),
                  fake.oracle_backend_transfers(0))
        session.run()
        moved = (fake.oracle_backend_transfers(1) - before[0],
                 fake.oracle_backend_transfers(0) - before[1])
        runs.append(([session.read(v, np.zeros(shape, np.float32))
                      for v in outputs], moved))
    session.free()
    return providers, runs


def test_mixed_session_stages_once_per_value(fake):
    """SOFTMAX and TANH left to the CPU provider over device memory: they
    run on host mirrors; per run the session copies device -> host the
    softmax input, the TANH input and x (3 copies, the constant is
    mirrored at creation) and host -> device the two values GPU nodes read
    next (softmax and tanh results) and the CPU-written OUTPUT z (3
    copies). Results equal the all-GPU session's bit for bit, on fresh
    inputs each run."""
    build = _mixed_graph(31)
    fake.oracle_backend_reset()
    fake.oracle_backend_transfers.restype = ctypes.c_size_t
    fake.oracle_backend_transfers.argtypes = [ctypes.c_int]
    gpu_providers, gpu_runs = _run_mixed(fake, build, None, True)
    providers, runs = _run_mixed(fake, build, "SOFTMAX,TANH", True)
    assert gpu_providers == [m3.PROVIDER_HIP] * 6
    assert providers == [m3.PROVIDER_HIP, m3.PROVIDER_CPU, m3.PROVIDER_HIP,
                         m3.PROVIDER_CPU, m3.PROVIDER_HIP, m3.PROVIDER_CPU]
    for (outputs, moved), (expected, _) in zip(runs, gpu_runs):
        assert moved == (3, 3)
        for a, b in zip(outputs, expected):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the two runs saw different inputs
    assert not np.array_equal(runs[0][0][0], runs[1][0][0])


def test_cpu_kinds_over_host_memory_run_in_place(fake):
    """Over host-visible memory the CPU provider's nodes need no mirrors
    and nothing is copied; results equal the all-GPU session's."""
    build = _mixed_graph(32)
    fake.oracle_backend_transfers.restype = ctypes.c_size_t
    fake.oracle_backend_transfers.argtypes = [ctypes.c_int]
    _, gpu_runs = _run_mixed(fake, build, None, False)
    providers, runs = _run_mixed(fake, build, "SOFTMAX,TANH", False)
    assert providers.count(m3.PROVIDER_CPU) == 3
    for (outputs, moved), (expected, _) in zip(runs, gpu_runs):
        assert moved == (0, 0)
        for a, b in zip(outputs, expected):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
