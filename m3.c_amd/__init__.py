"""Python bindings (ctypes) for the m3 HIP execution provider.

The product is native: ``libm3.so`` (C11 host layer: graph, session,
scheduler, backend) linked against ``libm3_hip.so`` (hipcc-built gfx950
kernels behind the C ABI of ``include/m3_hip.h``). This module only loads
those libraries and mirrors the C structs so tests and benchmarks can drive
the public API of ``include/m3.h`` from Python. Nothing here computes
tensor values; when the libraries are missing, :func:`load` raises.

The package directory is named ``m3.c_amd`` (not an importable dotted
name); load it with :func:`importlib.util.spec_from_file_location`.
"""

import ctypes
import os

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PACKAGE_DIR)
# M3_LIBRARY_DIR selects another build of the host layer (the sanitizer
# build of the CPU suite); the kernels always come from this package.
LIBRARY_PATH = os.path.join(os.environ.get("M3_LIBRARY_DIR", PACKAGE_DIR),
                            "libm3.so")
HIP_LIBRARY_PATH = os.path.join(PACKAGE_DIR, "libm3_hip.so")

MAX_RANK = 8
VALUE_NONE = 0xFFFFFFFF

# m3_status
OK, INVALID_ARGUMENT, OUT_OF_RANGE, OVERFLOW, OUT_OF_MEMORY, IO, \
    INVALID_FORMAT, UNSUPPORTED, CANCELLED, INTERNAL = range(10)
STATUS_NAMES = {
    0: "OK", 1: "INVALID_ARGUMENT", 2: "OUT_OF_RANGE", 3: "OVERFLOW",
    4: "OUT_OF_MEMORY", 5: "IO", 6: "INVALID_FORMAT", 7: "UNSUPPORTED",
    8: "CANCELLED", 9: "INTERNAL",
}

# m3_dtype
F32, F16, BF16, I32 = range(4)
DTYPE_SIZES = {F32: 4, F16: 2, BF16: 2, I32: 4}

# m3_op_kind (reference values; SUB and DIV appended)
(OP_COPY, OP_CAST, OP_ADD, OP_MUL, OP_EMBEDDING, OP_MATMUL, OP_LINEAR,
 OP_RMS_NORM, OP_LAYER_NORM, OP_ROPE, OP_ATTENTION, OP_GATED_SILU,
 OP_SOFTMAX, OP_TOP_K, OP_CATEGORICAL, OP_CONV1D, OP_CONV_TRANSPOSE1D,
 OP_NEAREST_RESIZE1D, OP_SNAKE1D, OP_TANH, OP_SUB, OP_DIV) = range(22)

# m3_provider_kind
PROVIDER_NEURAL_ENGINE, PROVIDER_METAL, PROVIDER_CPU, PROVIDER_HIP = range(4)

# m3_graph_value_role
INPUT, CONSTANT, TEMPORARY, OUTPUT = range(4)

# m3_backend_kind
BACKEND_HOST, BACKEND_METAL, BACKEND_HIP = range(3)


class Error(ctypes.Structure):
    _fields_ = [("status", ctypes.c_int), ("message", ctypes.c_char * 256)]

    def text(self):
        return self.message.decode("utf-8", "replace")


class ValueDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("rank", ctypes.c_uint8),
                ("shape", ctypes.c_uint64 * MAX_RANK), ("role", ctypes.c_int)]


class _NodeParameters(ctypes.Union):
    _fields_ = [("words", ctypes.c_uint64 * 6)]


class NodeDesc(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int),
                ("inputs", ctypes.c_uint32 * 5),
                ("outputs", ctypes.c_uint32 * 2),
                ("parameters", _NodeParameters)]


class SessionOptions(ctypes.Structure):
    _fields_ = [("allow_neural_engine", ctypes.c_bool),
                ("allow_metal", ctypes.c_bool),
                ("allow_cpu", ctypes.c_bool)]


class PlanInfo(ctypes.Structure):
    _fields_ = [("value_count", ctypes.c_size_t),
                ("node_count", ctypes.c_size_t),
                ("storage_slot_count", ctypes.c_size_t),
                ("allocated_bytes", ctypes.c_size_t)]


class TensorMetadata(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int), ("rank", ctypes.c_uint8),
                ("shape", ctypes.c_uint64 * MAX_RANK),
                ("element_count", ctypes.c_size_t),
                ("byte_count", ctypes.c_size_t)]


class TensorView(ctypes.Structure):
    _fields_ = [("metadata", TensorMetadata),
                ("byte_offset", ctypes.c_size_t),
                ("byte_strides", ctypes.c_size_t * MAX_RANK),
                ("storage", ctypes.c_void_p)]


class _CommandDescriptor(ctypes.Union):
    # Largest member of the reference union: ConvTranspose1d, four view
    # pointers and six 64-bit parameters.
    _fields_ = [("views", ctypes.POINTER(TensorView) * 4),
                ("words", ctypes.c_uint64 * 10)]


class Command(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("descriptor", _CommandDescriptor)]


class BackendInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("kind", ctypes.c_int),
                ("unified_memory", ctypes.c_bool),
                ("recommended_working_set_bytes", ctypes.c_uint64),
                ("maximum_storage_bytes", ctypes.c_uint64)]


class AllocationStats(ctypes.Structure):
    _fields_ = [("live_allocated_bytes", ctypes.c_size_t),
                ("peak_allocated_bytes", ctypes.c_size_t),
                ("live_storage_count", ctypes.c_size_t),
                ("peak_storage_count", ctypes.c_size_t)]


class ScratchArena(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("capacity", ctypes.c_size_t),
                ("offset", ctypes.c_size_t)]


class Rng(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64), ("increment", ctypes.c_uint64),
                ("spare_normal", ctypes.c_float),
                ("has_spare_normal", ctypes.c_bool)]


class HipView(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("byte_offset", ctypes.c_uint64),
                ("element_count", ctypes.c_uint64),
                ("shape", ctypes.c_uint64 * MAX_RANK),
                ("byte_strides", ctypes.c_uint64 * MAX_RANK),
                ("rank", ctypes.c_uint32), ("dtype", ctypes.c_uint32)]


class HipKernelTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("launches", ctypes.c_uint64),
                ("total_ms", ctypes.c_double)]


# Every exported symbol of include/m3.h, include/m3_backend.h,
# include/m3_backend_hip.h, include/m3_rng.h (libm3.so) and
# include/m3_hip.h (libm3_hip.so).
EXPORTS_M3 = [
    "m3_version", "m3_status_string", "m3_error_reset", "m3_error_message",
    "m3_graph_value_desc_init", "m3_graph_node_desc_init",
    "m3_session_options_init", "m3_graph_create", "m3_graph_free",
    "m3_graph_add_value", "m3_graph_set_constant",
    "m3_graph_add_inferred_value", "m3_graph_add_node",
    "m3_graph_add_coreml_partition", "m3_session_create", "m3_session_free",
    "m3_session_write_input", "m3_session_read_output", "m3_session_run",
    "m3_session_get_plan_info", "m3_session_get_node_provider",
    "m3_error_set", "m3_error_set_v", "m3_dtype_name", "m3_dtype_size",
    "m3_tensor_metadata_init", "m3_tensor_view_init",
    "m3_tensor_view_contiguous", "m3_tensor_view_strided",
    "m3_tensor_is_contiguous", "m3_tensor_const_data", "m3_tensor_data",
    "m3_tensor_element_offset", "m3_tensor_slice", "m3_tensor_reshape",
    "m3_tensor_permute", "m3_scratch_arena_init", "m3_scratch_arena_mark",
    "m3_scratch_arena_rewind", "m3_command_validate",
    "m3_commands_scratch_bytes", "m3_backend_execute", "m3_backend_finish",
    "m3_backend_create_internal", "m3_backend_create_hip",
    "m3_backend_create_host", "m3_hip_owns_execute", "m3_hip_context_device",
    "m3_backend_free",
    "m3_backend_get_info", "m3_backend_get_allocation_stats",
    "m3_backend_reserve", "m3_backend_context_internal",
    "m3_storage_allocate", "m3_storage_free", "m3_storage_size",
    "m3_storage_data", "m3_storage_const_data", "m3_storage_device_data",
    "m3_storage_handle_internal", "m3_storage_backend",
    "m3_storage_host_visible", "m3_storage_write", "m3_storage_read",
    "m3_command_executor_init", "m3_command_executor_dispose",
    "m3_command_executor_execute", "m3_provider_set_gpu_factory",
    "m3_session_backend", "m3_backend_hip_device",
    "m3_rng_seed", "m3_rng_u32", "m3_rng_uniform_f32",
    "m3_rng_normal_f32_fill", "m3_rng_uniform_f32_fill",
    "m3_rng_normal_f32_fill_scaled",
]
EXPORTS_HIP = [
    "m3_hip_device_count", "m3_hip_device_open", "m3_hip_device_close",
    "m3_hip_device_properties", "m3_hip_arena_reserve",
    "m3_hip_arena_release", "m3_hip_copy_h2d", "m3_hip_copy_d2h",
    "m3_hip_fill_zero", "m3_hip_launch_binary", "m3_hip_launch_cast",
    "m3_hip_launch_copy", "m3_hip_launch_softmax", "m3_hip_launch_snake1d",
    "m3_hip_scan_views", "m3_hip_synchronize", "m3_hip_timing_enable",
    "m3_hip_timing_reset", "m3_hip_timing_read", "m3_hip_timing_samples",
    "m3_hip_stream",
    "m3_hip_launch_program", "m3_hip_launch_tanh", "m3_hip_launch_gated_silu",
    "m3_hip_prepare_program", "m3_hip_scan_views_static",
    "m3_hip_scan_views_begin", "m3_hip_scan_views_collect",
    "m3_hip_gate_open", "m3_hip_gate_check", "m3_hip_gate_close",
    "m3_hip_launch_program_checked", "m3_hip_gate_pending",
    "m3_hip_host_waits", "m3_hip_allocation_count",
]

_LIB = None
_HIP = None


def _declare(lib, name, restype, *argtypes):
    fn = getattr(lib, name)
    fn.restype = restype
    fn.argtypes = list(argtypes)


def load():
    """Loads libm3.so and libm3_hip.so (raises OSError when not built)."""
    global _LIB, _HIP
    if _LIB is not None:
        return _LIB, _HIP
    for path in (HIP_LIBRARY_PATH, LIBRARY_PATH):
        if not os.path.exists(path):
            raise OSError(
                "%s is not built; run __graft_entry__.build() (or make -C "
                "m3.c_amd) first" % path)
    hip = ctypes.CDLL(HIP_LIBRARY_PATH, mode=ctypes.RTLD_GLOBAL)
    lib = ctypes.CDLL(LIBRARY_PATH)
    P = ctypes.POINTER
    vp = ctypes.c_void_p
    sz = ctypes.c_size_t
    err = P(Error)
    st = ctypes.c_int
    _declare(lib, "m3_version", ctypes.c_char_p)
    _declare(lib, "m3_status_string", ctypes.c_char_p, st)
    _declare(lib, "m3_graph_value_desc_init", None, P(ValueDesc), st, st,
             ctypes.c_uint8, P(ctypes.c_uint64))
    _declare(lib, "m3_graph_node_desc_init", None, P(NodeDesc), st)
    _declare(lib, "m3_session_options_init", None, P(SessionOptions))
    _declare(lib, "m3_graph_create", st, P(vp), err)
    _declare(lib, "m3_graph_free", None, vp)
    _declare(lib, "m3_graph_add_value", st, vp, P(ValueDesc),
             P(ctypes.c_uint32), err)
    _declare(lib, "m3_graph_set_constant", st, vp, ctypes.c_uint32, vp, sz,
             err)
    _declare(lib, "m3_graph_add_inferred_value", st, vp, P(NodeDesc), sz, st,
             st, P(ctypes.c_uint32), err)
    _declare(lib, "m3_graph_add_node", st, vp, P(NodeDesc), err)
    _declare(lib, "m3_graph_add_coreml_partition", st, vp, vp, err)
    _declare(lib, "m3_session_create", st, P(vp), vp, P(SessionOptions), err)
    _declare(lib, "m3_session_free", None, vp)
    _declare(lib, "m3_session_write_input", st, vp, ctypes.c_uint32, vp, sz,
             err)
    _declare(lib, "m3_session_read_output", st, vp, ctypes.c_uint32, vp, sz,
             err)
    _declare(lib, "m3_session_run", st, vp, err)
    _declare(lib, "m3_session_get_plan_info", st, vp, P(PlanInfo), err)
    _declare(lib, "m3_session_get_node_provider", st, vp, sz, P(ctypes.c_int),
             err)
    _declare(lib, "m3_session_backend", vp, vp)
    _declare(lib, "m3_backend_hip_device", vp, vp)
    _declare(lib, "m3_dtype_size", sz, st)
    _declare(lib, "m3_tensor_view_init", None, P(TensorView))
    _declare(lib, "m3_tensor_view_contiguous", st, P(TensorView), vp, st,
             ctypes.c_uint8, P(ctypes.c_uint64), sz, err)
    _declare(lib, "m3_tensor_view_strided", st, P(TensorView), vp, st,
             ctypes.c_uint8, P(ctypes.c_uint64), P(ctypes.c_size_t), sz, err)
    _declare(lib, "m3_tensor_is_contiguous", ctypes.c_bool, P(TensorView))
    _declare(lib, "m3_tensor_slice", st, P(TensorView), ctypes.c_uint8,
             ctypes.c_uint64, ctypes.c_uint64, P(TensorView), err)
    _declare(lib, "m3_command_validate", st, vp, P(Command), err)
    _declare(lib, "m3_backend_execute", st, vp, P(Command), sz,
             P(ScratchArena), err)
    _declare(lib, "m3_backend_finish", st, vp, err)
    _declare(lib, "m3_backend_create_hip", st, P(vp), err)
    _declare(lib, "m3_backend_create_host", st, P(vp), err)
    _declare(lib, "m3_backend_free", None, vp)
    _declare(lib, "m3_backend_get_info", st, vp, P(BackendInfo), err)
    _declare(lib, "m3_backend_get_allocation_stats", st, vp,
             P(AllocationStats), err)
    _declare(lib, "m3_storage_allocate", st, vp, sz, sz, P(vp), err)
    _declare(lib, "m3_storage_free", None, vp)
    _declare(lib, "m3_storage_size", sz, vp)
    _declare(lib, "m3_storage_data", vp, vp)
    _declare(lib, "m3_storage_device_data", vp, vp)
    _declare(lib, "m3_storage_backend", vp, vp)
    _declare(lib, "m3_storage_write", st, vp, sz, vp, sz, err)
    _declare(lib, "m3_storage_read", st, vp, sz, vp, sz, err)
    _declare(lib, "m3_rng_seed", st, P(Rng), ctypes.c_uint64, ctypes.c_uint64,
             err)
    _declare(lib, "m3_rng_u32", st, P(Rng), P(ctypes.c_uint32), err)
    _declare(lib, "m3_rng_uniform_f32", st, P(Rng), P(ctypes.c_float), err)
    _declare(lib, "m3_rng_normal_f32_fill", st, P(Rng), vp, sz, err)
    _declare(lib, "m3_rng_uniform_f32_fill", st, P(Rng), vp, sz,
             ctypes.c_float, ctypes.c_float, err)
    _declare(lib, "m3_rng_normal_f32_fill_scaled", st, P(Rng), vp, sz,
             ctypes.c_float, err)
    _declare(hip, "m3_hip_device_count", st, P(ctypes.c_int), ctypes.c_char_p,
             sz)
    _declare(hip, "m3_hip_timing_enable", st, vp, ctypes.c_int)
    _declare(hip, "m3_hip_timing_reset", st, vp)
    _declare(hip, "m3_hip_timing_read", st, vp, P(HipKernelTime), sz, P(sz),
             ctypes.c_char_p, sz)
    _declare(hip, "m3_hip_timing_samples", st, vp, ctypes.c_char_p,
             P(ctypes.c_float), sz, P(sz), ctypes.c_char_p, sz)
    _declare(hip, "m3_hip_stream", vp, vp)
    _declare(hip, "m3_hip_synchronize", st, vp, ctypes.c_char_p, sz)
    _declare(hip, "m3_hip_host_waits", st, vp, P(ctypes.c_uint64))
    _declare(hip, "m3_hip_launch_program", st, vp, P(ctypes.c_uint32), vp,
             sz, ctypes.c_char_p, sz)
    _LIB, _HIP = lib, hip
    return lib, hip


def status_name(status):
    return STATUS_NAMES.get(status, str(status))


class M3Error(RuntimeError):
    def __init__(self, status, message):
        super().__init__("%s: %s" % (status_name(status), message))
        self.status = status
        self.message = message


def check(status, error):
    if status != OK:
        raise M3Error(status, error.text())


def hip_device_count():
    """Number of HIP devices (0 without a GPU); never initialises kernels."""
    _, hip = load()
    count = ctypes.c_int(0)
    message = ctypes.create_string_buffer(256)
    hip.m3_hip_device_count(ctypes.byref(count), message, 256)
    return count.value


def _shape_array(shape):
    array = (ctypes.c_uint64 * MAX_RANK)()
    for i, dim in enumerate(shape):
        array[i] = dim
    return array


class Graph:
    """Thin owner of an m3_graph built through the public C API."""

    def __init__(self):
        self.lib, _ = load()
        self.handle = ctypes.c_void_p()
        error = Error()
        check(self.lib.m3_graph_create(ctypes.byref(self.handle),
                                       ctypes.byref(error)), error)
        self.values = {}

    def add_value(self, role, dtype, shape):
        desc = ValueDesc()
        self.lib.m3_graph_value_desc_init(ctypes.byref(desc), role, dtype,
                                          len(shape), _shape_array(shape))
        value = ctypes.c_uint32()
        error = Error()
        check(self.lib.m3_graph_add_value(self.handle, ctypes.byref(desc),
                                          ctypes.byref(value),
                                          ctypes.byref(error)), error)
        self.values[value.value] = (dtype, tuple(shape), role)
        return value.value

    def set_constant(self, value, array):
        error = Error()
        data = array.ctypes.data_as(ctypes.c_void_p)
        check(self.lib.m3_graph_set_constant(self.handle, value, data,
                                             array.nbytes,
                                             ctypes.byref(error)), error)

    def add_node(self, kind, inputs, outputs):
        node = NodeDesc()
        self.lib.m3_graph_node_desc_init(ctypes.byref(node), kind)
        for i, value in enumerate(inputs):
            node.inputs[i] = value
        for i, value in enumerate(outputs):
            node.outputs[i] = value
        error = Error()
        check(self.lib.m3_graph_add_node(self.handle, ctypes.byref(node),
                                         ctypes.byref(error)), error)

    def add_inferred(self, kind, inputs, role, dtype, output_index=0):
        """m3_graph_add_inferred_value: a new value whose shape (and, for
        some kinds, dtype) is inferred from a node of `kind` over
        `inputs`; returns its id."""
        node = NodeDesc()
        self.lib.m3_graph_node_desc_init(ctypes.byref(node), kind)
        for i, value in enumerate(inputs):
            node.inputs[i] = value
        value = ctypes.c_uint32()
        error = Error()
        check(self.lib.m3_graph_add_inferred_value(
            self.handle, ctypes.byref(node), output_index, role, dtype,
            ctypes.byref(value), ctypes.byref(error)), error)
        self.values[value.value] = (dtype, None, role)
        return value.value

    def free(self):
        if self.handle:
            self.lib.m3_graph_free(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Session:
    """Owner of an m3_session (public API), with HIP timing access."""

    def __init__(self, graph, allow_metal=True, allow_cpu=True,
                 allow_neural_engine=True):
        self.lib, self.hip = load()
        self.handle = ctypes.c_void_p()
        options = SessionOptions(allow_neural_engine, allow_metal, allow_cpu)
        error = Error()
        check(self.lib.m3_session_create(ctypes.byref(self.handle),
                                         graph.handle, ctypes.byref(options),
                                         ctypes.byref(error)), error)
        self.values = dict(graph.values)

    def write(self, value, array):
        error = Error()
        check(self.lib.m3_session_write_input(
            self.handle, value, array.ctypes.data_as(ctypes.c_void_p),
            array.nbytes, ctypes.byref(error)), error)

    def read(self, value, out):
        error = Error()
        check(self.lib.m3_session_read_output(
            self.handle, value, out.ctypes.data_as(ctypes.c_void_p),
            out.nbytes, ctypes.byref(error)), error)
        return out

    def run(self):
        error = Error()
        status = self.lib.m3_session_run(self.handle, ctypes.byref(error))
        check(status, error)

    def plan(self):
        info = PlanInfo()
        error = Error()
        check(self.lib.m3_session_get_plan_info(self.handle,
                                                ctypes.byref(info),
                                                ctypes.byref(error)), error)
        return info

    def provider(self, node):
        kind = ctypes.c_int()
        error = Error()
        check(self.lib.m3_session_get_node_provider(
            self.handle, node, ctypes.byref(kind), ctypes.byref(error)),
            error)
        return kind.value

    def hip_device(self):
        backend = self.lib.m3_session_backend(self.handle)
        return self.lib.m3_backend_hip_device(backend)

    def host_waits(self):
        """How many times the host has waited for this session's stream."""
        waits = ctypes.c_uint64(0)
        check_hip = self.hip.m3_hip_host_waits(self.hip_device(),
                                               ctypes.byref(waits))
        if check_hip != 0:
            raise M3Error(INTERNAL, "m3_hip_host_waits failed")
        return waits.value

    def timing_enable(self, enabled):
        """True: events on every launch; "stream": the same stream waits
        without events (for an external profiler); False: off."""
        mode = 2 if enabled == "stream" else 1 if enabled else 0
        self.hip.m3_hip_timing_enable(self.hip_device(), mode)

    def timing_reset(self):
        self.hip.m3_hip_timing_reset(self.hip_device())

    def timing_read(self):
        entries = (HipKernelTime * 64)()
        count = ctypes.c_size_t()
        message = ctypes.create_string_buffer(256)
        status = self.hip.m3_hip_timing_read(self.hip_device(), entries, 64,
                                             ctypes.byref(count), message,
                                             256)
        if status != 0:
            raise M3Error(INTERNAL, message.value.decode())
        return {entries[i].name.decode(): (entries[i].launches,
                                           entries[i].total_ms)
                for i in range(min(count.value, 64))}

    def timing_samples(self, name, capacity=4096):
        """Durations (ms) of the launches of kernel `name` since the last
        timing reset, in launch order."""
        durations = (ctypes.c_float * capacity)()
        count = ctypes.c_size_t()
        message = ctypes.create_string_buffer(256)
        status = self.hip.m3_hip_timing_samples(
            self.hip_device(), name.encode(), durations, capacity,
            ctypes.byref(count), message, 256)
        if status != 0:
            raise M3Error(INTERNAL, message.value.decode())
        return [float(durations[i]) for i in range(min(count.value,
                                                       capacity))]

    def free(self):
        if self.handle:
            self.lib.m3_session_free(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def rng_fill(kind, count, seed, sequence=0, a=0.0, b=1.0, rng=None):
    """Draws `count` float32 values from the library's PCG32 stream.

    kind "uniform": a + (b - a) * U[0,1); kind "normal": a * N(0, 1).
    Pass `rng` (an Rng from rng_new) to continue one stream across calls.
    """
    import numpy as np
    lib, _ = load()
    if rng is None:
        rng = rng_new(seed, sequence)
    out = np.empty(count, dtype=np.float32)
    error = Error()
    ptr = out.ctypes.data_as(ctypes.c_void_p)
    if kind == "uniform":
        status = lib.m3_rng_uniform_f32_fill(ctypes.byref(rng), ptr, count,
                                             a, b, ctypes.byref(error))
    else:
        status = lib.m3_rng_normal_f32_fill_scaled(ctypes.byref(rng), ptr,
                                                   count, a,
                                                   ctypes.byref(error))
    check(status, error)
    return out


def rng_new(seed, sequence=0):
    lib, _ = load()
    rng = Rng()
    error = Error()
    check(lib.m3_rng_seed(ctypes.byref(rng), seed, sequence,
                          ctypes.byref(error)), error)
    return rng
