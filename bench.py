"""Benchmark of the m3 HIP execution provider on one MI355X.

A step is one ``m3_session_run`` of a graph built through the public API
(include/m3.h), with its inputs already resident in HBM. The headline
workload is last-axis softmax F32 on an attention-score tensor
[16, 1024, 1024] (logits ~ N(0, 3), strict upper triangle -inf); the other
op classes (broadcast MUL, the four casts, Snake1d, TANH, GATED_SILU, the
30-step Euler CFG graph) are measured the same way and reported under
``op_classes``; ``executor`` times the reference's flow math issued one
command per m3_command_executor_execute call.

For every class:
  * ms_per_run    wall time of m3_session_run (includes the softmax NaN
                  scan, launches and the closing stream synchronize);
  * kernel_us     average duration of the dominant kernel from the HIP
                  events the library attaches to each of its dispatches
                  (hipExtLaunchKernelGGL on the session's own stream), with
                  the median over runs and the fastest and slowest run
                  beside it (VALU-bound kernels vary with the GPU clock);
  * GB/s          algorithmic bytes (unique tensor bytes read + written)
                  divided by those times; peak HBM is 8.0 TB/s.
Sessions rotate so that the inputs read between two runs of one session
total at least 512 MB, twice the 256 MB Infinity Cache: outputs are written
with streaming stores that do not stay in it, so only inputs could be
served from it, and with this rotation every run reads its inputs from HBM.

The CPU baseline times the reference's own CPU provider (compiled from its
sources into oracle/_ref when the reference tree was present) or, without
it, the oracle restatement, single-threaded as the reference is, on the
sample stated in the output. Every class is also checked bit for bit
against that CPU result.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import ctypes
import importlib.util
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PEAK_GBPS = 8000.0
CACHE_DEFEAT_BYTES = 512 << 20  # input bytes between two runs of a session
# --no-events: the timed pass waits on the stream after each run as usual
# but attaches no timing events, for runs under an external kernel
# profiler (whose trace then gives the kernel durations)
EVENTS = True
# Host pause (seconds) before each run of the event-timed pass: the GPU
# then idles that much longer before each run's first kernel, as it does
# under a kernel profiler, which adds its own host work to every dispatch.
PAUSE = 0.0


def pause():
    if PAUSE > 0.0:
        end = time.perf_counter() + PAUSE
        while time.perf_counter() < end:
            pass
METRIC = ("achieved HBM GB/s (% of MI355X peak) per op class; "
          "ms per m3_session_run")


def _package():
    spec = importlib.util.spec_from_file_location(
        "m3c_amd", os.path.join(ROOT, "m3.c_amd", "__init__.py"))
    module = importlib.util.module_from_spec(spec)
    sys.modules["m3c_amd"] = module
    spec.loader.exec_module(module)
    return module


m3 = _package()


def log(*parts):
    print(*parts, file=sys.stderr, flush=True)


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter passes
    (profiles/hbm_traffic.json: FETCH_SIZE and WRITE_SIZE, each scaled by
    the same counter's reading for a plain copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as handle:
            table = json.load(handle)
    except (OSError, ValueError):
        return None
    entry = table.get("kernels", {}).get(kernel)
    return None if entry is None else entry.get("traffic_bytes")


# ---- CPU baseline (oracle/_ref or the oracle) ------------------------------

class CpuBaseline:
    """The reference CPU provider (kind "reference") or the oracle ("port")."""

    def __init__(self):
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import harness  # noqa: E402  (test harness, loaded only for this leg)
        self.harness = harness
        self.kind = "reference" if harness.ref_available() else "port"

    def run(self, kind, storages, views):
        if self.kind == "reference":
            return self.harness.run_ref(kind, storages, views)
        return self.harness.run_oracle(kind, storages, views)

    def timed(self, kind, storages, views, runs=3):
        """The result and the median wall time of `runs` runs."""
        seconds = []
        for _ in range(runs):
            start = time.perf_counter()
            status, out = self.run(kind, storages, views)
            seconds.append(time.perf_counter() - start)
        return status, out, float(np.median(seconds))


def cpu_model():
    """The host CPU's model name, as /proc/cpuinfo gives it."""
    try:
        with open("/proc/cpuinfo") as handle:
            for line in handle:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


# ---- workloads -------------------------------------------------------------

def softmax_input(rows_per_matrix=1024, matrices=16, seed=0):
    n = rows_per_matrix
    s = m3.rng_fill("normal", matrices * n * n, seed=seed, a=3.0)
    s = s.reshape(matrices, n, n)
    mask = np.triu(np.ones((n, n), dtype=bool), k=1)
    s[:, mask] = -np.inf
    return s


def cast_inputs(n=4096, seed=0):
    rng = m3.rng_new(seed, 0)
    t = m3.rng_fill("normal", n * n, seed=seed, a=1000.0, rng=rng)
    pick = m3.rng_fill("uniform", n * n, seed=seed, rng=rng)
    special_kind = m3.rng_fill("uniform", n * n, seed=seed, a=0.0, b=6.0,
                               rng=rng)
    payload = (m3.rng_fill("uniform", n * n, seed=seed, a=0.0,
                           b=float(1 << 22), rng=rng)).astype(np.uint32)
    bits = t.view(np.uint32).copy()
    special = pick < 0.05
    kinds = special_kind.astype(np.uint32)
    table = [
        payload & 0x7fffff,                       # subnormal
        np.zeros_like(payload),                   # +0
        np.full_like(payload, 0x80000000),        # -0
        np.full_like(payload, 0x7f800000),        # +inf
        np.full_like(payload, 0xff800000),        # -inf
        0x7f800000 | (payload | 1),               # NaN payloads (q and s)
    ]
    chosen = np.choose(np.minimum(kinds, 5), table).astype(np.uint32)
    signs = (payload & 1).astype(np.uint32) << 31
    chosen = np.where(kinds == 5, chosen | signs, chosen)
    bits[special] = chosen[special]
    t = bits.view(np.float32).reshape(n, n)
    half = t.astype(np.float16).view(np.uint16)
    brain = (t.view(np.uint32) >> 16).astype(np.uint16)
    return t, half, brain


class Workload:
    """One graph, `rotate` independent sessions of it, and its CPU check."""

    def __init__(self, name, build, inputs, algorithmic_bytes, kernel,
                 rotate, cpu):
        self.name = name
        self.algorithmic_bytes = algorithmic_bytes
        self.kernel = kernel
        self.sessions = []
        self.outputs = None
        self.cpu = cpu
        input_bytes = sum(a.nbytes for a in inputs)
        rotate = max(rotate, -(-CACHE_DEFEAT_BYTES // max(input_bytes, 1)))
        self.rotate = rotate
        for _ in range(rotate):
            graph, feeds, outputs = build()
            session = m3.Session(graph)
            graph.free()
            for value, array in feeds:
                session.write(value, array)
            self.sessions.append(session)
            self.outputs = outputs
            self.feeds = feeds
        for session in self.sessions:
            for node in range(session.plan().node_count):
                if session.provider(node) != m3.PROVIDER_HIP:
                    raise RuntimeError("%s: node %d is not on the HIP "
                                       "provider" % (name, node))
        self.inputs = inputs

    def measure(self, steps, warmup):
        # every session runs at least once before timing: a session's first
        # run after an input write includes that input's data scan, which
        # later runs on the unchanged input skip (measured separately by
        # measure_after_write)
        for i in range(max(warmup, len(self.sessions))):
            self.sessions[i % len(self.sessions)].run()
        for session in self.sessions:
            session.timing_reset()
            session.timing_enable(False)
        start = time.perf_counter()
        for i in range(steps):
            self.sessions[i % len(self.sessions)].run()
        wall = (time.perf_counter() - start) / steps
        # The same steps again, back to back, with the library's timing
        # events on every dispatch; the durations are read once at the end,
        # so the runs follow each other as in the wall-clock pass (a host
        # pause of tens of microseconds between runs slows the VALU-heavy
        # kernels that follow it). Each run's dominant-kernel average is
        # kept, for the median beside the mean (VALU-bound kernels vary
        # with the clock from run to run). Unmeasured timed runs come first,
        # as many per session as the measured pass makes, so that every
        # session's event pool already holds the events it will use (a
        # launch that has to create its events reads a microsecond or two
        # long).
        visits = -(-steps // len(self.sessions))
        mode = True if EVENTS else "stream"
        for session in self.sessions:
            session.timing_enable(mode)
            for _ in range(visits):
                session.run()
            session.timing_reset()
        # runs of this workload before the event-timed pass (warm-up,
        # wall-clock pass, event pool warm-up): a kernel trace of the
        # process finds the timed pass's dispatches after as many runs
        self.runs_before_timed = (max(warmup, len(self.sessions)) + steps +
                                  visits * len(self.sessions))
        for i in range(steps):
            pause()
            self.sessions[i % len(self.sessions)].run()
        per_kernel = {}
        per_session = []
        for session in self.sessions:
            for name, (count, ms) in session.timing_read().items():
                previous = per_kernel.get(name, (0, 0.0))
                per_kernel[name] = (previous[0] + count, previous[1] + ms)
            samples = []
            for name in self.kernel:
                samples = session.timing_samples(name)
                if samples:
                    break
            per_session.append(samples)
            session.timing_enable(False)
        launches = sum(per_kernel.get(name, (0, 0.0))[0]
                       for name in self.kernel)
        total_ms = sum(per_kernel.get(name, (0, 0.0))[1]
                       for name in self.kernel)
        # session j ran steps j, j + n, ...: its k-th group of launches is
        # step j + k n
        self.run_kernel_us = []
        per_run = max(launches // steps, 1)
        for i in range(steps):
            n = len(self.sessions)
            samples = per_session[i % n]
            chunk = samples[(i // n) * per_run:(i // n + 1) * per_run]
            if chunk:
                self.run_kernel_us.append(1000.0 * sum(chunk) / len(chunk))
        kernel_us = 1000.0 * total_ms / max(launches, 1)
        runs_kernel_ms = sum(ms for _, ms in per_kernel.values()) / steps
        return wall * 1000.0, kernel_us, launches // steps, per_kernel, \
            runs_kernel_ms

    def measure_after_write(self, feeds_of, repeats=5):
        """Median wall time of write_input + run (the input scan included)
        and of the run alone right after the write."""
        totals, runs = [], []
        for i in range(repeats):
            session = self.sessions[i % len(self.sessions)]
            start = time.perf_counter()
            for value, array in feeds_of():
                session.write(value, array)
            middle = time.perf_counter()
            session.run()
            end = time.perf_counter()
            totals.append(end - start)
            runs.append(end - middle)
        return (1000.0 * float(np.median(runs)),
                1000.0 * float(np.median(totals)))

    def read_output(self, index=0):
        value, shape, dtype = self.outputs
        out = np.empty(shape, dtype=dtype)
        return self.sessions[index].read(value, out)

    def free(self):
        for session in self.sessions:
            session.free()
        self.sessions = []


def build_softmax(s):
    def build():
        graph = m3.Graph()
        vin = graph.add_value(m3.INPUT, m3.F32, s.shape)
        vout = graph.add_value(m3.OUTPUT, m3.F32, s.shape)
        graph.add_node(m3.OP_SOFTMAX, [vin], [vout])
        return graph, [(vin, s)], (vout, s.shape, np.float32)
    return build


def build_attention(scores, causal):
    def build():
        shape = scores.shape
        graph = m3.Graph()
        vs = graph.add_value(m3.INPUT, m3.F32, shape)
        vscale = graph.add_value(m3.CONSTANT, m3.F32, (1,))
        vmask = graph.add_value(m3.CONSTANT, m3.F32, causal.shape)
        graph.set_constant(vscale, np.array([0.125], np.float32))
        graph.set_constant(vmask, causal)
        t0 = graph.add_value(m3.TEMPORARY, m3.F32, shape)
        graph.add_node(m3.OP_MUL, [vs, vscale], [t0])
        t1 = graph.add_value(m3.TEMPORARY, m3.F32, shape)
        graph.add_node(m3.OP_ADD, [t0, vmask], [t1])
        vy = graph.add_value(m3.OUTPUT, m3.F32, shape)
        graph.add_node(m3.OP_SOFTMAX, [t1], [vy])
        return graph, [(vs, scores)], (vy, shape, np.float32)
    return build


def build_mul(x, c):
    def build():
        graph = m3.Graph()
        vx = graph.add_value(m3.INPUT, m3.F32, x.shape)
        vc = graph.add_value(m3.CONSTANT, m3.F32, c.shape)
        vy = graph.add_value(m3.OUTPUT, m3.F32, x.shape)
        graph.set_constant(vc, c)
        graph.add_node(m3.OP_MUL, [vx, vc], [vy])
        return graph, [(vx, x)], (vy, x.shape, np.float32)
    return build


def build_cast(src, src_dtype, dst_dtype, dst_np):
    def build():
        graph = m3.Graph()
        vin = graph.add_value(m3.INPUT, src_dtype, src.shape)
        vout = graph.add_value(m3.OUTPUT, dst_dtype, src.shape)
        graph.add_node(m3.OP_CAST, [vin], [vout])
        return graph, [(vin, src)], (vout, src.shape, dst_np)
    return build


def build_snake(x, alpha):
    def build():
        graph = m3.Graph()
        vx = graph.add_value(m3.INPUT, m3.F32, x.shape)
        va = graph.add_value(m3.CONSTANT, m3.F32, alpha.shape)
        vy = graph.add_value(m3.OUTPUT, m3.F32, x.shape)
        graph.set_constant(va, alpha)
        graph.add_node(m3.OP_SNAKE1D, [vx, va], [vy])
        return graph, [(vx, x)], (vy, x.shape, np.float32)
    return build


def build_tanh(x):
    def build():
        graph = m3.Graph()
        vx = graph.add_value(m3.INPUT, m3.F32, x.shape)
        vy = graph.add_value(m3.OUTPUT, m3.F32, x.shape)
        graph.add_node(m3.OP_TANH, [vx], [vy])
        return graph, [(vx, x)], (vy, x.shape, np.float32)
    return build


def build_gated_silu(gate, up, dtype, out_np):
    def build():
        graph = m3.Graph()
        vg = graph.add_value(m3.INPUT, dtype, gate.shape)
        vu = graph.add_value(m3.INPUT, dtype, up.shape)
        vy = graph.add_value(m3.OUTPUT, dtype, gate.shape)
        graph.add_node(m3.OP_GATED_SILU, [vg, vu], [vy])
        return graph, [(vg, gate), (vu, up)], (vy, gate.shape, out_np)
    return build


def build_euler(x, vus, vcs, scale=3.0, dt=1.0 / 30.0):
    """30-step CFG + Euler graph in the reference's op order
    (src/m3_flow_solver_math.c:36-135): a = vu*(-1); a = vc + a; a = a*s;
    v = vu + a; b = v*dt; x = x + b."""
    def build():
        graph = m3.Graph()
        shape = x.shape
        vx = graph.add_value(m3.INPUT, m3.F32, shape)
        consts = {}
        for name, value in (("minus_one", -1.0), ("scale", scale),
                            ("dt", dt)):
            vid = graph.add_value(m3.CONSTANT, m3.F32, (1,))
            graph.set_constant(vid, np.array([value], np.float32))
            consts[name] = vid
        current = vx
        steps = len(vus)
        for k in range(steps):
            vu = graph.add_value(m3.CONSTANT, m3.F32, shape)
            vc = graph.add_value(m3.CONSTANT, m3.F32, shape)
            graph.set_constant(vu, vus[k])
            graph.set_constant(vc, vcs[k])
            t = [graph.add_value(m3.TEMPORARY, m3.F32, shape)
                 for _ in range(5)]
            nxt = graph.add_value(m3.OUTPUT if k == steps - 1
                                  else m3.TEMPORARY, m3.F32, shape)
            graph.add_node(m3.OP_MUL, [vu, consts["minus_one"]], [t[0]])
            graph.add_node(m3.OP_ADD, [vc, t[0]], [t[1]])
            graph.add_node(m3.OP_MUL, [t[1], consts["scale"]], [t[2]])
            graph.add_node(m3.OP_ADD, [vu, t[2]], [t[3]])
            graph.add_node(m3.OP_MUL, [t[3], consts["dt"]], [t[4]])
            graph.add_node(m3.OP_ADD, [current, t[4]], [nxt])
            current = nxt
        return graph, [(vx, x)], (current, shape, np.float32)
    return build


class FlowExecutor:
    """The flow math of the reference run the way its flow code runs it
    (src/m3_flow_solver_math.c:36-135): one command per
    m3_command_executor_execute call on a HIP backend, the one-element
    scalar rewritten from the host between commands. Buffers: velocity
    [2, L, C] (conditional half, unconditional half), latent and arithmetic
    [1, L, C]."""

    def __init__(self, length, channels):
        self.lib, self.hip = m3.load()
        self.backend = ctypes.c_void_p()
        error = m3.Error()
        m3.check(self.lib.m3_backend_create_hip(ctypes.byref(self.backend),
                                                ctypes.byref(error)), error)
        self.shape = (1, length, channels)
        self.bytes = 4 * length * channels
        self.storages = {}
        for name, size in (("velocity", 2 * self.bytes),
                           ("latent", self.bytes), ("arith", self.bytes),
                           ("scalar", 4)):
            storage = ctypes.c_void_p()
            m3.check(self.lib.m3_storage_allocate(
                self.backend, size, 256, ctypes.byref(storage),
                ctypes.byref(error)), error)
            self.storages[name] = storage
        self.views = {}
        for name, storage, shape, offset in (
                ("cond", "velocity", self.shape, 0),
                ("uncond", "velocity", self.shape, self.bytes),
                ("latent", "latent", self.shape, 0),
                ("arith", "arith", self.shape, 0),
                ("scalar", "scalar", (1,), 0)):
            view = m3.TensorView()
            dims = (ctypes.c_uint64 * 8)(*shape)
            m3.check(self.lib.m3_tensor_view_contiguous(
                ctypes.byref(view), self.storages[storage], m3.F32,
                len(shape), dims, offset, ctypes.byref(error)), error)
            self.views[name] = view
        self.executor = (ctypes.c_uint8 * 64)()
        self.lib.m3_command_executor_init(self.executor, self.backend)
        self.lib.m3_command_executor_execute.argtypes = [
            ctypes.c_void_p, ctypes.POINTER(m3.Command), ctypes.c_size_t,
            ctypes.POINTER(m3.Error)]
        self.finish_each = False

    def write(self, name, array):
        array = np.ascontiguousarray(array, np.float32)
        error = m3.Error()
        m3.check(self.lib.m3_storage_write(
            self.storages[name], 0, array.ctypes.data_as(ctypes.c_void_p),
            array.nbytes, ctypes.byref(error)), error)

    def read(self, name):
        out = np.zeros(self.shape, np.float32)
        error = m3.Error()
        m3.check(self.lib.m3_storage_read(
            self.storages[name], 0, out.ctypes.data_as(ctypes.c_void_p),
            out.nbytes, ctypes.byref(error)), error)
        return out

    def finish(self):
        error = m3.Error()
        m3.check(self.lib.m3_backend_finish(self.backend,
                                            ctypes.byref(error)), error)

    def op(self, kind, left, right, output):
        command = m3.Command()
        command.kind = kind
        for i, name in enumerate((left, right, output)):
            command.descriptor.views[i] = ctypes.pointer(self.views[name])
        error = m3.Error()
        m3.check(self.lib.m3_command_executor_execute(
            self.executor, ctypes.byref(command), 1, ctypes.byref(error)),
            error)
        if self.finish_each:
            self.finish()

    def step(self, guidance, delta):
        """Guided velocity then one Euler step: 3 scalar writes, 6 lists."""
        self.write("scalar", [-1.0])
        self.op(m3.OP_MUL, "uncond", "scalar", "arith")
        self.op(m3.OP_ADD, "cond", "arith", "arith")
        self.write("scalar", [guidance])
        self.op(m3.OP_MUL, "arith", "scalar", "arith")
        self.op(m3.OP_ADD, "uncond", "arith", "arith")
        self.write("scalar", [delta])
        self.op(m3.OP_MUL, "arith", "scalar", "arith")
        self.op(m3.OP_ADD, "latent", "arith", "latent")

    def timing(self, enabled):
        device = self.lib.m3_backend_hip_device(self.backend)
        self.hip.m3_hip_timing_reset(device)
        self.hip.m3_hip_timing_enable(device, 1 if enabled else 0)

    def kernel_ms(self):
        device = self.lib.m3_backend_hip_device(self.backend)
        entries = (m3.HipKernelTime * 64)()
        count = ctypes.c_size_t()
        message = ctypes.create_string_buffer(256)
        self.hip.m3_hip_timing_read(device, entries, 64, ctypes.byref(count),
                                    message, 256)
        return {entries[i].name.decode(): (entries[i].launches,
                                           entries[i].total_ms)
                for i in range(count.value)}

    def free(self):
        self.lib.m3_command_executor_dispose(self.executor)
        for storage in self.storages.values():
            self.lib.m3_storage_free(storage)
        self.lib.m3_backend_free(self.backend)


def spec(storage, dtype, shape, strides=None):
    return baseline_harness().ViewSpec(storage, dtype, tuple(shape), strides)


_HARNESS = None


def baseline_harness():
    global _HARNESS
    if _HARNESS is None:
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import harness
        _HARNESS = harness
    return _HARNESS


def as_bytes(array):
    return np.ascontiguousarray(array).view(np.uint8).reshape(-1).copy()


def result_entry(name, workload, wall_ms, kernel_us, launches, bytes_total,
                 kernel_bytes, parity, cpu_seconds=None, cpu_bytes=None):
    launches = launches if EVENTS else None
    kernel_gbps = kernel_bytes / (kernel_us * 1e-6) / 1e9 if kernel_us else 0
    entry = {
        "op_class": name,
        "algorithmic_bytes_per_run": bytes_total,
        "ms_per_run": round(wall_ms, 4),
        "run_GBps": round(bytes_total / (wall_ms * 1e-3) / 1e9, 1),
        "kernel": workload.kernel[0],
        "kernel_launches_per_run": launches,
        "kernel_us": round(kernel_us, 3),
        "kernel_GBps": round(kernel_gbps, 1),
        "kernel_frac_of_peak": round(kernel_gbps / PEAK_GBPS, 4),
        "parity": parity,
    }
    runs = getattr(workload, "run_kernel_us", None)
    if runs:
        median_us = float(np.median(runs))
        entry["kernel_us_median"] = round(median_us, 3)
        entry["kernel_frac_of_peak_median"] = round(
            kernel_bytes / (median_us * 1e-6) / 1e9 / PEAK_GBPS, 4)
        entry["kernel_us_min_max"] = [round(min(runs), 3),
                                      round(max(runs), 3)]
        entry["kernel_us_runs"] = [round(u, 2) for u in runs]
    if hasattr(workload, "runs_before_timed"):
        entry["runs_before_timed_pass"] = workload.runs_before_timed
    if cpu_seconds is not None:
        entry["cpu_GBps"] = round(cpu_bytes / cpu_seconds / 1e9, 4)
    return entry


def main():
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--rotate", type=int, default=4)
    parser.add_argument("--classes",
                        default="softmax,attention,softmax_wide,mul,cast,"
                                "copy,snake,tanh,gated_silu,euler,executor",
                        help="comma-separated op classes to run")
    parser.add_argument("--no-cpu", action="store_true",
                        help="skip the CPU baseline and CPU parity check")
    parser.add_argument("--no-events", action="store_true",
                        help="no timing events in the timed pass (run it "
                             "under a kernel profiler for the durations)")
    parser.add_argument("--pause-us", type=float, default=0.0,
                        help="host pause before each run of the timed "
                             "pass, in microseconds (default none)")
    args = parser.parse_args()
    global EVENTS, PAUSE
    EVENTS = not args.no_events
    PAUSE = max(args.pause_us, 0.0) * 1e-6
    if args.gpus != 1:
        print("bench.py measures one GPU: this provider has no multi-GPU "
              "path (each op shards with zero exchange; see the design "
              "notes). Run with --gpus 1.", file=sys.stderr)
        return 2
    m3.load()
    if m3.hip_device_count() == 0:
        print("no HIP device visible: the HIP provider cannot run",
              file=sys.stderr)
        return 1
    classes = [c for c in args.classes.split(",") if c]
    cpu = None if args.no_cpu else CpuBaseline()
    results = {}
    headline = None
    cpu_line = None

    if "softmax" in classes:
        log("softmax: generating [16,1024,1024] logits")
        s = softmax_input()
        nbytes = 2 * s.nbytes
        w = Workload("softmax", build_softmax(s), [s], nbytes,
                     ["m3_softmax_rows"], args.rotate, cpu)
        wall, kus, launches, kernels, _ = w.measure(args.steps, args.warmup)
        parity = None
        cpu_seconds = None
        if cpu is not None:
            out = w.read_output()
            status, storages, cpu_seconds = cpu.timed(
                m3.OP_SOFTMAX, [as_bytes(s), np.zeros(s.nbytes, np.uint8)],
                [spec(0, m3.F32, s.shape), spec(1, m3.F32, s.shape)])
            ref = storages[1].view(np.float32).reshape(s.shape)
            mismatches = int(np.count_nonzero(ref.view(np.uint32) !=
                                              out.view(np.uint32)))
            parity = "bit-exact" if mismatches == 0 else \
                "%d of %d elements differ" % (mismatches, s.size)
            cpu_line = {"value": round(nbytes / cpu_seconds / 1e9, 4),
                        "unit": "GB/s", "cores": 1, "kind": cpu.kind,
                        "model": cpu_model(),
                        "runs": 3,
                        "sample": "the full [16,1024,1024] softmax, median "
                                  "of 3 runs of the single-threaded CPU "
                                  "provider"}
        results["softmax"] = result_entry("softmax", w, wall, kus, launches,
                                          nbytes, nbytes, parity, cpu_seconds,
                                          nbytes)
        results["softmax"]["kernels"] = {k: v[1] / max(v[0], 1) * 1000
                                         for k, v in kernels.items()}
        # a run right after the input was written: the NaN scan (one extra
        # read of the input, 67.1 MB) is then part of the run
        run_ms, write_run_ms = w.measure_after_write(lambda: w.feeds)
        results["softmax"]["ms_per_run_after_write"] = round(run_ms, 4)
        results["softmax"]["ms_write_input_and_run"] = round(write_run_ms, 4)
        results["softmax"]["nan_scan_bytes"] = s.nbytes
        headline = (w.rotate, wall, kus, nbytes)
        w.free()
        log("softmax:", json.dumps(results["softmax"]))

    if "attention" in classes:
        # scores * scale + causal mask -> SOFTMAX in one run: the softmax
        # input is produced inside the run (by the fused scale-and-mask
        # program) and checked for NaN on the device before the softmax,
        # with one host wait per run
        log("attention: generating [16,1024,1024] scores")
        shape = (16, 1024, 1024)
        scores = m3.rng_fill("normal", int(np.prod(shape)), seed=0,
                             a=8.0).reshape(shape)
        causal = np.where(np.triu(np.ones(shape[1:], bool), 1), -np.inf,
                          0.0).astype(np.float32)
        unique = 2 * scores.nbytes + causal.nbytes
        w = Workload("attention", build_attention(scores, causal),
                     [scores], unique, ["m3_softmax_rows"], args.rotate, cpu)
        wall, kus, launches, kernels, run_kernel_ms = w.measure(
            args.steps, args.warmup)
        parity = None
        if cpu is not None:
            out = w.read_output()
            f = np.float32
            logits = ((scores * f(0.125)).astype(f) + causal).astype(f)
            status, storages = cpu.run(
                m3.OP_SOFTMAX, [as_bytes(logits),
                                np.zeros(logits.nbytes, np.uint8)],
                [spec(0, m3.F32, shape), spec(1, m3.F32, shape)])
            ref = storages[1].view(np.float32).reshape(shape)
            mismatches = int(np.count_nonzero(ref.view(np.uint32) !=
                                              out.view(np.uint32)))
            parity = ("bit-exact vs float32 scale and mask, then the CPU "
                      "provider's softmax" if mismatches == 0 else
                      "%d of %d elements differ" % (mismatches, scores.size))
        # host waits of one plain run (the completion-word path)
        session = w.sessions[0]
        before = session.host_waits()
        session.run()
        waits_per_run = session.host_waits() - before
        entry = result_entry("attention", w, wall, kus, launches, unique,
                             2 * scores.nbytes, parity)
        entry["kernels"] = {k: v[1] / max(v[0], 1) * 1000
                            for k, v in kernels.items()}
        entry["kernel_time_per_run_ms"] = round(run_kernel_ms, 4)
        entry["host_waits_per_run"] = waits_per_run
        entry["hbm_bytes_per_run"] = (3 * scores.nbytes + causal.nbytes +
                                      3 * scores.nbytes)
        results["attention"] = entry
        w.free()
        log("attention:", json.dumps(results["attention"]))

    if "softmax_wide" in classes:
        log("softmax_wide: generating [4096,16384] logits")
        s = m3.rng_fill("normal", 4096 * 16384, seed=1, a=3.0).reshape(
            4096, 16384)
        nbytes = 2 * s.nbytes
        w = Workload("softmax_wide", build_softmax(s), [s], nbytes,
                     ["m3_softmax_rows_wide", "m3_softmax_rows_streamed"], args.rotate, cpu)
        wall, kus, launches, kernels, _ = w.measure(args.steps, args.warmup)
        parity = None
        cpu_seconds = None
        if cpu is not None:
            out = w.read_output()
            status, storages, cpu_seconds = cpu.timed(
                m3.OP_SOFTMAX, [as_bytes(s), np.zeros(s.nbytes, np.uint8)],
                [spec(0, m3.F32, s.shape), spec(1, m3.F32, s.shape)])
            ref = storages[1].view(np.float32).reshape(s.shape)
            mismatches = int(np.count_nonzero(ref.view(np.uint32) !=
                                              out.view(np.uint32)))
            parity = "bit-exact" if mismatches == 0 else \
                "%d of %d elements differ" % (mismatches, s.size)
        results["softmax_wide"] = result_entry(
            "softmax_wide", w, wall, kus, launches, nbytes, nbytes, parity,
            cpu_seconds, nbytes)
        results["softmax_wide"]["kernels"] = {
            k: v[1] / max(v[0], 1) * 1000 for k, v in kernels.items()}
        w.free()
        log("softmax_wide:", json.dumps(results["softmax_wide"]))

    if "mul" in classes:
        log("mul: generating x[8,1024,1536], c[1536]")
        rng = m3.rng_new(0, 0)
        x = m3.rng_fill("uniform", 8 * 1024 * 1536, seed=0, a=-1.0, b=1.0,
                        rng=rng).reshape(8, 1024, 1536)
        c = m3.rng_fill("normal", 1536, seed=0, a=1.0, rng=rng)
        nbytes = 2 * x.nbytes + c.nbytes
        w = Workload("mul", build_mul(x, c), [x, c], nbytes,
                     ["m3_binary_mul"], args.rotate, cpu)
        wall, kus, launches, _, _ = w.measure(args.steps, args.warmup)
        parity = None
        cpu_seconds = None
        if cpu is not None:
            out = w.read_output()
            status, storages, cpu_seconds = cpu.timed(
                m3.OP_MUL, [as_bytes(x), as_bytes(c),
                            np.zeros(x.nbytes, np.uint8)],
                [spec(0, m3.F32, x.shape), spec(1, m3.F32, c.shape),
                 spec(2, m3.F32, x.shape)])
            ref = storages[2].view(np.uint32)
            mismatches = int(np.count_nonzero(ref != out.view(np.uint32)
                                              .reshape(-1)))
            parity = "bit-exact" if mismatches == 0 else \
                "%d elements differ" % mismatches
        results["mul"] = result_entry("mul", w, wall, kus, launches, nbytes,
                                      nbytes, parity, cpu_seconds, nbytes)
        w.free()
        log("mul:", json.dumps(results["mul"]))

    if "cast" in classes:
        log("cast: generating [4096,4096] with 5% specials")
        t, half, brain = cast_inputs()
        pairs = [("cast_f32_f16", t, m3.F32, m3.F16, np.uint16,
                  "m3_cast_f32_f16"),
                 ("cast_f16_f32", half, m3.F16, m3.F32, np.float32,
                  "m3_cast_f16_f32"),
                 ("cast_f32_bf16", t, m3.F32, m3.BF16, np.uint16,
                  "m3_cast_f32_bf16"),
                 ("cast_bf16_f32", brain, m3.BF16, m3.F32, np.float32,
                  "m3_cast_bf16_f32")]
        for name, src, sd, dd, dnp, kernel in pairs:
            out_bytes = src.size * np.dtype(dnp).itemsize
            nbytes = src.nbytes + out_bytes
            w = Workload(name, build_cast(src, sd, dd, dnp), [src], nbytes,
                         [kernel], args.rotate, cpu)
            wall, kus, launches, _, _ = w.measure(args.steps, args.warmup)
            parity = None
            cpu_seconds = None
            if cpu is not None:
                out = w.read_output()
                status, storages, cpu_seconds = cpu.timed(
                    m3.OP_CAST, [as_bytes(src), np.zeros(out_bytes,
                                                         np.uint8)],
                    [spec(0, sd, src.shape), spec(1, dd, src.shape)])
                mismatches = int(np.count_nonzero(
                    storages[1] != out.view(np.uint8).reshape(-1)))
                parity = "bit-exact" if mismatches == 0 else \
                    "%d bytes differ" % mismatches
            results[name] = result_entry(name, w, wall, kus, launches,
                                         nbytes, nbytes, parity, cpu_seconds,
                                         nbytes)
            w.free()
            log(name + ":", json.dumps(results[name]))

    if "copy" in classes:
        # A plain device copy of known size (a same-dtype CAST runs the
        # byte-copy kernel): the reference point that scales the HBM
        # traffic counters, and the practical ceiling for the other classes.
        log("copy: [4096,4096] F32 -> F32")
        src = m3.rng_fill("normal", 4096 * 4096, seed=0, a=1.0,
                          rng=m3.rng_new(0, 0)).reshape(4096, 4096)
        nbytes = 2 * src.nbytes
        w = Workload("copy", build_cast(src, m3.F32, m3.F32, np.float32),
                     [src], nbytes, ["m3_copy"], args.rotate, cpu)
        wall, kus, launches, _, _ = w.measure(args.steps, args.warmup)
        out = w.read_output()
        parity = "bit-exact" if np.array_equal(out.view(np.uint32),
                                               src.view(np.uint32)) else \
            "copy differs from its source"
        results["copy"] = result_entry("copy", w, wall, kus, launches,
                                       nbytes, nbytes, parity)
        w.free()
        log("copy:", json.dumps(results["copy"]))

    if "snake" in classes:
        log("snake: generating x[2,1536,65536], alpha[1,1536,1]")
        rng = m3.rng_new(0, 0)
        x = m3.rng_fill("normal", 2 * 1536 * 65536, seed=0, a=1.0,
                        rng=rng).reshape(2, 1536, 65536)
        alpha = m3.rng_fill("uniform", 1536, seed=0, a=0.1, b=2.0,
                            rng=rng).reshape(1, 1536, 1)
        nbytes = 2 * x.nbytes + alpha.nbytes
        w = Workload("snake", build_snake(x, alpha), [x, alpha], nbytes,
                     ["m3_snake1d"], 1, cpu)
        wall, kus, launches, _, _ = w.measure(args.steps, args.warmup)
        parity = None
        cpu_seconds = None
        if cpu is not None:
            out = w.read_output()
            sample = x[:, :96, :]  # 96 channels of both batches (1/16)
            status, storages, cpu_seconds = cpu.timed(
                m3.OP_SNAKE1D, [as_bytes(sample), as_bytes(alpha[:, :96]),
                                np.zeros(sample.nbytes, np.uint8)],
                [spec(0, m3.F32, sample.shape),
                 spec(1, m3.F32, (1, 96, 1)),
                 spec(2, m3.F32, sample.shape)])
            ref = storages[2].view(np.uint32).reshape(sample.shape)
            mismatches = int(np.count_nonzero(
                ref != out[:, :96, :].view(np.uint32)))
            parity = ("bit-exact on the CPU sample (channels 0-95)"
                      if mismatches == 0 else
                      "%d of %d sampled elements differ" %
                      (mismatches, sample.size))
        results["snake"] = result_entry(
            "snake", w, wall, kus, launches, nbytes, nbytes, parity,
            cpu_seconds, 2 * x[:, :96, :].nbytes)
        w.free()
        log("snake:", json.dumps(results["snake"]))

    if "tanh" in classes:
        log("tanh: generating x[2,1536,65536]")
        rng = m3.rng_new(0, 1)
        x = m3.rng_fill("normal", 2 * 1536 * 65536, seed=0, a=1.5,
                        rng=rng).reshape(2, 1536, 65536)
        nbytes = 2 * x.nbytes
        w = Workload("tanh", build_tanh(x), [x], nbytes, ["m3_tanh"], 1,
                     cpu)
        wall, kus, launches, _, _ = w.measure(args.steps, args.warmup)
        parity = None
        cpu_seconds = None
        if cpu is not None:
            out = w.read_output()
            sample = x[:, :96, :]
            status, storages, cpu_seconds = cpu.timed(
                m3.OP_TANH, [as_bytes(sample),
                             np.zeros(sample.nbytes, np.uint8)],
                [spec(0, m3.F32, sample.shape),
                 spec(1, m3.F32, sample.shape)])
            ref = storages[1].view(np.uint32).reshape(sample.shape)
            mismatches = int(np.count_nonzero(
                ref != out[:, :96, :].view(np.uint32)))
            parity = ("bit-exact on the CPU sample (channels 0-95)"
                      if mismatches == 0 else
                      "%d of %d sampled elements differ" %
                      (mismatches, sample.size))
        results["tanh"] = result_entry(
            "tanh", w, wall, kus, launches, nbytes, nbytes, parity,
            cpu_seconds, 2 * x[:, :96, :].nbytes)
        w.free()
        log("tanh:", json.dumps(results["tanh"]))

    if "gated_silu" in classes:
        shape = (16384, 3072)
        log("gated_silu: generating gate and up [16384,3072] F32 and BF16")
        rng = m3.rng_new(0, 2)
        count = shape[0] * shape[1]
        gate = m3.rng_fill("normal", count, seed=0, a=3.0,
                           rng=rng).reshape(shape)
        up = m3.rng_fill("normal", count, seed=0, a=1.0,
                         rng=rng).reshape(shape)
        gate16 = (gate.view(np.uint32) >> 16).astype(np.uint16)
        up16 = (up.view(np.uint32) >> 16).astype(np.uint16)
        for name, dtype, g, u, out_np, kernel in (
                ("gated_silu", m3.F32, gate, up, np.float32,
                 "m3_gated_silu"),
                ("gated_silu_bf16", m3.BF16, gate16, up16, np.uint16,
                 "m3_gated_silu_bf16")):
            nbytes = 3 * g.nbytes
            w = Workload(name, build_gated_silu(g, u, dtype, out_np), [g, u],
                         nbytes, [kernel], 1, cpu)
            wall, kus, launches, _, _ = w.measure(args.steps, args.warmup)
            parity = None
            cpu_seconds = None
            if cpu is not None:
                out = w.read_output()
                rows = 1024
                size = g.itemsize
                status, storages, cpu_seconds = cpu.timed(
                    m3.OP_GATED_SILU,
                    [as_bytes(g[:rows]), as_bytes(u[:rows]),
                     np.zeros(rows * shape[1] * size, np.uint8)],
                    [spec(0, dtype, (rows, shape[1])),
                     spec(1, dtype, (rows, shape[1])),
                     spec(2, dtype, (rows, shape[1]))])
                ref = storages[2].view(out_np).reshape(rows, shape[1])
                mismatches = int(np.count_nonzero(
                    ref.view(np.uint8) != out[:rows].view(np.uint8)))
                parity = ("bit-exact on the CPU sample (rows 0-1023)"
                          if mismatches == 0 else
                          "%d sampled bytes differ" % mismatches)
            results[name] = result_entry(
                name, w, wall, kus, launches, nbytes, nbytes, parity,
                cpu_seconds, 3 * g[:1024].nbytes)
            w.free()
            log(name + ":", json.dumps(results[name]))

    if "euler" in classes:
        log("euler: generating x and 30 x (vu, vc) [2,4096,1536]")
        shape = (2, 4096, 1536)
        count = int(np.prod(shape))
        rng = m3.rng_new(0, 0)
        x = m3.rng_fill("normal", count, seed=0, a=1.0,
                        rng=rng).reshape(shape)
        vus, vcs = [], []
        for _ in range(30):
            vus.append(m3.rng_fill("normal", count, seed=0, a=1.0,
                                   rng=rng).reshape(shape))
            vcs.append(m3.rng_fill("normal", count, seed=0, a=1.0,
                                   rng=rng).reshape(shape))
        tensor = x.nbytes
        nbytes = 15 * tensor * 30
        # one fused program reads x and the 60 per-step tensors and writes
        # the output: 62 tensors of HBM traffic per run
        fused_bytes = (2 * 30 + 2) * tensor
        w = Workload("euler", build_euler(x, vus, vcs), [x] + vus + vcs,
                     nbytes, ["m3_program", "m3_program_interpreted",
                              "m3_binary_add", "m3_binary_mul"], 1, cpu)
        wall, kus, launches, kernels, run_kernel_ms = w.measure(
            args.steps, args.warmup)
        parity = None
        cpu_seconds = None
        if cpu is not None:
            out = w.read_output()
            parity = euler_parity(cpu, x, vus, vcs, out)
        fused = launches == 1
        # the rates use the unique tensor bytes the graph reads and writes
        # (what one fused program moves); the sum over the 180 nodes of
        # their own operand bytes is reported beside them, not as a rate
        entry = result_entry("euler", w, wall, kus, launches, fused_bytes,
                             fused_bytes if fused else nbytes / 180.0,
                             parity)
        entry["kernel_time_per_run_ms"] = round(run_kernel_ms, 4)
        entry["node_sum_bytes_per_run"] = nbytes
        entry["fused_lower_bound_bytes"] = 4 * tensor * 30
        entry["hbm_bytes_per_run"] = fused_bytes if fused else nbytes
        entry["slots"] = None
        results["euler"] = entry
        w.free()
        log("euler:", json.dumps(results["euler"]))

    if "executor" in classes:
        length, channels, steps = 4096, 128, 30
        log("executor: flow math through m3_command_executor_execute, "
            "latent [1,%d,%d], %d steps" % (length, channels, steps))
        rng = np.random.default_rng(5)
        velocity = rng.standard_normal((2, length, channels)).astype(
            np.float32)
        latent0 = rng.standard_normal((1, length, channels)).astype(
            np.float32)
        guidance, delta = 3.0, 1.0 / steps
        flow = FlowExecutor(length, channels)
        flow.write("velocity", velocity)
        timings = {}
        for mode in ("queued", "finish_each"):
            flow.finish_each = mode == "finish_each"
            flow.write("latent", latent0)
            flow.step(guidance, delta)  # warm-up
            flow.write("latent", latent0)
            flow.finish()
            start = time.perf_counter()
            for _ in range(steps):
                flow.step(guidance, delta)
            flow.finish()
            timings[mode] = 1000.0 * (time.perf_counter() - start) / steps
        flow.finish_each = False
        flow.write("latent", latent0)
        flow.timing(True)
        for _ in range(steps):
            flow.step(guidance, delta)
        kernels = flow.kernel_ms()
        flow.timing(False)
        out = flow.read("latent")
        f = np.float32
        expected = latent0.copy()
        cond, uncond = velocity[0:1], velocity[1:2]
        for _ in range(steps):
            a = (uncond * f(-1.0)).astype(f)
            a = (cond + a).astype(f)
            a = (a * f(guidance)).astype(f)
            a = (uncond + a).astype(f)
            a = (a * f(delta)).astype(f)
            expected = (expected + a).astype(f)
        parity = ("bit-exact vs the same float32 operations in numpy"
                  if np.array_equal(out.view(np.uint32),
                                    expected.view(np.uint32))
                  else "latent differs")
        flow.free()
        tensor = 4 * length * channels
        results["executor"] = {
            "op_class": "executor",
            "workload": "per Euler step: guided velocity and one Euler "
                        "update, 3 host scalar writes and 6 single-command "
                        "lists (src/m3_flow_solver_math.c:36-135)",
            "algorithmic_bytes_per_step": 15 * tensor,
            "ms_per_step": round(timings["queued"], 4),
            "ms_per_step_finish_each_list": round(timings["finish_each"], 4),
            "kernel_ms_per_step": round(
                sum(ms for _, ms in kernels.values()) / steps, 4),
            "kernels": {name: [count // steps, round(ms / max(count, 1), 4)]
                        for name, (count, ms) in kernels.items()},
            "parity": parity,
        }
        log("executor:", json.dumps(results["executor"]))

    if headline is None:
        print(json.dumps({"metric": METRIC, "op_classes": results}))
        return 0
    rotation, wall, kus, nbytes = headline
    achieved = nbytes / (kus * 1e-6) / 1e9 if kus else 0.0
    line = {
        "metric": METRIC,
        "value": round(nbytes / (wall * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (PCG32 seed 0, the reference generator)",
        "config": {"workload": "softmax F32 [16,1024,1024], logits ~N(0,3), "
                               "causal -inf upper triangle, one "
                               "m3_session_run per step",
                   "rotating_sessions": rotation},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1),
                     "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBPS, 4),
                     "traffic": measured_traffic("m3_softmax_rows")},
        "cpu_baseline": cpu_line,
        "op_classes": results,
    }
    print(json.dumps(line))
    return 0


def euler_parity(cpu, x, vus, vcs, out):
    """Replays the 30-step graph on the CPU provider for the first 96 rows
    of the latent (the op sequence is elementwise, so any slice is exact)."""
    rows = 96
    xs = np.ascontiguousarray(x[:, :rows, :])
    shape = xs.shape
    scalars = {"m1": np.array([-1.0], np.float32),
               "s": np.array([3.0], np.float32),
               "dt": np.array([1.0 / 30.0], np.float32)}

    def op(kind, a, b):
        status, storages = cpu.run(
            kind, [as_bytes(a), as_bytes(b), np.zeros(a.nbytes, np.uint8)],
            [spec(0, m3.F32, a.shape), spec(1, m3.F32, b.shape),
             spec(2, m3.F32, a.shape)])
        return storages[2].view(np.float32).reshape(a.shape)

    current = xs
    for k in range(len(vus)):
        vu = np.ascontiguousarray(vus[k][:, :rows, :])
        vc = np.ascontiguousarray(vcs[k][:, :rows, :])
        a = op(m3.OP_MUL, vu, scalars["m1"])
        a = op(m3.OP_ADD, vc, a)
        a = op(m3.OP_MUL, a, scalars["s"])
        v = op(m3.OP_ADD, vu, a)
        b = op(m3.OP_MUL, v, scalars["dt"])
        current = op(m3.OP_ADD, current, b)
    got = out[:, :rows, :]
    mismatches = int(np.count_nonzero(current.view(np.uint32) !=
                                      got.view(np.uint32)))
    return ("bit-exact on the CPU sample (rows 0-95)" if mismatches == 0
            else "%d of %d sampled elements differ" % (mismatches,
                                                       current.size))


if __name__ == "__main__":
    sys.exit(main())
