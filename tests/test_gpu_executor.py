"""The command-executor path on the HIP backend (GPU).

The reference's flow code drives the provider one single-command list at a
time through m3_command_executor_execute, rewriting a one-element scalar
from the host between commands (src/m3_flow_solver_math.c:36-135,
src/m3_command_executor.c:55-92). On the HIP backend such lists return once
queued; the host's scalar writes and the final read are ordered after them
on the backend's stream. These tests replay the classifier-free guidance
and Euler steps that way, with the conditional and unconditional halves as
offset views of one velocity storage, and compare the latent with the same
float32 operations in numpy bit for bit.
"""
import ctypes
import sys

import numpy as np
import pytest

from conftest import m3

pytestmark = pytest.mark.gpu


class FlowMath:
    """The flow math's buffers on one backend: velocity [2, L, C] (the
    conditional half, then the unconditional one), latent, arithmetic
    [1, L, C] and a one-element scalar."""

    def __init__(self, backend, length, channels):
        self.lib, _ = m3.load()
        self.shape = (1, length, channels)
        self.bytes = 4 * length * channels
        self.storages = {}
        for name, size in (("velocity", 2 * self.bytes),
                           ("latent", self.bytes), ("arith", self.bytes),
                           ("scalar", 4)):
            storage = ctypes.c_void_p()
            assert self.lib.m3_storage_allocate(
                backend, size, 256, ctypes.byref(storage), None) == m3.OK
            self.storages[name] = storage
        self.views = {
            "cond": self._view("velocity", self.shape, 0),
            "uncond": self._view("velocity", self.shape, self.bytes),
            "latent": self._view("latent", self.shape, 0),
            "arith": self._view("arith", self.shape, 0),
            "scalar": self._view("scalar", (1,), 0),
        }
        self.executor = (ctypes.c_uint8 * 64)()
        self.lib.m3_command_executor_init(self.executor, backend)
        self.lib.m3_command_executor_execute.argtypes = [
            ctypes.c_void_p, ctypes.POINTER(m3.Command), ctypes.c_size_t,
            ctypes.POINTER(m3.Error)]

    def _view(self, storage, shape, offset):
        view = m3.TensorView()
        dims = (ctypes.c_uint64 * 8)(*shape)
        assert self.lib.m3_tensor_view_contiguous(
            ctypes.byref(view), self.storages[storage], m3.F32, len(shape),
            dims, offset, None) == m3.OK
        return view

    def write(self, name, array, offset=0):
        array = np.ascontiguousarray(array, np.float32)
        assert self.lib.m3_storage_write(
            self.storages[name], offset,
            array.ctypes.data_as(ctypes.c_void_p), array.nbytes,
            None) == m3.OK

    def read(self, name):
        out = np.zeros(self.shape, np.float32)
        assert self.lib.m3_storage_read(
            self.storages[name], 0, out.ctypes.data_as(ctypes.c_void_p),
            out.nbytes, None) == m3.OK
        return out

    def op(self, kind, left, right, output):
        command = m3.Command()
        command.kind = kind
        for i, name in enumerate((left, right, output)):
            command.descriptor.views[i] = ctypes.pointer(self.views[name])
        error = m3.Error()
        status = self.lib.m3_command_executor_execute(
            self.executor, ctypes.byref(command), 1, ctypes.byref(error))
        assert status == m3.OK, error.text()

    def guided_velocity(self, guidance):
        """src/m3_flow_solver_math.c:36-96: arithmetic = uncond +
        guidance * (cond + uncond * -1)."""
        self.write("scalar", [-1.0])
        self.op(m3.OP_MUL, "uncond", "scalar", "arith")
        self.op(m3.OP_ADD, "cond", "arith", "arith")
        self.write("scalar", [guidance])
        self.op(m3.OP_MUL, "arith", "scalar", "arith")
        self.op(m3.OP_ADD, "uncond", "arith", "arith")

    def euler_step(self, delta):
        """src/m3_flow_solver_math.c:98-135: latent += velocity * delta."""
        self.write("scalar", [delta])
        self.op(m3.OP_MUL, "arith", "scalar", "arith")
        self.op(m3.OP_ADD, "latent", "arith", "latent")

    def free(self):
        self.lib.m3_command_executor_dispose(self.executor)
        for storage in self.storages.values():
            self.lib.m3_storage_free(storage)


def expected_step(latent, velocity, guidance, delta):
    f = np.float32
    cond, uncond = velocity[0:1], velocity[1:2]
    a = (uncond * f(-1.0)).astype(f)
    a = (cond + a).astype(f)
    a = (a * f(guidance)).astype(f)
    a = (uncond + a).astype(f)
    a = (a * f(delta)).astype(f)
    return (latent + a).astype(f)


@pytest.mark.parametrize("length,channels", [(64, 96), (4096, 1536)])
def test_flow_steps_through_the_executor(gpu, length, channels):
    print("gpu case executor flow", length, channels, flush=True,
          file=sys.stderr)
    lib, _ = m3.load()
    backend = ctypes.c_void_p()
    error = m3.Error()
    assert lib.m3_backend_create_hip(ctypes.byref(backend),
                                     ctypes.byref(error)) == m3.OK
    rng = np.random.default_rng(length)
    flow = FlowMath(backend, length, channels)
    try:
        latent = rng.standard_normal((1, length, channels)).astype(np.float32)
        flow.write("latent", latent)
        steps, guidance = 6, 3.0
        for step in range(steps):
            velocity = rng.standard_normal(
                (2, length, channels)).astype(np.float32)
            flow.write("velocity", velocity)
            delta = 1.0 / steps
            flow.guided_velocity(guidance)
            flow.euler_step(delta)
            latent = expected_step(latent, velocity, guidance, delta)
        assert lib.m3_backend_finish(backend, ctypes.byref(error)) == m3.OK
        got = flow.read("latent")
        assert np.array_equal(got.view(np.uint32), latent.view(np.uint32))
    finally:
        flow.free()
        lib.m3_backend_free(backend)
