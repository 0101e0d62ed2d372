"""ctypes binding of libuq_hip.so, the C-ABI GPU library (include/uq_graph.h).

Mirrors how the reference's own tests bind its native library
(tests/test_residual_add.py:62-69: ug_load / ug_run through ctypes), plus the
batch extension. Raises if the built library is missing: there is no CPU
fallback anywhere in the product path.
"""
import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
DEFAULT_LIBRARY = HERE / "libuq_hip.so"

# Every function declared in include/uq_graph.h: (name, restype, argtypes).
SIGNATURES = [
    ("ug_load", C.c_int, [C.c_void_p, C.c_uint32]),
    ("ug_run", C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32]),
    ("ug_input_bytes", C.c_uint32, []),
    ("ug_output_bytes", C.c_uint32, []),
    ("ug_snapshot", C.c_int, [C.c_uint32, C.c_void_p, C.c_uint32]),
    ("ug_profile", C.c_int, [C.c_uint32, C.c_void_p, C.c_uint32]),
    ("ug_stream_begin", C.c_int, []),
    ("ug_stream_end", C.c_int, []),
    ("ug_run_batch", C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64, C.c_uint32]),
    ("ug_run_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32]),
    ("ug_enqueue_device", C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32]),
    ("ug_enqueue_device_noalloc", C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32]),
    ("ug_synchronize", C.c_int, []),
    ("ug_snapshot_images", C.c_int, [C.c_uint32, C.c_void_p, C.c_uint64]),
    ("ug_device_alloc", C.c_void_p, [C.c_uint64]),
    ("ug_device_free", C.c_int, [C.c_void_p]),
    ("ug_device_upload", C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64]),
    ("ug_device_download", C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64]),
    ("ug_op_count", C.c_uint32, []),
    ("ug_bundle_plan", C.c_int, [C.c_void_p, C.c_uint64, C.POINTER(C.c_void_p), C.POINTER(C.c_uint32)]),
    ("ug_load_bundle", C.c_int, [C.c_void_p, C.c_uint64]),
    ("uq_sha256", None, [C.c_void_p, C.c_uint64, C.c_void_p]),
    ("ug_run_batch_pipelined", C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint32]),
    ("ug_host_alloc", C.c_void_p, [C.c_uint64]),
    ("ug_host_free", C.c_int, [C.c_void_p]),
    ("ug_open_mode", C.c_void_p, [C.c_void_p, C.c_uint32, C.c_int, C.POINTER(C.c_int)]),
    ("ug_open", C.c_void_p, [C.c_void_p, C.c_uint32, C.POINTER(C.c_int)]),
    ("ug_infer", C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32]),
    ("ug_close", None, [C.c_void_p]),
    ("ug_snapshot_tensor", C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32]),
    ("ug_profile_control", C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32]),
]


class NativeError(RuntimeError):
    def __init__(self, where, code):
        super().__init__(f"{where} returned {code}")
        self.code = code


def open_library(path=None):
    path = Path(path or os.environ.get("UQ_HIP_LIBRARY", DEFAULT_LIBRARY))
    if not path.exists():
        raise FileNotFoundError(f"{path} is not built; run __graft_entry__.build()")
    lib = C.CDLL(str(path))
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    # Test hooks outside the plan ABI: launches of the large-tile GEMM, of the
    # fused bottleneck, stem, banded bottleneck, conv + mean and row gather
    # kernels.
    for hook in ("uqk_gemm_launches", "uqk_ib_launches", "uqk_stem_conv_launches", "uqk_uib_launches",
                 "uqk_conv_mean_launches", "uqk_gather_launches"):
        getattr(lib, hook).restype = C.c_uint64
        getattr(lib, hook).argtypes = []
    # Measurement hook: the sustained int8 matrix-core rate of a register-only
    # MFMA loop (iters, warm-up launches, timed launches -> TOP/s, us/launch).
    lib.uqk_mfma_ceiling.restype = C.c_int
    lib.uqk_mfma_ceiling.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double)]
    return lib


def mfma_ceiling(lib, iters, warmup=3, reps=10):
    """(TOP/s, us per launch) of the register-only int8 MFMA loop."""
    tops, us = C.c_double(), C.c_double()
    rc = lib.uqk_mfma_ceiling(iters, warmup, reps, C.byref(tops), C.byref(us))
    if rc:
        raise RuntimeError(f"uqk_mfma_ceiling failed: {rc}")
    return tops.value, us.value


class Graph:
    """One loaded plan in the (process-global) GPU library."""

    def __init__(self, plan, lib=None):
        self.lib = lib or open_library()
        self.plan = bytes(plan)
        self._buf = C.create_string_buffer(self.plan, len(self.plan))
        rc = self.lib.ug_load(self._buf, len(self.plan))
        if rc:
            raise NativeError("ug_load", rc)
        self.input_bytes = self.lib.ug_input_bytes()
        self.output_bytes = self.lib.ug_output_bytes()

    def run(self, x):
        x = np.ascontiguousarray(x, dtype=np.int8).reshape(-1)
        y = np.empty(self.output_bytes, np.int8)
        rc = self.lib.ug_run(x.ctypes.data, x.nbytes, y.ctypes.data, y.nbytes)
        if rc:
            raise NativeError("ug_run", rc)
        return y

    def run_batch(self, x, images):
        x = np.ascontiguousarray(x, dtype=np.int8).reshape(-1)
        y = np.empty(images * self.output_bytes, np.int8)
        rc = self.lib.ug_run_batch(x.ctypes.data, x.nbytes, y.ctypes.data, y.nbytes, images)
        if rc:
            raise NativeError("ug_run_batch", rc)
        return y

    def snapshot_images(self, tensor, nbytes):
        y = np.empty(nbytes, np.int8)
        rc = self.lib.ug_snapshot_images(tensor, y.ctypes.data, nbytes)
        if rc:
            raise NativeError("ug_snapshot_images", rc)
        return y

    def profile(self, command):
        counters = np.zeros(514, np.uint64)
        rc = self.lib.ug_profile(command, counters.ctypes.data, counters.nbytes)
        if rc:
            raise NativeError("ug_profile", rc)
        return counters


class Session:
    """The reference's HardwareSession contract (src/unoq_dsp/transport.py:
    19-79) over the bridge ABI of this library: one model per process, calls
    serialised, close idempotent, "mailbox" or "rpc" pipeline."""

    def __init__(self, plan, pipeline="mailbox", lib=None):
        if pipeline not in ("mailbox", "rpc"):
            raise ValueError("pipeline must be mailbox or rpc")
        self.lib = lib or open_library()
        error = C.c_int()
        buf = C.create_string_buffer(bytes(plan), len(plan))
        self.handle = self.lib.ug_open_mode(buf, len(plan), int(pipeline == "mailbox"), C.byref(error))
        if not self.handle:
            raise NativeError("ug_open_mode", error.value & 0xffffffff)
        self.input_bytes = self.lib.ug_input_bytes()
        self.output_bytes = self.lib.ug_output_bytes()

    def run(self, x):
        if not self.handle:
            raise RuntimeError("Session closed")
        x = np.ascontiguousarray(x, dtype=np.int8).reshape(-1)
        y = np.empty(self.output_bytes, np.int8)
        rc = self.lib.ug_infer(self.handle, x.ctypes.data, x.nbytes, y.ctypes.data, y.nbytes)
        if rc:
            raise NativeError("ug_infer", rc)
        return y

    def close(self):
        if self.handle:
            self.lib.ug_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *args):
        self.close()


class DeviceBuffer:
    """A device allocation made through the library's helpers."""

    def __init__(self, lib, nbytes):
        self.lib = lib
        self.nbytes = int(nbytes)
        self.ptr = lib.ug_device_alloc(self.nbytes)
        if not self.ptr:
            raise MemoryError(f"ug_device_alloc({nbytes}) failed")

    def upload(self, array):
        a = np.ascontiguousarray(array).reshape(-1).view(np.uint8)
        assert a.nbytes <= self.nbytes
        rc = self.lib.ug_device_upload(self.ptr, a.ctypes.data, a.nbytes)
        if rc:
            raise NativeError("ug_device_upload", rc)

    def download(self, nbytes=None):
        out = np.empty(self.nbytes if nbytes is None else nbytes, np.int8)
        rc = self.lib.ug_device_download(out.ctypes.data, self.ptr, out.nbytes)
        if rc:
            raise NativeError("ug_device_download", rc)
        return out

    def free(self):
        if self.ptr:
            self.lib.ug_device_free(self.ptr)
            self.ptr = None
