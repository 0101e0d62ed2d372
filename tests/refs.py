"""Test-side bindings of the CPU oracle (oracle/liboracle.so) and of the
reference's own portable C runtime built from its sources (oracle/_ref).

Only tests, the smoke check and the benchmark's CPU baseline import this."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
ORACLE = ROOT / "oracle" / "liboracle.so"
REF_RELEASE = ROOT / "oracle" / "_ref" / "libuq_ref_release.so"
REF_PLAIN = ROOT / "oracle" / "_ref" / "libuq_ref_plain.so"
NONE = 0xFFFFFFFF


def oracle():
    if not ORACLE.exists():
        pytest.skip("oracle not built (make -C oracle oracle)")
    lib = C.CDLL(str(ORACLE))
    lib.uqo_run.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p]
    lib.uqo_run.restype = C.c_int
    lib.uqo_scale.argtypes = [C.c_int32, C.c_int32, C.c_int32]
    lib.uqo_scale.restype = C.c_int32
    return lib


def oracle_run(plan, x, images, out_bytes, snap=None, snap_bytes=0):
    lib = oracle()
    x = np.ascontiguousarray(x, dtype=np.int8).reshape(-1)
    y = np.empty(images * out_bytes, np.int8)
    s = np.empty(max(snap_bytes, 1), np.int8)
    rc = lib.uqo_run(plan, len(plan), x.ctypes.data, images, y.ctypes.data,
                     NONE if snap is None else snap, s.ctypes.data)
    assert rc == 0, f"oracle rc {rc}"
    return (y, s[:snap_bytes]) if snap is not None else y


class RefLib:
    """The reference runtime (one global model per library copy)."""

    def __init__(self, path):
        if not Path(path).exists():
            pytest.skip(f"{path} not built (make -C oracle ref, needs the reference tree)")
        self.lib = C.CDLL(str(path))
        self.lib.ug_load.argtypes = [C.c_void_p, C.c_uint32]
        self.lib.ug_run.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32]
        self.lib.ug_input_bytes.restype = C.c_uint32
        self.lib.ug_output_bytes.restype = C.c_uint32
        self.lib.ug_snapshot.argtypes = [C.c_uint32, C.c_void_p, C.c_uint32]

    def load(self, plan):
        self._buf = C.create_string_buffer(bytes(plan), len(plan))
        return self.lib.ug_load(self._buf, len(plan))

    def run_images(self, x, images):
        ib, ob = self.lib.ug_input_bytes(), self.lib.ug_output_bytes()
        x = np.ascontiguousarray(x, dtype=np.int8).reshape(-1)
        y = np.empty(images * ob, np.int8)
        for j in range(images):
            rc = self.lib.ug_run(x[j * ib:].ctypes.data, ib, y[j * ob:].ctypes.data, ob)
            assert rc == 0, f"reference ug_run rc {rc}"
        return y


def ref_release():
    return RefLib(REF_RELEASE)


def ref_plain():
    return RefLib(REF_PLAIN)


def have_ref():
    return REF_RELEASE.exists() and REF_PLAIN.exists()
