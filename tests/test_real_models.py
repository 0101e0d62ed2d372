"""End to end on the reference's shipped MobileNetV4-small bundle
(tests/golden/mobilenetv4-small.uqmodel, real weights and quantisation:
positive shifts, zero-multiplier channels, 60 ops). Expected outputs for four
images come from the reference's own C runtime
(tests/golden/make_real_model_fixtures.py).

CPU: the bundle reader accepts the file and the oracle reproduces the
fixture. GPU: ug_load_bundle + the batch entry points reproduce it byte for
byte, and a 256-image batch agrees image by image with the oracle."""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import uq_plan as P
from refs import oracle_run

GOLDEN = Path(__file__).resolve().parent / "golden"
BUNDLE = GOLDEN / "mobilenetv4-small.uqmodel"


def _fixture():
    data = BUNDLE.read_bytes()
    nm = int.from_bytes(data[12:16], "little")
    with np.load(GOLDEN / "mobilenetv4_small_expected.npz", allow_pickle=False) as z:
        return data, data[52 + nm:], z["input"], z["output"]


def test_bundle_reader_accepts_shipped_model():
    from uq_native import open_library
    lib = open_library()
    data, plan, _, _ = _fixture()
    buf = C.create_string_buffer(data, len(data))
    ptr, n = C.c_void_p(), C.c_uint32()
    assert lib.ug_bundle_plan(buf, len(data), C.byref(ptr), C.byref(n)) == 0
    assert C.string_at(ptr.value, n.value) == plan


def test_oracle_reproduces_shipped_model():
    _, plan, x, want = _fixture()
    images = x.size // P.input_bytes(plan)
    np.testing.assert_array_equal(oracle_run(plan, x, images, P.output_bytes(plan)), want)


@pytest.mark.gpu
def test_gpu_runs_shipped_bundle():
    from uq_native import DeviceBuffer, open_library
    lib = open_library()
    data, plan, x, want = _fixture()
    buf = C.create_string_buffer(data, len(data))
    assert lib.ug_load_bundle(buf, len(data)) == 0
    ib, ob = lib.ug_input_bytes(), lib.ug_output_bytes()
    images = x.size // ib
    y = np.empty(images * ob, np.int8)
    assert lib.ug_run_batch(x.ctypes.data, x.nbytes, y.ctypes.data, y.nbytes, images) == 0
    np.testing.assert_array_equal(y, want)
    y1 = np.empty(ob, np.int8)
    assert lib.ug_run(x.ctypes.data, ib, y1.ctypes.data, ob) == 0
    np.testing.assert_array_equal(y1, want[:ob])
    # Full batch on device buffers; sampled images against the oracle.
    big = 256
    xb = P.random_input(plan, big, 77)
    din, dout = DeviceBuffer(lib, xb.nbytes), DeviceBuffer(lib, big * ob)
    din.upload(xb)
    assert lib.ug_run_device(din.ptr, dout.ptr, big) == 0
    yb = dout.download()
    din.free()
    dout.free()
    for j in (0, 100, 255):
        np.testing.assert_array_equal(yb[j * ob:(j + 1) * ob], oracle_run(plan, xb[j * ib:(j + 1) * ib], 1, ob),
                                      err_msg=f"image {j}")
