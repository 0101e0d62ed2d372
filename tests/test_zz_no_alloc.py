"""ug_enqueue_device_noalloc (include/uq_graph.h): every intermediate
activation in the library's static per-GPU scratch, no allocation. Its
results equal ug_enqueue_device's byte for byte on two calls in a row, the
second with fewer images; batches whose activations exceed the scratch are
refused with 22 before any GPU work."""
import numpy as np
import pytest

import uq_plan as P
import uq_workloads as W
from plan_fuzz import CONSTANT_OPS, random_plan
from uq_native import DeviceBuffer, Graph, open_library

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


@pytest.fixture(scope="module")
def lib():
    return open_library()


def _device_run(lib, fn, g, x, images):
    din = DeviceBuffer(lib, x.nbytes)
    dout = DeviceBuffer(lib, images * g.output_bytes)
    din.upload(x)
    assert fn(din.ptr, dout.ptr, images) == 0
    assert lib.ug_synchronize() == 0
    y = dout.download()
    din.free()
    dout.free()
    return y


def _activation_bytes(plan, images):
    """Scratch bytes of a batch: every tensor but the input, the output and
    constants, each images * bytes rounded up to 256 (the workloads used
    here read no constant per image, which would take a slot too)."""
    recs = P.tensor_records(plan)
    inp, out = (int.from_bytes(plan[o:o + 4], "little") for o in (20, 24))
    total = 0
    for i, r in enumerate(recs):
        if i in (inp, out) or r[8]:
            continue
        total += (images * r[1] + 255) & ~255
    return total


@pytest.mark.parametrize("name,counts", [("mnv4", (6, 2)), ("yolo", (2, 1))])
def test_noalloc_matches_enqueue_device(lib, name, counts):
    plan, _ = W.WORKLOADS[name]()
    g = Graph(plan, lib)
    for images in counts:
        assert _activation_bytes(plan, images) <= SCRATCH
        x = P.random_input(plan, images, 40 + images)
        want = _device_run(lib, lib.ug_enqueue_device, g, x, images)
        got = _device_run(lib, lib.ug_enqueue_device_noalloc, g, x, images)
        assert np.array_equal(got, want), f"{name} at {images} images"


@pytest.mark.parametrize("seed", range(6))
def test_noalloc_constant_operands_and_two_slices(lib, seed):
    """Constants in per-image slots (copied into the scratch), at 130 images
    (two image slices on two streams), then 3 images."""
    plan = random_plan(8000 + seed, ops=CONSTANT_OPS)
    g = Graph(plan, lib)
    for images in (130, 3):
        x = P.random_input(plan, images, seed)
        want = _device_run(lib, lib.ug_enqueue_device, g, x, images)
        got = _device_run(lib, lib.ug_enqueue_device_noalloc, g, x, images)
        assert np.array_equal(got, want), f"constant-operand plan {8000 + seed} at {images} images"


def test_noalloc_refuses_batches_beyond_the_scratch(lib):
    plan, _ = W.mnv4()
    g = Graph(plan, lib)
    images = 64
    assert _activation_bytes(plan, images) > SCRATCH
    din = DeviceBuffer(lib, images * g.input_bytes)
    dout = DeviceBuffer(lib, images * g.output_bytes)
    assert lib.ug_enqueue_device_noalloc(din.ptr, dout.ptr, images) == 22
    assert lib.ug_enqueue_device_noalloc(din.ptr, dout.ptr, 0) == 22
    # Still loaded and usable.
    x = P.random_input(plan, 1, 3)
    assert np.array_equal(_device_run(lib, lib.ug_enqueue_device_noalloc, g, x, 1),
                          _device_run(lib, lib.ug_enqueue_device, g, x, 1))
    din.free()
    dout.free()
