"""The reference's host session ABI (runtime/bridge.c:70-185), as its Python
HardwareSession binds it (src/unoq_dsp/transport.py:35-43), and the pipelined
host-buffer batch.

CPU: argument checks and codes that need no GPU (1 for bad arguments, the
loader's code for a bad plan, 24 for a valid plan without a GPU, 1003 for a
null session). GPU: both pipeline modes produce the oracle's bytes image after
image; one session at a time (1001); snapshots refused in mailbox mode (1003);
profile control; the pipelined batch equals the oracle for chunk sizes that
divide the batch and for ragged last chunks, from pageable and pinned host
memory."""
import ctypes as C

import numpy as np
import pytest

import uq_plan as P
import uq_workloads as W
from refs import oracle_run
from uq_native import NativeError, Session, open_library


@pytest.fixture(scope="module")
def lib():
    return open_library()


def _open(lib, plan, pipeline):
    err = C.c_int(-7)
    buf = C.create_string_buffer(bytes(plan), max(len(plan), 1))
    h = lib.ug_open_mode(buf, len(plan), pipeline, C.byref(err))
    return h, err.value


def test_open_argument_checks(lib):
    plan, _ = W.pointwise()
    err = C.c_int(-7)
    assert not lib.ug_open_mode(None, 100, 0, C.byref(err)) and err.value == 1
    buf = C.create_string_buffer(plan, len(plan))
    assert not lib.ug_open_mode(buf, len(plan), 2, C.byref(err)) and err.value == 1
    assert not lib.ug_open_mode(buf, len(plan), -1, C.byref(err)) and err.value == 1
    assert not lib.ug_open_mode(buf, 17 * 1024 * 1024 + 1, 0, C.byref(err)) and err.value == 1
    bad = bytearray(plan)
    bad[0] ^= 1
    h, code = _open(lib, bad, 0)
    assert not h and code == 11


def test_null_session_codes(lib):
    x = np.zeros(16, np.int8)
    assert lib.ug_infer(None, x.ctypes.data, 16, x.ctypes.data, 16) == 1003
    assert lib.ug_snapshot_tensor(None, 0, x.ctypes.data, 16) == 1003
    counters = np.zeros(514, np.uint64)
    assert lib.ug_profile_control(None, 2, counters.ctypes.data, counters.nbytes) == 1003
    lib.ug_close(None)


def test_open_without_gpu_reports_worker_unavailable(lib):
    if lib.uqk_device_count() if hasattr(lib, "uqk_device_count") else False:
        pytest.skip("GPU present")
    plan, _ = W.pointwise()
    h, code = _open(lib, plan, 1)
    if h:
        lib.ug_close(h)
        pytest.skip("GPU present")
    assert code == 24


@pytest.mark.gpu
@pytest.mark.parametrize("pipeline", ["rpc", "mailbox"])
@pytest.mark.parametrize("name", ["pointwise", "mnv4", "yolo"])
def test_session_matches_oracle(lib, pipeline, name):
    plan, _ = W.WORKLOADS[name]()
    x = P.random_input(plan, 3, 41)
    want = oracle_run(plan, x, 3, P.output_bytes(plan))
    ib, ob = P.input_bytes(plan), P.output_bytes(plan)
    with Session(plan, pipeline, lib) as s:
        for j in range(3):
            got = s.run(x[j * ib:(j + 1) * ib])
            np.testing.assert_array_equal(got, want[j * ob:(j + 1) * ob], err_msg=f"{name} {pipeline} image {j}")


@pytest.mark.gpu
def test_one_session_at_a_time_and_mode_rules(lib):
    plan, _ = W.pointwise()
    with Session(plan, "mailbox", lib) as s:
        h, code = _open(lib, plan, 0)
        assert not h and code == 1001
        out = np.zeros(P.output_bytes(plan), np.int8)
        assert lib.ug_snapshot_tensor(s.handle, 0, out.ctypes.data, out.nbytes) == 1003
        counters = np.zeros(514, np.uint64)
        assert lib.ug_profile_control(s.handle, 1, counters.ctypes.data, counters.nbytes) == 0
        x = P.random_input(plan, 1, 3)
        s.run(x)      # profiled calls take the direct path
        s.run(x)
        assert lib.ug_profile_control(s.handle, 2, counters.ctypes.data, counters.nbytes) == 0
        assert counters[0] == 2 and counters[2] > 0
        assert lib.ug_profile_control(s.handle, 3, counters.ctypes.data, counters.nbytes) == 1003
        assert lib.ug_profile_control(s.handle, 0, counters.ctypes.data, 100) == 1003
        assert lib.ug_infer(s.handle, x.ctypes.data, x.nbytes - 1, out.ctypes.data, out.nbytes) == 1003
    # Closed: a new session opens; rpc mode allows snapshots.
    with Session(plan, "rpc", lib) as s:
        x = P.random_input(plan, 1, 5)
        s.run(x)
        recs = P.tensor_records(plan)
        t = P.op_records(plan)[0][3]
        snap = np.zeros(recs[t][1], np.int8)
        assert lib.ug_snapshot_tensor(s.handle, t, snap.ctypes.data, snap.nbytes) == 0
        _, want = oracle_run(plan, x, 1, P.output_bytes(plan), snap=t, snap_bytes=recs[t][1])
        np.testing.assert_array_equal(snap, want)


@pytest.mark.gpu
def test_mailbox_graph_follows_reload(lib):
    """A session's captured graph is rebuilt when device buffers move (a
    larger batch through the batch entry point in between)."""
    plan, _ = W.pointwise()
    ib, ob = P.input_bytes(plan), P.output_bytes(plan)
    with Session(plan, "mailbox", lib) as s:
        x = P.random_input(plan, 6, 9)
        want = oracle_run(plan, x, 6, ob)
        np.testing.assert_array_equal(s.run(x[:ib]), want[:ob])
        y = np.empty(6 * ob, np.int8)
        assert lib.ug_run_batch(x.ctypes.data, x.nbytes, y.ctypes.data, y.nbytes, 6) == 0
        np.testing.assert_array_equal(y, want)
        np.testing.assert_array_equal(s.run(x[ib:2 * ib]), want[ob:2 * ob])


@pytest.mark.gpu
@pytest.mark.parametrize("name,images,chunk", [("pointwise", 7, 3), ("pointwise", 8, 2), ("mnv4", 256, 64),
                                               ("mnv4", 100, 0), ("yolo", 64, 16), ("dw3s2", 64, 24),
                                               ("mnv4", 512, 256)])
@pytest.mark.parametrize("pinned", [False, True])
def test_pipelined_batch(lib, name, images, chunk, pinned):
    plan, _ = W.WORKLOADS[name]()
    x = P.random_input(plan, images, 61)
    ib, ob = P.input_bytes(plan), P.output_bytes(plan)
    g_ok = lib.ug_load(C.create_string_buffer(plan, len(plan)), len(plan))
    assert g_ok == 0
    if pinned:
        hin, hout = lib.ug_host_alloc(x.nbytes), lib.ug_host_alloc(images * ob)
        assert hin and hout
        C.memmove(hin, x.ctypes.data, x.nbytes)
        rc = lib.ug_run_batch_pipelined(hin, x.nbytes, hout, images * ob, images, chunk)
        y = np.frombuffer(C.string_at(hout, images * ob), np.int8).copy()
        lib.ug_host_free(hin)
        lib.ug_host_free(hout)
    else:
        y = np.empty(images * ob, np.int8)
        rc = lib.ug_run_batch_pipelined(x.ctypes.data, x.nbytes, y.ctypes.data, y.nbytes, images, chunk)
    assert rc == 0
    samples = range(images) if images <= 8 else (0, chunk - 1 if chunk else 1, images // 2, images - 1)
    if chunk >= 128:
        # Chunks this large run as two image slices on two streams: images
        # of the second slice of each chunk too.
        samples = sorted(set(samples) | {chunk // 2 + 1, chunk + chunk // 2 + 3})
    for j in samples:
        np.testing.assert_array_equal(y[j * ob:(j + 1) * ob], oracle_run(plan, x[j * ib:(j + 1) * ib], 1, ob),
                                      err_msg=f"{name} image {j}")
