"""GPU parity: libuq_hip.so through its C ABI against the CPU oracle, byte for
byte, on the same seeded inputs.

Small image counts are compared in full; full-batch runs (256 / 512 images)
are checked through size-independent properties: every sampled image of the
batch equals that image run alone through the oracle, and a batch result is
identical between the host and the device entry points."""
import struct

import numpy as np
import pytest

import uq_plan as P
import uq_workloads as W
from plan_fuzz import (ATTENTION_OPS, CONSTANT_OPS, conv_add_bytes_plan, conv_add_plan, conv_mean_plan, dw_band_plan,
                       gather_plan, pack_plan, conv_lut_plan,
                       dw_mfma_plan, gemm_plan, gemm_rows_plan, ib_plan, random_plan, pointwise_wide_plan,
                       rows_conv_plan, stem_conv_plan, stem_plan, uib_block)
from test_oracle_vs_reference import (BMM_SHAPES, TRANSPOSES, bmm_plan, softmax_plan, softmax_table_plan,
                                      transpose_plan)
from refs import oracle_run
from uq_native import DeviceBuffer, Graph, NativeError, open_library

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return open_library()


def _oracle(plan, x, images):
    return oracle_run(plan, x, images, P.output_bytes(plan))


def _assert_same(got, want, what):
    if not np.array_equal(got, want):
        bad = np.flatnonzero(got != want)
        raise AssertionError(f"{what}: {bad.size} of {want.size} bytes differ; first at {bad[0]}: "
                             f"got {got[bad[0]]} want {want[bad[0]]}")


@pytest.mark.parametrize("name,images", [("pointwise", 1), ("pointwise", 3), ("dw3s1", 64), ("dw3s2", 64),
                                         ("dw5s1", 64), ("dw5s2", 64), ("head", 16), ("conv3x3", 2), ("mnv4", 3),
                                         ("yolo", 2)])
def test_workload_bit_exact(lib, name, images):
    plan, _ = W.WORKLOADS[name]()
    x = P.random_input(plan, images, 21)
    g = Graph(plan, lib)
    _assert_same(g.run_batch(x, images), _oracle(plan, x, images), name)


def test_single_image_entry_point(lib):
    plan, _ = W.pointwise(tail_weights=True)
    x = P.random_input(plan, 1, 4)
    _assert_same(Graph(plan, lib).run(x), _oracle(plan, x, 1), "ug_run")


def _run_device(lib, g, x, images):
    din = DeviceBuffer(lib, x.nbytes)
    dout = DeviceBuffer(lib, images * g.output_bytes)
    din.upload(x)
    assert lib.ug_run_device(din.ptr, dout.ptr, images) == 0
    y = dout.download()
    din.free()
    dout.free()
    return y


# Sampled images: the first and last image of the batch, of each image slice
# (MobileNetV4-S runs as two slices of 128 images) and the images holding the
# first and last boundary of the GEMM's 256-pixel tiles (head: 49 pixels per
# image, so tile boundaries fall inside images 5 and 506; conv3x3: 6400
# pixels per image, whole tiles).
@pytest.mark.parametrize("name,images,samples", [("mnv4", 256, (0, 127, 128, 255)), ("yolo", 64, (0, 63)),
                                                 ("head", 512, (0, 5, 255, 256, 506, 511)),
                                                 ("conv3x3", 512, (0, 1, 256, 511))])
def test_full_batch_sampled_images(lib, name, images, samples):
    plan, _ = W.WORKLOADS[name]()
    x = P.random_input(plan, images, 33)
    g = Graph(plan, lib)
    y = _run_device(lib, g, x, images)
    ib, ob = g.input_bytes, g.output_bytes
    for j in samples:
        _assert_same(y[j * ob:(j + 1) * ob], _oracle(plan, x[j * ib:(j + 1) * ib], 1), f"{name} image {j}")
    if name == "mnv4":
        # Host and device entry points agree on the whole batch, and so do
        # two image slices and one stream.
        _assert_same(g.run_batch(x, images), y, "run_batch vs run_device")


@pytest.mark.parametrize("name", ["head", "conv3x3"])
def test_gemm_whole_batch_matches_conv_kernels(lib, name, monkeypatch):
    """The large-tile GEMM (which the 512-image launches take) and the
    16x16x64 conv kernels (UQ_GEMM=0) are independent implementations;
    they agree on every byte of the batch."""
    plan, images = W.WORKLOADS[name]()
    x = P.random_input(plan, images, 34)
    before = lib.uqk_gemm_launches()
    y = _run_device(lib, Graph(plan, lib), x, images)
    assert lib.uqk_gemm_launches() > before, "the large-tile GEMM did not run"
    monkeypatch.setenv("UQ_GEMM", "0")
    before = lib.uqk_gemm_launches()
    y0 = _run_device(lib, Graph(plan, lib), x, images)
    assert lib.uqk_gemm_launches() == before
    _assert_same(y, y0, f"{name}: GEMM vs conv kernels")


@pytest.mark.parametrize("seed", range(40))
def test_gemm_rows_plans(lib, seed, monkeypatch):
    """Convs on the row-staged GEMM (persistent blocks over 512-pixel tiles
    of staged input rows), several images per batch, compared in full with
    the oracle."""
    monkeypatch.setenv("UQ_GEMM", "1")
    monkeypatch.setenv("UQ_GEMM_TILE", "4")
    plan = gemm_rows_plan(9500 + seed)
    images = 1 + seed % 4
    x = P.random_input(plan, images, seed)
    g = Graph(plan, lib)
    before = lib.uqk_gemm_launches()
    y = g.run_batch(x, images)
    assert lib.uqk_gemm_launches() > before, "the GEMM did not run"
    _assert_same(y, _oracle(plan, x, images), f"gemm rows plan {9500 + seed}")


@pytest.mark.parametrize("seed", range(48))
def test_gemm_plans(lib, seed, monkeypatch):
    """Convs forced onto the large-tile GEMM (all four tile configurations,
    one or two output tiles per block) with pixel, channel and K tails,
    compared in full with the oracle."""
    monkeypatch.setenv("UQ_GEMM", "1")
    monkeypatch.setenv("UQ_GEMM_TILE", str(seed % 4))
    monkeypatch.setenv("UQ_GEMM_TPB", str(1 + (seed // 4) % 2))
    plan = gemm_plan(9000 + seed)
    images = 2 + seed % 3
    x = P.random_input(plan, images, seed)
    g = Graph(plan, lib)
    before = lib.uqk_gemm_launches()
    y = g.run_batch(x, images)
    assert lib.uqk_gemm_launches() > before, "the large-tile GEMM did not run"
    _assert_same(y, _oracle(plan, x, images), f"gemm plan {9000 + seed}")


@pytest.mark.parametrize("seed", range(80))
def test_random_plans(lib, seed):
    plan = random_plan(1000 + seed)
    images = 3
    x = P.random_input(plan, images, seed)
    _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"random plan {1000 + seed}")


@pytest.mark.parametrize("seed", range(40))
def test_attention_plans(lib, seed):
    plan = random_plan(7000 + seed, ops=ATTENTION_OPS)
    images = 3
    x = P.random_input(plan, images, seed)
    _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"attention plan {7000 + seed}")


@pytest.mark.parametrize("seed", range(30))
def test_constant_operand_plans(lib, seed):
    """Constants in per-image operand slots, several images per batch."""
    plan = random_plan(8000 + seed, ops=CONSTANT_OPS)
    images = 5
    x = P.random_input(plan, images, seed)
    _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"constant-operand plan {8000 + seed}")


@pytest.mark.parametrize("width", [1, 3, 17, 100, 256, 512, 2048])
@pytest.mark.parametrize("beta_scale", [0.001, 0.17, 16.0])
def test_softmax(lib, width, beta_scale):
    plan = softmax_plan(width, beta_scale)
    images = 7
    x = P.random_input(plan, images, width)
    x[:3 * width] = np.repeat(np.array([-128, 0, 127], np.int8), width)   # all-tie rows
    _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"softmax w={width}")


@pytest.mark.parametrize("width", [1, 17, 100, 2048])
@pytest.mark.parametrize("beta_scale", [0.001, 16.0])
def test_softmax_table(lib, width, beta_scale):
    plan = softmax_table_plan(width, beta_scale)
    images = 5
    x = P.random_input(plan, images, width)
    x[:3 * width] = np.repeat(np.array([-128, 0, 127], np.int8), width)
    _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"softmax17 w={width}")


@pytest.mark.parametrize("shape,perm", TRANSPOSES)
def test_transpose(lib, shape, perm):
    plan = transpose_plan(shape, perm)
    x = P.random_input(plan, 4, 2)
    _assert_same(Graph(plan, lib).run_batch(x, 4), _oracle(plan, x, 4), f"transpose {shape} {perm}")


@pytest.mark.parametrize("shape", BMM_SHAPES + [(3, 100, 32, 100), (1, 5, 8192, 3), (2, 3, 40, 2048)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_bmm(lib, shape, ta, tb):
    plan = bmm_plan(*shape, bool(ta), bool(tb))
    images = 3
    x = P.random_input(plan, images, 6)
    _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"bmm {shape} {ta}{tb}")


def test_snapshot_intermediate(lib):
    plan, _ = W.mnv4()
    images = 2
    x = P.random_input(plan, images, 8)
    g = Graph(plan, lib)
    g.run_batch(x, images)
    recs = P.tensor_records(plan)
    activations = [t for t, r in enumerate(recs) if not r[8]]
    consts = [t for t, r in enumerate(recs) if r[8]]
    for t in (activations[1], activations[len(activations) // 2], activations[-2]):
        nbytes = images * recs[t][1]
        _, want = oracle_run(plan, x, images, P.output_bytes(plan), snap=t, snap_bytes=nbytes)
        _assert_same(g.snapshot_images(t, nbytes), want, f"snapshot tensor {t}")
    t = consts[3]
    _, want = oracle_run(plan, x, images, P.output_bytes(plan), snap=t, snap_bytes=recs[t][1])
    _assert_same(g.snapshot_images(t, recs[t][1]), want, f"snapshot constant {t}")


def test_profile_counters(lib):
    plan, _ = W.pointwise()
    g = Graph(plan, lib)
    g.profile(1)
    x = P.random_input(plan, 1, 1)
    for _ in range(3):
        g.run(x)
    c = g.profile(2)
    assert c[0] == 3 and c[1] > 0 and c[2] > 0


@pytest.mark.parametrize("name", ["mnv4", "yolo"])
def test_profiled_run_keeps_bytes(lib, name):
    """A profiled run (every op alone on the stream, its kernels stamping the
    op's events) gives the unprofiled bytes, and every op that launches work
    gets ticks no larger than the run's total."""
    plan, _ = W.WORKLOADS[name]()
    images = 3
    x = P.random_input(plan, images, 8)
    g = Graph(plan, lib)
    want = g.run_batch(x, images)
    g.profile(1)
    _assert_same(g.run_batch(x, images), want, f"{name} profiled")
    c = g.profile(2)
    g.profile(0)
    kinds = [o[0] for o in P.op_records(plan)]
    ticks = c[2:2 + len(kinds)]
    assert c[0] == 1 and c[1] == ticks.sum()
    assert all(ticks[i] > 0 for i, k in enumerate(kinds) if k != 5)


def test_bad_sizes_rejected(lib):
    plan, _ = W.pointwise()
    g = Graph(plan, lib)
    x = np.zeros(g.input_bytes + 1, np.int8)
    y = np.zeros(g.output_bytes, np.int8)
    assert lib.ug_run(x.ctypes.data, x.nbytes, y.ctypes.data, y.nbytes) == 22
    with pytest.raises(NativeError):
        g.run_batch(np.zeros(3 * g.input_bytes, np.int8), 2)


@pytest.mark.parametrize("name,images", [("mnv4", 3), ("mnv4", 256)])
def test_fused_bottleneck_opt_in(lib, monkeypatch, name, images):
    """1x1 -> depthwise -> 1x1 (-> add) groups run as one launch (the default;
    UQ_FUSE_BOTTLENECK=1 asks for it explicitly); the bytes must not change,
    and snapshots of a group's inner tensors are rebuilt from the group
    input."""
    plan, _ = W.WORKLOADS[name]()
    x = P.random_input(plan, images, 41)
    monkeypatch.setenv("UQ_FUSE_BOTTLENECK", "1")
    g = Graph(plan, lib)
    y = g.run_batch(x, images)
    ib, ob = g.input_bytes, g.output_bytes
    for j in sorted({0, images // 2, images - 1}):
        _assert_same(y[j * ob:(j + 1) * ob], _oracle(plan, x[j * ib:(j + 1) * ib], 1), f"fused {name} image {j}")
    if images > 8:
        return
    recs = P.tensor_records(plan)
    activations = [t for t, r in enumerate(recs) if not r[8]]
    for t in activations[2:-1:5]:
        nbytes = images * recs[t][1]
        _, want = oracle_run(plan, x, images, P.output_bytes(plan), snap=t, snap_bytes=nbytes)
        _assert_same(g.snapshot_images(t, nbytes), want, f"fused snapshot tensor {t}")


@pytest.mark.parametrize("seed", range(40))
def test_fused_bottleneck_plans(lib, monkeypatch, seed):
    """Random inverted bottlenecks run fused: the fused kernel runs, and one
    to three images match the oracle byte for byte, as they do with fusion
    off (UQ_FUSE_BOTTLENECK=0)."""
    monkeypatch.setenv("UQ_FUSE_BOTTLENECK", "1")
    plan = ib_plan(seed)
    images = 1 + seed % 3
    x = P.random_input(plan, images, seed)
    g = Graph(plan, lib)
    before = lib.uqk_ib_launches()
    y = g.run_batch(x, images)
    assert lib.uqk_ib_launches() > before, "the fused bottleneck kernel did not run"
    want = _oracle(plan, x, images)
    _assert_same(y, want, f"fused bottleneck plan {seed}")
    monkeypatch.setenv("UQ_FUSE_BOTTLENECK", "0")
    before = lib.uqk_ib_launches()
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"unfused bottleneck plan {seed}")
    assert lib.uqk_ib_launches() == before


@pytest.mark.parametrize("seed", range(40))
def test_banded_bottleneck_plans(lib, monkeypatch, seed):
    """Random universal inverted bottlenecks (a start depthwise and/or a
    stride-1 or stride-2 depthwise between the two 1x1 convs, an optional
    add) run as one banded launch: the kernel runs, one to three images
    match the oracle byte for byte, as they do unfused (UQ_FUSE_UIB=0), and a
    snapshot of the block's first inner tensor is rebuilt from the block
    input. UQ_FUSE_UIB=2 fuses blocks of several bands too; by default only
    single-band blocks run fused (or, when the whole block needs several
    bands, possibly its part after the start depthwise), with the same
    bytes."""
    plan, rows, out_rows = uib_block(seed)
    monkeypatch.setenv("UQ_FUSE_UIB", "2")
    images = 1 + seed % 3
    x = P.random_input(plan, images, seed)
    want = _oracle(plan, x, images)
    g = Graph(plan, lib)
    before = lib.uqk_uib_launches()
    _assert_same(g.run_batch(x, images), want, f"banded bottleneck plan {seed}")
    assert lib.uqk_uib_launches() > before, "the banded bottleneck kernel did not run"
    inner = P.op_records(plan)[1][3]            # op 0 is the post table in front of the block
    nbytes = images * P.tensor_records(plan)[inner][1]
    _, snap = oracle_run(plan, x, images, P.output_bytes(plan), snap=inner, snap_bytes=nbytes)
    _assert_same(g.snapshot_images(inner, nbytes), snap, f"banded bottleneck plan {seed}: inner snapshot")
    monkeypatch.delenv("UQ_FUSE_UIB")
    before = lib.uqk_uib_launches()
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"default banded bottleneck plan {seed}")
    if rows == out_rows:
        assert lib.uqk_uib_launches() > before, "a single-band block did not run fused by default"
    monkeypatch.setenv("UQ_FUSE_UIB", "0")
    before = lib.uqk_uib_launches()
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"unfused banded bottleneck plan {seed}")
    assert lib.uqk_uib_launches() == before


@pytest.mark.parametrize("mode,launches", [("1", 2), ("2", 3)])
def test_mnv4_banded_groups(lib, monkeypatch, mode, launches):
    """MobileNetV4's 14x14 and 7x7 ExtraDW blocks run on the banded kernel in
    one band by default (the 7x7 one with its records read from L2); with
    UQ_FUSE_UIB=2 its 28x28 block with a stride-2 depthwise (five bands) does
    too; the bytes match the oracle either way (batch 3, one image slice)."""
    monkeypatch.setenv("UQ_FUSE_UIB", mode)
    plan, _ = W.mnv4()
    x = P.random_input(plan, 3, 77)
    before = lib.uqk_uib_launches()
    _assert_same(Graph(plan, lib).run_batch(x, 3), _oracle(plan, x, 3), "mnv4 with banded groups")
    assert lib.uqk_uib_launches() - before == launches


@pytest.mark.parametrize("seed", range(40))
def test_stem_conv_fusion(lib, monkeypatch, seed):
    """A stem conv and the 3x3 stride-2 conv over its output (and a 1x1
    32 -> 32 conv right after, when there is one) run as one launch by
    default: one to three images match the oracle byte for byte, as they do
    with the 1x1 apart (UQ_FUSE_STEM=2) and unfused (UQ_FUSE_STEM=0). After a
    host-buffer run snapshots of the inner tensors are rebuilt; after a
    device-buffer run (the stem read the caller's buffer) they are refused
    with 22."""
    plan = stem_conv_plan(seed)
    images = 1 + seed % 3
    x = P.random_input(plan, images, seed)
    want = _oracle(plan, x, images)
    g = Graph(plan, lib)
    before = lib.uqk_stem_conv_launches()
    _assert_same(g.run_batch(x, images), want, f"fused stem plan {seed}")
    assert lib.uqk_stem_conv_launches() > before, "the fused stem kernel did not run"
    ops = P.op_records(plan)
    stem_out = ops[0][3]
    nbytes = images * P.tensor_records(plan)[stem_out][1]
    _, snap = oracle_run(plan, x, images, P.output_bytes(plan), snap=stem_out, snap_bytes=nbytes)
    _assert_same(g.snapshot_images(stem_out, nbytes), snap, f"fused stem plan {seed}: stem output snapshot")
    if len(ops) > 2 and ops[2][0] == 14 and ops[2][1] == ops[1][3]:
        # The 1x1 ran in the same launch: the 3x3's output is rebuilt too.
        g.run_batch(x, images)
        mid = ops[1][3]
        mbytes = images * P.tensor_records(plan)[mid][1]
        _, msnap = oracle_run(plan, x, images, P.output_bytes(plan), snap=mid, snap_bytes=mbytes)
        _assert_same(g.snapshot_images(mid, mbytes), msnap, f"fused stem plan {seed}: 3x3 output snapshot")
    din, dout = DeviceBuffer(lib, x.nbytes), DeviceBuffer(lib, images * g.output_bytes)
    din.upload(x)
    assert lib.ug_run_device(din.ptr, dout.ptr, images) == 0
    _assert_same(dout.download(), want, f"fused stem plan {seed}, device buffers")
    buf = np.empty(nbytes, np.int8)
    assert lib.ug_snapshot_images(stem_out, buf.ctypes.data, buf.nbytes) == 22
    if len(ops) > 2 and ops[2][0] == 14 and ops[2][1] == ops[1][3]:
        # The 3x3's output is inside the fused launch as well.
        mbuf = np.empty(images * P.tensor_records(plan)[ops[1][3]][1], np.int8)
        assert lib.ug_snapshot_images(ops[1][3], mbuf.ctypes.data, mbuf.nbytes) == 22
    din.free()
    dout.free()
    monkeypatch.setenv("UQ_FUSE_STEM", "2")
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"stem plan {seed}, 1x1 not fused")
    monkeypatch.setenv("UQ_FUSE_STEM", "0")
    before = lib.uqk_stem_conv_launches()
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"unfused stem plan {seed}")
    assert lib.uqk_stem_conv_launches() == before


@pytest.mark.parametrize("seed", range(40))
def test_gather_fusion(lib, monkeypatch, seed):
    """A concat whose operands are table lookups of slices (YOLO's split /
    SiLU / concat chains and variants) runs as one row gather: 1, 2, 3 or
    130 images (two image slices) match the oracle byte for byte, as they do
    with the fusion off (UQ_FUSE_GATHER=0); after a host run the skipped
    ops' outputs (slices, lookups, inner concat) are rebuilt for snapshots."""
    plan = gather_plan(seed)
    images = [1, 2, 3, 130][seed % 4]
    x = P.random_input(plan, images, seed)
    want = _oracle(plan, x, images)
    g = Graph(plan, lib)
    before = lib.uqk_gather_launches()
    _assert_same(g.run_batch(x, images), want, f"gather plan {seed}, {images} images")
    assert lib.uqk_gather_launches() > before
    if images < 128:
        ops, tensors = P.op_records(plan), P.tensor_records(plan)
        output = ops[-1][3]
        for code, a, b, t, *_ in ops:
            if code in (20, 22, 26) and t != output:
                nbytes = images * tensors[t][1]
                _, snap = oracle_run(plan, x, images, P.output_bytes(plan), snap=t, snap_bytes=nbytes)
                _assert_same(g.snapshot_images(t, nbytes), snap, f"gather plan {seed}: snapshot of tensor {t}")
    monkeypatch.setenv("UQ_FUSE_GATHER", "0")
    before = lib.uqk_gather_launches()
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"gather plan {seed} unfused")
    assert lib.uqk_gather_launches() == before


@pytest.mark.parametrize("seed", range(30))
def test_conv_lut_fusion(lib, monkeypatch, seed):
    """A conv whose output only feeds a table lookup runs as one conv launch
    with the tables composed: 1-3 images against the oracle, a snapshot of
    the conv's output rebuilt after a host run, and the same plans unfused
    (UQ_FUSE_LUT=0)."""
    plan = conv_lut_plan(seed)
    images = 1 + seed % 3
    x = P.random_input(plan, images, seed)
    want = _oracle(plan, x, images)
    g = Graph(plan, lib)
    _assert_same(g.run_batch(x, images), want, f"conv+lut plan {seed}")
    conv_out = P.op_records(plan)[0][3]
    nbytes = images * P.tensor_records(plan)[conv_out][1]
    _, snap = oracle_run(plan, x, images, P.output_bytes(plan), snap=conv_out, snap_bytes=nbytes)
    _assert_same(g.snapshot_images(conv_out, nbytes), snap, f"conv+lut plan {seed}: conv output snapshot")
    monkeypatch.setenv("UQ_FUSE_LUT", "0")
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"conv+lut plan {seed} unfused")


@pytest.mark.parametrize("seed", range(20))
def test_pack_outputs(lib, monkeypatch, seed):
    """A pack of two to nine outputs (one row gather up to eight, a copy per
    tensor past that or with UQ_FUSE_GATHER=0), 1-3 images, byte for byte
    against the oracle."""
    plan = pack_plan(seed)
    images = 1 + seed % 3
    x = P.random_input(plan, images, seed)
    want = _oracle(plan, x, images)
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"pack plan {seed}")
    monkeypatch.setenv("UQ_FUSE_GATHER", "0")
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"pack plan {seed}, a copy per tensor")


@pytest.mark.parametrize("seed", range(40))
def test_conv_mean_fusion(lib, monkeypatch, seed):
    """A 1x1 conv and the global mean over its output run as one launch
    (head.hip) unless the conv's output has a second reader: one to three
    images match the oracle byte for byte, as they do unfused
    (UQ_FUSE_MEAN=0); after a host-buffer run a snapshot of the conv's output
    is rebuilt. The fused kernel's channel tiles are split over one to four
    workgroups per image (UQ_MEAN_PARTS; more parts than tiles are capped)."""
    plan = conv_mean_plan(seed)
    images = 1 + seed % 3
    x = P.random_input(plan, images, seed)
    want = _oracle(plan, x, images)
    ops = P.op_records(plan)
    conv_out = ops[0][3]
    fused = sum(1 for o in ops if conv_out in (o[1], o[2])) == 1
    monkeypatch.setenv("UQ_MEAN_PARTS", str(1 + (seed // 3) % 4))
    g = Graph(plan, lib)
    before = lib.uqk_conv_mean_launches()
    _assert_same(g.run_batch(x, images), want, f"conv+mean plan {seed}")
    assert (lib.uqk_conv_mean_launches() > before) == fused
    nbytes = images * P.tensor_records(plan)[conv_out][1]
    _, snap = oracle_run(plan, x, images, P.output_bytes(plan), snap=conv_out, snap_bytes=nbytes)
    _assert_same(g.snapshot_images(conv_out, nbytes), snap, f"conv+mean plan {seed}: conv output snapshot")
    monkeypatch.setenv("UQ_FUSE_MEAN", "0")
    before = lib.uqk_conv_mean_launches()
    _assert_same(Graph(plan, lib).run_batch(x, images), want, f"unfused conv+mean plan {seed}")
    assert lib.uqk_conv_mean_launches() == before


@pytest.mark.parametrize("seed", range(40))
def test_conv_add_fusion(lib, seed):
    """A 1x1 conv followed by a residual add runs as one launch (the add in
    the conv's epilogue): both operand orders, byte-tail channel counts."""
    for plan, images in ((conv_add_plan(seed), 3), (conv_add_bytes_plan(seed), 2)):
        x = P.random_input(plan, images, seed)
        _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"conv+add plan {seed}")


def _fused_conv_outputs(plan):
    """Conv outputs read only by the add right after them (not written by a fused run)."""
    ops = P.op_records(plan)
    uses = {}
    for o in ops:
        for t in (o[1], o[2]):
            uses[t] = uses.get(t, 0) + 1
    return [c[3] for c, ad in zip(ops, ops[1:]) if c[0] == 14 and ad[0] == 18 and c[3] in (ad[1], ad[2])
            and uses[c[3]] == 1]


@pytest.mark.parametrize("name", ["mnv4", "fuzz"])
def test_snapshot_of_fused_conv_output(lib, name):
    """Snapshots of a fused conv's own output (never written by the fused
    launch) are rebuilt from the group's inputs, and the run's output is
    unchanged by the rebuild."""
    plan = W.mnv4()[0] if name == "mnv4" else conv_add_plan(5)
    images = 2
    x = P.random_input(plan, images, 9)
    g = Graph(plan, lib)
    y = g.run_batch(x, images)
    recs = P.tensor_records(plan)
    targets = _fused_conv_outputs(plan)
    assert targets
    for t in targets[:4] + targets[-1:]:
        nbytes = images * recs[t][1]
        _, want = oracle_run(plan, x, images, P.output_bytes(plan), snap=t, snap_bytes=nbytes)
        _assert_same(g.snapshot_images(t, nbytes), want, f"{name} snapshot tensor {t}")
    _assert_same(g.run_batch(x, images), y, f"{name} rerun after snapshots")


@pytest.mark.parametrize("name,images", [("mnv4", 131), ("yolo", 130)])
def test_split_batch_matches_single_stream(lib, monkeypatch, name, images):
    """A batch run as two image slices on two streams (uneven slices here)
    gives the single-stream bytes through both entry points, the images on
    either side of the slice boundary match the oracle, and a snapshot of a
    fused conv's output after the split run covers the whole batch."""
    plan, _ = W.WORKLOADS[name]()
    x = P.random_input(plan, images, 17)
    recs = P.tensor_records(plan)
    targets = _fused_conv_outputs(plan)[:2]
    outs, snaps = {}, {}
    for streams in ("1", "2"):
        monkeypatch.setenv("UQ_STREAMS", streams)
        g = Graph(plan, lib)
        outs[streams] = g.run_batch(x, images)
        snaps[streams] = [g.snapshot_images(t, images * recs[t][1]) for t in targets]
        din = DeviceBuffer(lib, x.nbytes)
        dout = DeviceBuffer(lib, images * g.output_bytes)
        din.upload(x)
        assert lib.ug_run_device(din.ptr, dout.ptr, images) == 0
        _assert_same(dout.download(), outs[streams], f"{name} device path, {streams} stream(s)")
        din.free()
        dout.free()
    _assert_same(outs["2"], outs["1"], f"{name} two slices vs one stream")
    for t, a, b in zip(targets, snaps["2"], snaps["1"]):
        _assert_same(a, b, f"{name} snapshot of tensor {t} after the split run")
    ib, ob = P.input_bytes(plan), P.output_bytes(plan)
    for i in (0, images // 2 - 1, images // 2, images - 1):
        _assert_same(outs["2"][i * ob:(i + 1) * ob], _oracle(plan, x[i * ib:(i + 1) * ib], 1), f"{name} image {i}")


@pytest.mark.parametrize("kind", ["random", "attention", "constant"])
@pytest.mark.parametrize("seed", range(12))
def test_split_batch_fuzz_plans(lib, monkeypatch, kind, seed):
    """Random, attention and constant-operand plans at 130 images: two image
    slices (65 + 65, on two streams) give the single-stream bytes, and the
    images on both sides of the slice boundary and at the batch ends match
    the oracle."""
    ops = {"random": None, "attention": ATTENTION_OPS, "constant": CONSTANT_OPS}[kind]
    plan = random_plan({"random": 1400, "attention": 7400, "constant": 8400}[kind] + seed, ops=ops)
    images = 130
    x = P.random_input(plan, images, seed)
    outs = {}
    for streams in ("1", "2"):
        monkeypatch.setenv("UQ_STREAMS", streams)
        outs[streams] = Graph(plan, lib).run_batch(x, images)
    _assert_same(outs["2"], outs["1"], f"{kind} plan {seed}: two slices vs one stream")
    ib, ob = P.input_bytes(plan), P.output_bytes(plan)
    for i in (0, 64, 65, 129):
        _assert_same(outs["2"][i * ob:(i + 1) * ob], _oracle(plan, x[i * ib:(i + 1) * ib], 1),
                     f"{kind} plan {seed} image {i}")


def test_split_batches_continue_across_calls(lib, monkeypatch):
    """Consecutive identical device batches keep their two slices on their
    own streams without joining; a batch on other buffers, a snapshot taken
    straight after an enqueue, and a host-buffer run in between all see
    finished results, equal to one stream's."""
    plan, _ = W.mnv4()
    images = 130
    x1, x2 = P.random_input(plan, images, 51), P.random_input(plan, images, 52)
    recs = P.tensor_records(plan)
    t = _fused_conv_outputs(plan)[0]
    monkeypatch.setenv("UQ_STREAMS", "1")
    g1 = Graph(plan, lib)
    y1, y2 = g1.run_batch(x1, images), g1.run_batch(x2, images)
    snap2 = g1.snapshot_images(t, images * recs[t][1])
    monkeypatch.setenv("UQ_STREAMS", "2")
    g = Graph(plan, lib)
    bufs = [(DeviceBuffer(lib, x1.nbytes), DeviceBuffer(lib, images * g.output_bytes)) for _ in range(2)]
    for (din, _), x in zip(bufs, (x1, x2)):
        din.upload(x)
    order = [0, 0, 0, 1, 0, 1, 1]
    for k in order:
        assert lib.ug_enqueue_device(bufs[k][0].ptr, bufs[k][1].ptr, images) == 0
    assert lib.ug_synchronize() == 0
    _assert_same(bufs[0][1].download(), y1, "batch 1 after interleaved enqueues")
    _assert_same(bufs[1][1].download(), y2, "batch 2 after interleaved enqueues")
    assert lib.ug_enqueue_device(bufs[1][0].ptr, bufs[1][1].ptr, images) == 0
    _assert_same(g.snapshot_images(t, images * recs[t][1]), snap2, f"snapshot of tensor {t} right after an enqueue")
    assert lib.ug_enqueue_device(bufs[0][0].ptr, bufs[0][1].ptr, images) == 0
    _assert_same(g.run_batch(x2, images), y2, "host-buffer run after an enqueue")
    assert lib.ug_synchronize() == 0
    _assert_same(bufs[0][1].download(), y1, "batch 1 after the host-buffer run")
    for din, dout in bufs:
        din.free()
        dout.free()


@pytest.mark.parametrize("images", [3, 130])
def test_device_path_output_reshape(lib, images):
    """MobileNetV4 ends in a reshape (op 5) of the classifier's output, which
    on the device path lands in the caller's buffer (the classifier writes
    it there, the reshape moves nothing): the output and a snapshot of the
    reshaped tensor match the oracle, on one stream and on two slices."""
    plan, _ = W.mnv4()
    ops, recs = P.op_records(plan), P.tensor_records(plan)
    out = struct.unpack_from("<I", plan, 24)[0]          # header: output tensor index
    last = [o for o in ops if o[0] == 5 and o[3] == out]
    assert last, "the plan's output is a reshape"
    src = last[0][1]
    x = P.random_input(plan, images, 23)
    g = Graph(plan, lib)
    din, dout = DeviceBuffer(lib, x.nbytes), DeviceBuffer(lib, images * g.output_bytes)
    din.upload(x)
    assert lib.ug_run_device(din.ptr, dout.ptr, images) == 0
    ib, ob = g.input_bytes, g.output_bytes
    y = dout.download()
    for j in (0, images // 2, images - 1):
        _assert_same(y[j * ob:(j + 1) * ob], _oracle(plan, x[j * ib:(j + 1) * ib], 1), f"image {j}")
    _, want = oracle_run(plan, x, images, P.output_bytes(plan), snap=src, snap_bytes=images * recs[src][1])
    _assert_same(g.snapshot_images(src, images * recs[src][1]), want, f"snapshot of tensor {src}")
    din.free()
    dout.free()


def test_gather_conv_with_fused_add(lib):
    """A 3x3 conv too wide for row staging (80x80x128, K = 1152: the gather
    kernel) followed by a residual add of its input: the add runs in the
    gather kernel's epilogue; the same kernel without an add (the conv3x3
    workload) must not touch the add's table."""
    p = P.Plan(31)
    x = p.input((1, 80, 80, 128), zp=5)
    y = p.conv(x, 128, k=3, act="relu", shift=(-12, -4))
    plan = p.build(p.add(y, x, act="none"))
    images = 2
    xin = P.random_input(plan, images, 12)
    _assert_same(Graph(plan, lib).run_batch(xin, images), _oracle(plan, xin, images), "gather conv + add")


@pytest.mark.parametrize("maker", [dw_mfma_plan, stem_plan, rows_conv_plan, pointwise_wide_plan])
@pytest.mark.parametrize("seed", range(40))
def test_kernel_shape_fuzz(lib, maker, seed):
    """Matrix-core depthwise (bands, channel groups, small maps), the stem
    (several row segments, IC 1-4) and the row-staged conv with its
    register-direct epilogue, byte for byte against the oracle."""
    plan = maker(seed)
    images = 2
    x = P.random_input(plan, images, seed)
    _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"{maker.__name__} {seed}")


@pytest.mark.parametrize("kernel", ["band", "mfma", "win"])
@pytest.mark.parametrize("seed", range(24))
def test_depthwise_kernels(lib, kernel, seed, monkeypatch):
    """Each depthwise kernel forced at load (band, matrix-core window, dot4
    window), on wide-channel band-shaped plans and matrix-core-shaped ones,
    one to three images, byte for byte against the oracle."""
    monkeypatch.setenv("UQ_DW", kernel)
    plan = dw_band_plan(seed) if seed % 2 == 0 else dw_mfma_plan(100 + seed)
    images = 1 + seed % 3
    x = P.random_input(plan, images, seed)
    _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"depthwise {kernel} {seed}")


@pytest.mark.parametrize("rows,seed", [(1, 0), (2, 1), (3, 2), (5, 3), (7, 4), (1, 5), (4, 6), (6, 7)])
def test_depthwise_window_bands(lib, rows, seed, monkeypatch):
    """The matrix-core window depthwise with its blocks forced to at most
    `rows` output rows (UQ_DW_ROWS), one to three images, byte for byte
    against the oracle (unforced, these small launches split their maps into
    equal bands of the launch's own choice: test_depthwise_kernels)."""
    monkeypatch.setenv("UQ_DW", "mfma")
    monkeypatch.setenv("UQ_DW_ROWS", str(rows))
    plan = dw_mfma_plan(200 + seed)
    images = 1 + seed % 3
    x = P.random_input(plan, images, seed)
    _assert_same(Graph(plan, lib).run_batch(x, images), _oracle(plan, x, images), f"depthwise bands {rows} {seed}")


def test_profile_counts_one_run_per_profiled_batch(lib):
    """ug_profile counters count finished profiled batches: a synchronize
    with none pending adds nothing; one device run adds one; two enqueues
    and a synchronize add two, each with its own op times."""
    plan, _ = W.pointwise()
    g = Graph(plan, lib)
    images = 4
    x = P.random_input(plan, images, 5)
    din = DeviceBuffer(lib, x.nbytes)
    dout = DeviceBuffer(lib, images * g.output_bytes)
    din.upload(x)
    g.profile(1)
    assert lib.ug_synchronize() == 0
    assert g.profile(2)[0] == 0
    assert lib.ug_run_device(din.ptr, dout.ptr, images) == 0
    assert lib.ug_synchronize() == 0
    c = g.profile(2)
    assert c[0] == 1 and c[1] > 0 and c[2] > 0
    one = int(c[1])
    assert lib.ug_enqueue_device(din.ptr, dout.ptr, images) == 0
    assert lib.ug_enqueue_device(din.ptr, dout.ptr, images) == 0
    assert lib.ug_synchronize() == 0
    c = g.profile(2)
    assert c[0] == 3 and c[1] > one
    g.profile(0)
    din.free()
    dout.free()


def test_snapshot_after_freeing_a_bound_buffer(lib):
    """Once a caller buffer the last run read or wrote is freed, activation
    snapshots return 22 instead of reading freed memory."""
    plan = random_plan(1003)
    g = Graph(plan, lib)
    images = 3
    x = P.random_input(plan, images, 6)
    din = DeviceBuffer(lib, x.nbytes)
    dout = DeviceBuffer(lib, images * g.output_bytes)
    din.upload(x)
    assert lib.ug_run_device(din.ptr, dout.ptr, images) == 0
    recs = P.tensor_records(plan)
    inp = struct.unpack_from("<I", plan, 20)[0]
    buf = np.empty(images * recs[inp][1], np.int8)
    assert lib.ug_snapshot_images(inp, buf.ctypes.data, buf.nbytes) == 0
    din.free()
    assert lib.ug_snapshot_images(inp, buf.ctypes.data, buf.nbytes) == 22
    assert lib.ug_snapshot(inp, buf.ctypes.data, recs[inp][1]) == 22
    dout.free()
    # A new run binds fresh buffers and snapshots work again.
    assert np.array_equal(g.run_batch(x, images), _oracle(plan, x, images))
    assert lib.ug_snapshot_images(inp, buf.ctypes.data, buf.nbytes) == 0
