"""Pins the CPU oracle (oracle/uq_oracle.c) against the reference's own C
runtime compiled from its sources (oracle/_ref), in both the release macro set
(runtime/vision_flags.sh:2: dot4 GEMMs, prepared affine requantisation,
constant-channel elimination, fixed depthwise kernels) and the plain build.

Pins: conv_image (code 14), window_image (codes 15 and 16), add_image,
mean_image, mul_image (25), bmm_image (27), softmax_image (28),
softmax_table_image (17),
transpose_image (10) and the byte ops 5/19/20/21/22/23/26 of uqo_run, plus
the whole of both shipped models (MobileNetV4-small, YOLO26n-320 with its
attention block) where the reference tree is present. The reference's
known-answer patterns are re-scored here by the reference C build, since
their LiteRT expected values cannot run offline:
  * test_residual_add.py:64-96  every int8 pair x 4 scale cases x 3 clamps
  * test_modern_ops.py:166-173  requantisation ties with identity weights
  * test_modern_ops.py:59-64    softmax widths 1..256 x five input scales
  * test_modern_ops.py:75-79    transposes of ranks 2, 3 and 4
  * test_modern_ops.py:87-94    bmm shapes x all four transpose flags
Residual blocks (conv -> add, the pair the GPU library fuses) are fuzzed
against the reference build too.
"""
import struct
from pathlib import Path

import numpy as np
import pytest

import uq_plan as P
import uq_workloads as W
from plan_fuzz import (ATTENTION_OPS, CONSTANT_OPS, conv_add_bytes_plan, conv_add_plan, conv_mean_plan, dw_band_plan,
                       gather_plan, conv_lut_plan,
                       dw_mfma_plan, gemm_plan, gemm_rows_plan, ib_plan, random_plan, pointwise_wide_plan,
                       rows_conv_plan, stem_conv_plan, stem_plan, uib_plan)
from refs import oracle_run, ref_plain, ref_release

MODELS = Path("/root/reference/models")


def _check_plan(plan, images, seed):
    x = P.random_input(plan, images, seed)
    ob = P.output_bytes(plan)
    rel, pla = ref_release(), ref_plain()
    assert rel.load(plan) == 0
    y_rel = rel.run_images(x, images)
    assert pla.load(plan) == 0
    y_pla = pla.run_images(x, images)
    y_orc = oracle_run(plan, x, images, ob)
    np.testing.assert_array_equal(y_rel, y_pla)
    np.testing.assert_array_equal(y_orc, y_rel)
    return y_orc


@pytest.mark.parametrize("name,images", [("pointwise", 2), ("dw3s1", 2), ("dw3s2", 2), ("dw5s1", 2),
                                         ("dw5s2", 2), ("head", 3), ("conv3x3", 1), ("mnv4", 1),
                                         ("yolo", 1)])
def test_workloads_match_reference(name, images):
    plan, _ = W.WORKLOADS[name]()
    y = _check_plan(plan, images, seed=11)
    assert len(np.unique(y)) > 4, "workload output degenerate; parity would be weak"


def test_pointwise_hostile_tail_weights():
    plan, _ = W.pointwise(seed=3, tail_weights=True)
    _check_plan(plan, 1, seed=5)


@pytest.mark.parametrize("seed", range(120))
def test_random_plans_match_reference(seed):
    _check_plan(random_plan(1000 + seed), 2, seed)


ADD_CASES = [(.0625, -27, .03125, 13, .125, -5), (.0039215689, -128, .031, 127, .0078, 0),
             (.017, 0, .019, -1, .011, 25), (.5, 127, .0001, -128, .00001, -128)]


@pytest.mark.parametrize("case", range(4))
@pytest.mark.parametrize("act", ["none", "relu", "relu6"])
def test_add_all_byte_pairs(case, act):
    xs, xz, bs, bz, ys, yz = ADD_CASES[case]
    p = P.Plan(7)
    x = p.input((1, 256, 256, 1), zp=xz)
    b = p.tensor((1, 256, 256, 1), P.TYPE_I8, np.tile(np.arange(-128, 128, dtype=np.int8), 256))
    p.zp[b] = bz
    try:
        z = p.add(x, b, act=act, yz=yz, scales=(xs, bs, ys))
    except ValueError:
        pytest.skip("ADD output scale outside the bounded kernel (rejected at compile time)")
    plan = p.build(z)
    xin = np.repeat(np.arange(-128, 128, dtype=np.int8), 256)
    rel = ref_release()
    assert rel.load(plan) == 0
    np.testing.assert_array_equal(oracle_run(plan, xin, 1, P.output_bytes(plan)), rel.run_images(xin, 1))


@pytest.mark.parametrize("exponent", [1, 2, 3, 7, 15])
@pytest.mark.parametrize("fraction", [.5, .75, .999])
@pytest.mark.parametrize("zero", [-17, 0, 77])
def test_requant_ties_identity_conv(exponent, fraction, zero):
    """1x1 conv, identity weights, bias -4..3, output scale fraction/2^exponent."""
    p = P.Plan(9)
    x = p.input((1, 1, 256, 8), zp=0)
    w = np.eye(8, dtype=np.int8)
    kp = 8
    packed = P.pack_conv_weights(w, kp)
    corrected = np.arange(-4, 4, dtype=np.int64) - 128 * w.astype(np.int64).sum(axis=1)
    m, s = P.frexp_multiplier(fraction / 2 ** exponent)
    q = [1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 1, 256, 0, zero, -128, 127, 8, 8, kp, 0]
    qt = p.tensor((44,), P.TYPE_I32, np.concatenate((q, corrected, [m] * 8, [s] * 8)))
    wt = p.tensor((len(packed),), P.TYPE_I8, packed)
    z = p.tensor((1, 1, 256, 8))
    p._op(14, x, wt, z, (qt, 0, 0, 0))
    plan = p.build(z)
    xin = np.resize(np.arange(-128, 128, dtype=np.int8), 256 * 8)
    rel = ref_release()
    assert rel.load(plan) == 0
    np.testing.assert_array_equal(oracle_run(plan, xin, 1, 2048), rel.run_images(xin, 1))


@pytest.mark.parametrize("seed", range(40))
def test_attention_plans_match_reference(seed):
    _check_plan(random_plan(7000 + seed, ops=ATTENTION_OPS), 2, seed)


@pytest.mark.parametrize("seed", range(30))
def test_constant_operand_plans_match_reference(seed):
    _check_plan(random_plan(8000 + seed, ops=CONSTANT_OPS), 3, seed)


@pytest.mark.parametrize("maker", [dw_mfma_plan, stem_plan, rows_conv_plan, pointwise_wide_plan, gemm_plan,
                                   gemm_rows_plan, dw_band_plan, ib_plan, stem_conv_plan, uib_plan, conv_mean_plan,
                                   gather_plan, conv_lut_plan])
@pytest.mark.parametrize("seed", range(12))
def test_kernel_shape_fuzz_matches_reference(maker, seed):
    """Shapes aimed at the GPU's specialised kernels (matrix-core depthwise,
    stem, row-staged conv), scored by the reference build."""
    _check_plan(maker(seed), 2, seed)


@pytest.mark.parametrize("seed", range(20))
def test_conv_add_plans_match_reference(seed):
    _check_plan(conv_add_plan(seed), 2, seed)
    _check_plan(conv_add_bytes_plan(seed), 2, seed)


def softmax_plan(width, beta_scale, rows=3, zp=-17):
    p = P.Plan(width)
    x = p.input((rows, width), zp=zp)
    return p.build(p.softmax(x, beta_scale=beta_scale))


@pytest.mark.parametrize("width", [1, 2, 3, 17, 100, 256, 511, 512, 2048])
@pytest.mark.parametrize("beta_scale", [0.001, 0.03, 0.17, 1.0, 16.0])
def test_softmax_widths_and_scales(width, beta_scale):
    plan = softmax_plan(width, beta_scale)
    _check_plan(plan, 2, width)
    # Rows of one repeated value (ties everywhere; the widest rows reach the
    # exponent >= 32 branch).
    xin = np.repeat(np.array([-128, 0, 127], np.int8), width)
    rel = ref_release()
    assert rel.load(plan) == 0
    np.testing.assert_array_equal(oracle_run(plan, xin, 1, P.output_bytes(plan)), rel.run_images(xin, 1))


def softmax_table_plan(width, beta_scale, rows=3, zp=-17):
    p = P.Plan(width + 1)
    x = p.input((rows, width), zp=zp)
    return p.build(p.softmax_table(x, beta_scale=beta_scale))


@pytest.mark.parametrize("width", [1, 2, 17, 100, 256, 2048])
@pytest.mark.parametrize("beta_scale", [0.001, 0.17, 16.0])
def test_softmax_table_widths_and_scales(width, beta_scale):
    plan = softmax_table_plan(width, beta_scale)
    _check_plan(plan, 2, width)
    xin = np.repeat(np.array([-128, 0, 127], np.int8), width)
    rel = ref_release()
    assert rel.load(plan) == 0
    np.testing.assert_array_equal(oracle_run(plan, xin, 1, P.output_bytes(plan)), rel.run_images(xin, 1))


TRANSPOSES = [((2, 3), (1, 0)), ((2, 3, 5), (0, 2, 1)), ((2, 3, 5, 7), (0, 3, 1, 2)), ((2, 3, 5, 7), (0, 2, 3, 1)),
              ((1, 2, 32, 100), (0, 1, 3, 2)), ((3, 1, 4, 2), (3, 2, 0, 1))]


def transpose_plan(shape, perm):
    p = P.Plan(len(shape))
    x = p.input(shape, zp=-19)
    return p.build(p.transpose(x, perm))


@pytest.mark.parametrize("shape,perm", TRANSPOSES)
def test_transpose_ranks(shape, perm):
    _check_plan(transpose_plan(shape, perm), 2, 3)


BMM_SHAPES = [(2, 7, 11, 9), (2, 33, 32, 35), (2, 64, 100, 100)]


def bmm_plan(batches, m, k, n, ta, tb, seed=98):
    p = P.Plan(seed)
    x = p.input((batches, k, m) if ta else (batches, m, k), zp=2)
    rng = P.Rng(seed, 5)
    bsh = (batches, n, k) if tb else (batches, k, n)
    b = p.tensor(bsh, values=rng.int8(int(np.prod(bsh))))
    p.zp[b] = -17
    return p.build(p.bmm(x, b, trans_a=ta, trans_b=tb, yz=-19))


@pytest.mark.parametrize("shape", BMM_SHAPES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_bmm_shapes_and_transposes(shape, ta, tb):
    _check_plan(bmm_plan(*shape, bool(ta), bool(tb)), 2, 4)


def real_plan(name):
    path = MODELS / name
    if not path.exists():
        pytest.skip("reference models not present")
    data = path.read_bytes()
    nm = struct.unpack_from("<I", data, 12)[0]
    return data[52 + nm:]


@pytest.mark.parametrize("name", ["mobilenetv4-small.uqmodel", "yolo26n-320.uqmodel"])
def test_shipped_models_match_reference(name):
    y = _check_plan(real_plan(name), 2, 17)
    assert len(np.unique(y)) > 16
