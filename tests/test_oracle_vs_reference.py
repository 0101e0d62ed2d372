"""Pins the CPU oracle (oracle/uq_oracle.c) against the reference's own C
runtime compiled from its sources (oracle/_ref), in both the release macro set
(runtime/vision_flags.sh:2: dot4 GEMMs, prepared affine requantisation,
constant-channel elimination, fixed depthwise kernels) and the plain build.

Pins: conv_image (code 14), window_image (codes 15 and 16), add_image,
mean_image, and the byte ops 5/19/20/21/22/23/26 of uqo_run. The reference's
known-answer patterns are re-scored here by the reference C build, since
their LiteRT expected values cannot run offline:
  * test_residual_add.py:64-96  every int8 pair x 4 scale cases x 3 clamps
  * test_modern_ops.py:166-173  requantisation ties with identity weights
"""
import numpy as np
import pytest

import uq_plan as P
import uq_workloads as W
from plan_fuzz import random_plan
from refs import oracle_run, ref_plain, ref_release


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
