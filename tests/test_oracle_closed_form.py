"""Pins the CPU oracle without the reference build, by independent
formulations of the same mathematics:

* uqo_scale (qnn.c:61-83) against gemmlowp's definitions evaluated with exact
  rationals: SaturatingRoundingDoublingHighMul = round-half-up(v*m / 2^31),
  RoundingDivideByPOT = round-half-away-from-zero(h / 2^n).
* conv (code 14), depthwise (15), pooling (16) against brute-force numpy
  sliding windows over an explicitly padded input, with weights kept in OHWI
  and packed for the plan only through gemm.h's layout, so an index, stride,
  dilation, padding or K-order mistake in the oracle fails.
* mean (24) and add (18) against direct evaluation of their definitions.
* the one-multiply requantisation used by the GPU epilogue (epilogue_record
  in graph.c) against uqo_scale over random and tie-producing operands.
"""
from fractions import Fraction
import math
import random

import numpy as np
import pytest

import uq_plan as P
from refs import oracle, oracle_run


def srdhm(v, m):
    return math.floor(Fraction(v * m, 1 << 31) + Fraction(1, 2))


def rdbp(h, n):
    if n == 0:
        return h
    x = Fraction(h, 1 << n)
    return int(math.copysign(math.floor(abs(x) + Fraction(1, 2)), x)) if x else 0


def scale_exact(v, m, s):
    return rdbp(srdhm(v * (1 << max(s, 0)), m), max(-s, 0))


def test_scale_matches_gemmlowp_definition():
    lib = oracle()
    rng = random.Random(5)
    cases = []
    for _ in range(20000):
        s = rng.randint(-31, 15)
        lim = (1 << 31) >> max(s, 0)
        v = rng.choice([rng.randint(-lim, lim - 1), rng.randint(-300, 300), -lim, lim - 1, 0])
        m = rng.choice([0, 1, (1 << 31) - 1, 1 << 30, rng.randint(0, (1 << 31) - 1)])
        cases.append((v, m, s))
    # exact ties of both roundings: m = 2^30 halves v exactly, then h = k*2^(n-2)
    for n in range(1, 31):
        for k in (-3, -1, 1, 3):
            for v in (k << (n - 1), k << n):
                if -(1 << 31) <= v < (1 << 31):
                    cases.append((v, 1 << 30, -n))
    for v, m, s in cases:
        assert lib.uqo_scale(v, m, s) == scale_exact(v, m, s), (v, m, s)


def test_one_multiply_requant_algebra():
    """The GPU epilogue's single int64 multiply-add form equals scale()+clamp."""
    lib = oracle()
    rng = random.Random(9)
    for _ in range(40000):
        s = rng.randint(-31, 15)
        lim = (1 << 31) >> max(s, 0)
        v = rng.choice([rng.randint(-lim, lim - 1), rng.randint(-4000, 4000)])
        m = rng.choice([0, rng.randint(0, (1 << 31) - 1), rng.randint(1 << 30, (1 << 31) - 1)])
        yz, lo = rng.randint(-128, 127), rng.randint(-128, 127)
        hi = rng.randint(lo, 127)
        want = min(max(lib.uqo_scale(v, m, s) + yz, lo), hi)
        n = max(-s, 0)
        q = (v << max(s, 0)) * m + (1 << 30) + ((1 << (30 + n)) if n else 0)
        if lo < yz and n and q < (1 << (30 + n)):
            q -= 1 << 31
        got = min(max((q >> (31 + n)) + yz, lo), hi)
        assert got == want, (v, m, s, yz, lo, hi)


def _single_op_plan(shape, xz, build):
    p = P.Plan(1)
    x = p.input(shape, zp=xz)
    z = build(p, x)
    return p.build(z)


def _requant(acc, bias, m, s, yz, lo, hi):
    lib = oracle()
    out = np.empty(acc.shape, np.int64)
    for idx in np.ndindex(acc.shape):
        c = idx[-1]
        out[idx] = min(max(lib.uqo_scale(int(acc[idx] + bias[c]), int(m[c]), int(s[c])) + yz, lo), hi)
    return out.astype(np.int8)


@pytest.mark.parametrize("seed", range(12))
def test_conv_brute_force(seed):
    rng = np.random.default_rng(seed)
    n, h, w = 1, int(rng.integers(1, 7)), int(rng.integers(1, 7))
    ic, oc = int(rng.choice([1, 3, 5, 8])), int(rng.choice([1, 3, 4, 6]))
    kh, kw = int(rng.integers(1, 4)), int(rng.integers(1, 4))
    sh, sw, dh, dw = (int(v) for v in rng.integers(1, 3, 4))
    pt, pl, pb, pr = (int(v) for v in rng.integers(0, 3, 4))
    pb = max(pb, (kh - 1) * dh + 1 - h - pt)
    pr = max(pr, (kw - 1) * dw + 1 - w - pl)
    oh = (h + pt + pb - (kh - 1) * dh - 1) // sh + 1
    ow = (w + pl + pr - (kw - 1) * dw - 1) // sw + 1
    xz, yz = int(rng.integers(-128, 128)), int(rng.integers(-128, 128))
    K = kh * kw * ic
    kp = (K + 7) & ~7
    wo = rng.integers(-127, 128, (oc, kh, kw, ic)).astype(np.int8)
    full = np.zeros((oc, kp), np.int8)
    full[:, :K] = wo.reshape(oc, K)
    full[:, K:] = rng.integers(-127, 128, (oc, kp - K))          # hostile K tail
    bias = rng.integers(-5000, 5000, oc)
    m = rng.integers(1 << 30, 1 << 31, oc)
    s = rng.integers(-14, -5, oc)

    def build(p, x):
        q = [kh, kw, sh, sw, dh, dw, pt, pl, pb, pr, oh, ow, xz, yz, -128, 127, ic, oc, kp, 0]
        qt = p.tensor((20 + 3 * oc,), P.TYPE_I32, np.concatenate((q, bias, m, s)))
        packed = P.pack_conv_weights(full, kp)
        wt = p.tensor((len(packed),), P.TYPE_I8, packed)
        z = p.tensor((n, oh, ow, oc))
        p._op(14, x, wt, z, (qt, 0, 0, 0))
        return z

    plan = _single_op_plan((n, h, w, ic), xz, build)
    x = rng.integers(-128, 128, (n, h, w, ic)).astype(np.int8)
    xp = np.full((n, h + pt + pb + 8, w + pl + pr + 8, ic), xz, np.int64)
    xp[:, pt:pt + h, pl:pl + w, :] = x
    acc = np.zeros((n, oh, ow, oc), np.int64)
    for ky in range(kh):
        for kx in range(kw):
            win = xp[:, ky * dh: ky * dh + (oh - 1) * sh + 1: sh, kx * dw: kx * dw + (ow - 1) * sw + 1: sw, :] + 128
            acc += np.einsum("nhwc,oc->nhwo", win, wo[:, ky, kx, :].astype(np.int64))
    acc += (xz + 128) * full[:, K:].astype(np.int64).sum(axis=1)
    want = _requant(acc, bias, m, s, yz, -128, 127)
    got = oracle_run(plan, x, 1, want.size).reshape(want.shape)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("seed", range(10))
def test_depthwise_and_pool_brute_force(seed):
    rng = np.random.default_rng(100 + seed)
    h, w, c = int(rng.integers(1, 8)), int(rng.integers(1, 8)), int(rng.choice([1, 3, 4, 7]))
    k = int(rng.choice([1, 2, 3, 5]))
    st, dl = int(rng.integers(1, 3)), int(rng.integers(1, 3))
    pt, pl = int(rng.integers(0, k)), int(rng.integers(0, k))
    pb = max(int(rng.integers(0, 3)), (k - 1) * dl + 1 - h - pt)
    pr = max(int(rng.integers(0, 3)), (k - 1) * dl + 1 - w - pl)
    oh = (h + pt + pb - (k - 1) * dl - 1) // st + 1
    ow = (w + pl + pr - (k - 1) * dl - 1) // st + 1
    xz, yz = int(rng.integers(-128, 128)), int(rng.integers(-128, 128))
    x = rng.integers(-128, 128, (1, h, w, c)).astype(np.int8)
    wt = rng.integers(-127, 128, (k, k, c)).astype(np.int8)
    bias = rng.integers(-3000, 3000, c)
    m = rng.integers(1 << 30, 1 << 31, c)
    s = rng.integers(-12, -4, c)

    def build_dw(p, xi):
        q = [k, k, st, st, dl, dl, pt, pl, pb, pr, oh, ow, xz, yz, -128, 127, c, c, (k * k + 7) & ~7, 0]
        qt = p.tensor((20 + 3 * c,), P.TYPE_I32, np.concatenate((q, bias, m, s)))
        wtt = p.tensor((k * k * c,), P.TYPE_I8, wt.reshape(-1))
        z = p.tensor((1, oh, ow, c))
        p._op(15, xi, wtt, z, (qt, 0, 0, 0))
        return z

    xp = np.full((1, h + pt + pb + 8, w + pl + pr + 8, c), xz, np.int64)
    xp[:, pt:pt + h, pl:pl + w, :] = x
    acc = np.zeros((1, oh, ow, c), np.int64)
    for ky in range(k):
        for kx in range(k):
            win = xp[:, ky * dl: ky * dl + (oh - 1) * st + 1: st, kx * dl: kx * dl + (ow - 1) * st + 1: st, :] + 128
            acc += win * wt[ky, kx].astype(np.int64)
    want = _requant(acc, bias, m, s, yz, -128, 127)
    plan = _single_op_plan((1, h, w, c), xz, build_dw)
    np.testing.assert_array_equal(oracle_run(plan, x, 1, want.size).reshape(want.shape), want)

    # pooling: dilation 1, explicit padding that leaves no empty window
    kp_ = min(k, h, w)
    pt2, pl2 = int(rng.integers(0, kp_)), int(rng.integers(0, kp_))
    oh2 = (h + pt2 - kp_) // st + 1
    ow2 = (w + pl2 - kp_) // st + 1
    for is_max in (0, 1):
        lo, hi = int(rng.integers(-128, 0)), int(rng.integers(0, 128))

        def build_pool(p, xi):
            q = [kp_, kp_, st, st, 1, 1, pt2, pl2, 0, 0, oh2, ow2, xz, xz, lo, hi, c, c, 8, is_max]
            qt = p.tensor((20,), P.TYPE_I32, q)
            z = p.tensor((1, oh2, ow2, c))
            p._op(16, xi, xi, z, (qt, 0, 0, 0))
            return z

        want = np.zeros((1, oh2, ow2, c), np.int64)
        for oy in range(oh2):
            for ox in range(ow2):
                ys = [oy * st - pt2 + t for t in range(kp_) if 0 <= oy * st - pt2 + t < h]
                xs = [ox * st - pl2 + t for t in range(kp_) if 0 <= ox * st - pl2 + t < w]
                win = x[0][np.ix_(ys, xs)].reshape(-1, c).astype(np.int64)
                if is_max:
                    v = np.maximum(win.max(axis=0), -128)
                else:
                    cnt = win.shape[0]
                    tot = win.sum(axis=0)
                    v = np.array([int(Fraction(int(t), cnt) + (Fraction(cnt // 2, cnt) if t > 0 else -Fraction(cnt // 2, cnt)))
                                  for t in tot])  # C division truncates toward zero
                want[0, oy, ox] = np.clip(v, lo, hi)
        plan = _single_op_plan((1, h, w, c), xz, build_pool)
        np.testing.assert_array_equal(oracle_run(plan, x, 1, want.size).reshape(want.shape), want.astype(np.int8))


def test_mean_and_add_definitions():
    rng = np.random.default_rng(3)
    x = rng.integers(-128, 128, (2, 5, 3, 6)).astype(np.int8)
    p = P.Plan(2)
    xi = p.input((2, 5, 3, 6), zp=-9)
    z = p.mean(xi, keepdims=False, scale_ratio=0.7, yz=4)
    plan = p.build(z)
    q = np.frombuffer(plan, "<i4", count=5, offset=P._arena_offset(plan) + P.tensor_records(plan)[1][0])
    cnt, xz, yz, qm, qs = (int(v) for v in q)
    sums = x.astype(np.int64).reshape(2, 15, 6).sum(axis=1)
    want = np.clip([[scale_exact(int(t) - cnt * xz, qm, qs) + yz for t in row] for row in sums], -128, 127)
    np.testing.assert_array_equal(oracle_run(plan, x, 1, 12).reshape(2, 6), want)

    p = P.Plan(3)
    a = p.input((1, 16, 16, 1), zp=-27)
    b = p.tensor((1, 16, 16, 1), P.TYPE_I8, np.arange(-128, 128, dtype=np.int8))
    p.zp[b] = 13
    z = p.add(a, b, act="relu", yz=-5, scales=(.0625, .03125, .125))
    plan = p.build(z)
    tab = np.frombuffer(plan, "<i4", count=520, offset=P._arena_offset(plan) + P.tensor_records(plan)[2][0])
    xa = np.arange(-128, 128, dtype=np.int8)[::-1].copy()
    bb = np.arange(-128, 128)
    want = [min(max(scale_exact(int(tab[8 + int(xa[i]) + 128]) + int(tab[264 + int(bb[i]) + 128]), int(tab[0]), int(tab[1])) + int(tab[2]),
                    int(tab[3])), int(tab[4])) for i in range(256)]
    np.testing.assert_array_equal(oracle_run(plan, xa, 1, 256), np.array(want, np.int8))
