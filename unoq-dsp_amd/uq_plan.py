"""Synthetic INT8 graph plans in the reference's plan format, with seeded data.

The byte layout is the reference's plan ABI (graph.h:15-17, written by
tflite.py:305-307): a 32-byte header, 48-byte tensor records, 32-byte op
records, then a 128-byte-aligned arena holding the constants. Per-op constant
layouts follow qnn.c:12-16 (conv/depthwise/pool parameter block),
gemm.h:7-13 (packed conv weights), tflite.py:152-156 (depthwise weights and the
corrected bias), quantization.py:31-41 (ADD tables), tflite.py:261-273 (MEAN)
and tflite.py:196-202 (nearest resize offsets).

All random data comes from SplitMix64 streams keyed by (seed, stream id), so
the same plan and inputs are reproduced on any host from the seed alone.
"""
import math
import struct

import numpy as np

MAGIC = 0x55474E31
TYPE_I8, TYPE_U8, TYPE_I32 = 3, 2, 4
_DT = {TYPE_I8: np.int8, TYPE_U8: np.uint8, TYPE_I32: np.int32}
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


class Rng:
    """SplitMix64 (Steele, Lea & Flood 2014), vectorised over its counter."""

    def __init__(self, seed, stream=0):
        self.state = np.uint64((int(seed) * 1_000_003 + int(stream) * 7919) & (2**64 - 1))
        self.count = 0

    def u64(self, n):
        i = np.arange(self.count + 1, self.count + 1 + n, dtype=np.uint64)
        self.count += n
        with np.errstate(over="ignore"):
            z = self.state + i * _GOLDEN
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))

    def int8(self, n):
        """Uniform int8 in [-128, 127]: the low byte of each draw."""
        return (self.u64(n) & np.uint64(255)).astype(np.uint8).view(np.int8)

    def uniform01(self, n):
        return ((self.u64(n) >> np.uint64(11)).astype(np.float64) + 0.5) / float(1 << 53)

    def normal(self, n, sigma, lo=None, hi=None):
        """Box-Muller in double, round half to even, optional clamp."""
        u1, u2 = self.uniform01(n), self.uniform01(n)
        v = np.rint(sigma * np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2))
        if lo is not None:
            v = np.clip(v, lo, hi)
        return v.astype(np.int64)

    def integers(self, n, lo, hi):
        """Uniform integers in [lo, hi]."""
        return (lo + (self.u64(n) % np.uint64(hi - lo + 1)).astype(np.int64)).astype(np.int64)

    def multipliers(self, n):
        """Q31 multipliers uniform in [2^30, 2^31)."""
        return (np.int64(1 << 30) + (self.u64(n) % np.uint64(1 << 30)).astype(np.int64))


def frexp_multiplier(value):
    """Real scale -> (Q31 multiplier, exponent) with round-half-up significand.
    Same contract as the reference's compile-time helper (quantization.py:7-17)."""
    if not math.isfinite(value) or value < 0:
        raise ValueError("invalid multiplier")
    significand, exponent = math.frexp(value)
    integer = int(math.floor(significand * (1 << 31) + 0.5))
    if integer == 1 << 31:
        integer //= 2
        exponent += 1
    if exponent < -31:
        integer = exponent = 0
    return integer, exponent


def rounding_multiply(values, m, shift):
    """Double-rounding fixed-point multiply for shift <= 0, in int64 numpy."""
    v = np.asarray(values, dtype=np.int64)
    high = (v * m + (1 << 30)) >> 31
    if shift == 0:
        return high
    n = -shift
    mask = (1 << n) - 1
    return (high >> n) + ((high & mask) > ((mask >> 1) + (high < 0)))


def add_tables(xs, xz, bs, bz, ys, yz, lo, hi):
    """op18 parameter block: [ym, yshift, yz, lo, hi, 0, 0, 0] + two 256-entry
    tables of (v - z) * 2^20 rescaled to twice the larger input scale
    (layout graph.c:117-124, qnn.c:175-183)."""
    twice = 2 * max(xs, bs)
    xm, xsh = frexp_multiplier(xs / twice)
    bm, bsh = frexp_multiplier(bs / twice)
    ym, ysh = frexp_multiplier(twice / ((1 << 20) * ys))
    if ysh > 0:
        raise ValueError("ADD output scale too small")
    dom = np.arange(-128, 128, dtype=np.int64)
    tx = rounding_multiply((dom - xz) * (1 << 20), xm, xsh)
    tb = rounding_multiply((dom - bz) * (1 << 20), bm, bsh)
    return np.concatenate(([ym, ysh, yz, lo, hi, 0, 0, 0], tx, tb)).astype(np.int32)


def same_padding(size, k, stride, dilation):
    """TFLite SAME padding (tflite.py:139): (before, after, output)."""
    out = (size + stride - 1) // stride
    total = max(0, (out - 1) * stride + (k - 1) * dilation + 1 - size)
    return total // 2, total - total // 2, out


def clamp_range(act, yz, q6=None):
    """Fused activation clamp (tflite.py:61-66)."""
    if act == "none":
        return -128, 127
    if act == "relu":
        return max(-128, yz), 127
    if act == "relu6":
        return max(-128, yz), min(127, yz + q6)
    raise ValueError(act)


def pack_conv_weights(w2d, kp):
    """(OC, K) int8 -> packed bytes of gemm.h:7-13, K padded to kp, OC to 4."""
    oc, k = w2d.shape
    pw = np.zeros((kp, (oc + 3) // 4 * 4), dtype=np.int8)
    pw[:k, :oc] = w2d.T
    return pw.reshape(kp // 8, 8, -1, 4).transpose(2, 0, 3, 1).reshape(-1).copy()


class Plan:
    """Incremental plan builder. Activations carry a zero point; constants
    are laid into the arena on 128-byte boundaries."""

    def __init__(self, seed, threads=1):
        self.seed = seed
        self.threads = threads
        self.tensors = []      # dict(shape, type, offset, bytes, const)
        self.ops = []          # 8-tuples
        self.arena = bytearray()
        self.zp = {}
        self.input_id = None
        self.streams = 0
        self.macs = 0

    # -- storage -----------------------------------------------------------
    def rng(self):
        self.streams += 1
        return Rng(self.seed, self.streams)

    def tensor(self, shape, typ=TYPE_I8, values=None):
        shape = tuple(int(s) for s in shape)
        nbytes = int(np.prod(shape)) * np.dtype(_DT[typ]).itemsize
        off = (len(self.arena) + 127) & ~127
        self.arena.extend(bytes(off - len(self.arena)))
        if values is None:
            self.arena.extend(bytes(nbytes))
        else:
            raw = np.ascontiguousarray(values, dtype=_DT[typ]).tobytes()
            assert len(raw) == nbytes, (len(raw), nbytes)
            self.arena.extend(raw)
        self.tensors.append(dict(shape=shape, type=typ, offset=off, bytes=nbytes, const=values is not None))
        return len(self.tensors) - 1

    def shape(self, t):
        return self.tensors[t]["shape"]

    def input(self, shape, zp=0):
        t = self.tensor(shape)
        self.input_id = t
        self.zp[t] = zp
        return t

    def _op(self, code, a, b, z, p=(0, 0, 0, 0)):
        self.ops.append((code, a, b, z) + tuple(int(v) & 0xFFFFFFFF for v in p))

    # -- quantisation helpers --------------------------------------------
    def _requant_params(self, rng, oc, k, shift, calibrate, w_rows, zero_mult=0.0):
        m = rng.multipliers(oc)
        if zero_mult:
            m = np.where(rng.uniform01(oc) < zero_mult, 0, m)
        if calibrate:
            # Keep activations alive through deep nets: scale the expected
            # accumulator spread (uniform inputs, sd ~74) to ~48 output codes.
            sd = np.sqrt(np.maximum((w_rows.astype(np.float64) ** 2).sum(axis=1), 1.0)) * 74.0
            s = np.ceil(np.log2(48.0 / sd)).astype(np.int64)
            s = np.clip(s, -31, 0)
        elif shift is None:
            s = rng.integers(oc, -10, -4)
        else:
            s = rng.integers(oc, shift[0], shift[1])
        return m, s

    def _check_bound(self, corrected, w_rows, shift):
        lo = corrected + 255 * np.minimum(w_rows.astype(np.int64), 0).sum(axis=1)
        hi = corrected + 255 * np.maximum(w_rows.astype(np.int64), 0).sum(axis=1)
        f = np.left_shift(np.int64(1), np.maximum(shift, 0))
        if (np.any(corrected < -2**31) or np.any(corrected > 2**31 - 1)
                or np.any(lo * f < -2**31) or np.any(hi * f > 2**31 - 1)):
            raise ValueError("INT32 accumulation bound exceeded")

    # -- ops ---------------------------------------------------------------
    def conv(self, x, oc, k=1, stride=1, dilation=1, padding="same", act="relu", yz=None,
             w_sigma=40, bias_sigma=4096, shift=None, calibrate=False, q6=None, lut=None,
             tail_weights=False, scalar=False, kw=None, stride_w=None, zero_mult=0.0):
        """Code 14: conv / pointwise / FC on NHWC int8 (tflite.py:118-171)."""
        n, ih, iw, ic = self.shape(x)
        kh, kw = k, (k if kw is None else kw)
        sh, sw = stride, (stride if stride_w is None else stride_w)
        if padding == "same":
            pt, pb, oh = same_padding(ih, kh, sh, dilation)
            pl, pr, ow = same_padding(iw, kw, sw, dilation)
        else:
            pt, pl, pb, pr = padding
            oh = (ih + pt + pb - (kh - 1) * dilation - 1) // sh + 1
            ow = (iw + pl + pr - (kw - 1) * dilation - 1) // sw + 1
        rng = self.rng()
        xz = self.zp[x]
        yz = int(rng.integers(1, -128, 127)[0]) if yz is None else yz
        kk = kh * kw * ic
        kp = (kk + 7) & ~7
        w = rng.normal(oc * kk, w_sigma, -127, 127).reshape(oc, kk).astype(np.int8)
        packed = pack_conv_weights(w, kp)
        if tail_weights and kp > kk:
            # Hostile but admissible: nonzero weights in the padded K tail.
            tail = rng.normal(oc * (kp - kk), w_sigma, -127, 127).reshape(oc, kp - kk)
            full = np.zeros((oc, kp), dtype=np.int8)
            full[:, :kk] = w
            full[:, kk:] = tail
            packed = pack_conv_weights(full, kp)
            w_rows = full
        else:
            w_rows = w
        bias = rng.normal(oc, bias_sigma)
        corrected = bias - (xz + 128) * w.astype(np.int64).sum(axis=1)
        m, s = self._requant_params(rng, oc, kk, shift, calibrate, w_rows, zero_mult)
        self._check_bound(corrected, w_rows, s)
        lo, hi = clamp_range(act, yz, q6)
        q = [kh, kw, sh, sw, dilation, dilation, pt, pl, pb, pr, oh, ow, xz, yz, lo, hi, ic, oc, kp, int(scalar)]
        qt = self.tensor((20 + 3 * oc,), TYPE_I32, np.concatenate((q, corrected, m, s)))
        wt = self.tensor((len(packed),), TYPE_I8, packed)
        z = self.tensor((n, oh, ow, oc))
        self.zp[z] = yz
        self._op(14, x, wt, z, (qt, 0 if lut is None else lut + 1, 0, 0))
        self.macs += n * oh * ow * oc * kk
        return z

    def depthwise(self, x, k=3, stride=1, dilation=1, padding="same", act="relu", yz=None,
                  w_sigma=40, bias_sigma=2048, shift=None, calibrate=False, q6=None, lut=None, zero_mult=0.0):
        """Code 15: depthwise, multiplier one (tflite.py:152-153)."""
        n, ih, iw, c = self.shape(x)
        if padding == "same":
            pt, pb, oh = same_padding(ih, k, stride, dilation)
            pl, pr, ow = same_padding(iw, k, stride, dilation)
        else:
            pt, pl, pb, pr = padding
            oh = (ih + pt + pb - (k - 1) * dilation - 1) // stride + 1
            ow = (iw + pl + pr - (k - 1) * dilation - 1) // stride + 1
        rng = self.rng()
        xz = self.zp[x]
        yz = int(rng.integers(1, -128, 127)[0]) if yz is None else yz
        taps = k * k
        w = rng.normal(taps * c, w_sigma, -127, 127).reshape(taps, c).astype(np.int8)
        bias = rng.normal(c, bias_sigma)
        corrected = bias - (xz + 128) * w.astype(np.int64).sum(axis=0)
        m, s = self._requant_params(rng, c, taps, shift, calibrate, w.T, zero_mult)
        self._check_bound(corrected, w.T, s)
        lo, hi = clamp_range(act, yz, q6)
        q = [k, k, stride, stride, dilation, dilation, pt, pl, pb, pr, oh, ow, xz, yz, lo, hi, c, c, (taps + 7) & ~7, 0]
        qt = self.tensor((20 + 3 * c,), TYPE_I32, np.concatenate((q, corrected, m, s)))
        wt = self.tensor((taps * c,), TYPE_I8, w.reshape(-1))
        z = self.tensor((n, oh, ow, c))
        self.zp[z] = yz
        self._op(15, x, wt, z, (qt, 0 if lut is None else lut + 1, 0, 0))
        self.macs += n * oh * ow * c * taps
        return z

    def pool(self, x, k, stride, kind="max", padding="same", act="none"):
        """Code 16: average / max pool (tflite.py:274-281)."""
        n, ih, iw, c = self.shape(x)
        if padding == "same":
            oh, ow = (ih + stride - 1) // stride, (iw + stride - 1) // stride
            ph, pw = max(0, (oh - 1) * stride + k - ih), max(0, (ow - 1) * stride + k - iw)
            pt, pl, pb, pr = ph // 2, pw // 2, ph - ph // 2, pw - pw // 2
        else:
            pt = pl = pb = pr = 0
            oh, ow = (ih - k) // stride + 1, (iw - k) // stride + 1
        zp = self.zp[x]
        lo, hi = clamp_range(act, zp)
        q = [k, k, stride, stride, 1, 1, pt, pl, pb, pr, oh, ow, zp, zp, lo, hi, c, c, 8, int(kind == "max")]
        qt = self.tensor((20,), TYPE_I32, q)
        z = self.tensor((n, oh, ow, c))
        self.zp[z] = zp
        self._op(16, x, x, z, (qt, 0, 0, 0))
        return z

    def add(self, a, b, act="none", yz=None, scales=None):
        """Code 18: residual add with separate input scales (quantization.py:31-41)."""
        rng = self.rng()
        if scales is None:
            u = rng.uniform01(3)
            scales = (0.02 + 0.08 * u[0], 0.02 + 0.08 * u[1], 0.04 + 0.1 * u[2])
        xs, bs, ys = scales
        yz = int(rng.integers(1, -128, 127)[0]) if yz is None else yz
        lo, hi = clamp_range(act, yz, int(round(6 / ys)))
        q = add_tables(xs, self.zp[a], bs, self.zp[b], ys, yz, lo, hi)
        qt = self.tensor((520,), TYPE_I32, q)
        z = self.tensor(self.shape(a))
        self.zp[z] = yz
        self._op(18, a, b, z, (qt, 0, 0, 0))
        return z

    def mean(self, x, keepdims=True, scale_ratio=1.0, yz=None):
        """Code 24: spatial global mean (tflite.py:261-273)."""
        n, h, w, c = self.shape(x)
        xz = self.zp[x]
        yz = xz if yz is None else yz
        count = h * w
        qm, qs = frexp_multiplier(scale_ratio)
        adjust = min(count.bit_length() - 1, 32, 31 + qs)
        qm = (qm << adjust) // count
        qs -= adjust
        qt = self.tensor((5,), TYPE_I32, [count, xz, yz, qm, qs])
        z = self.tensor((n, 1, 1, c) if keepdims else (n, c))
        self.zp[z] = yz
        self._op(24, x, qt, z)
        return z

    def copy(self, x, shape=None):
        """Code 5: byte copy / reshape."""
        z = self.tensor(self.shape(x) if shape is None else shape, self.tensors[x]["type"])
        self.zp[z] = self.zp.get(x, 0)
        self._op(5, x, x, z)
        return z

    def concat(self, a, b, axis=3):
        """Code 20: same-quantisation concatenation."""
        sa, sb = self.shape(a), self.shape(b)
        out = list(sa)
        out[axis] += sb[axis]
        z = self.tensor(out)
        self.zp[z] = self.zp[a]
        self._op(20, a, b, z, (axis, 0, 0, 0))
        return z

    def resize(self, x, oh, ow):
        """Code 21: nearest resize with prepared offsets (tflite.py:196-202)."""
        n, ih, iw, c = self.shape(x)
        rows = np.clip(np.floor(np.arange(oh, dtype=np.float32) * np.float32(ih / oh)), 0, ih - 1).astype(np.int64)
        cols = np.clip(np.floor(np.arange(ow, dtype=np.float32) * np.float32(iw / ow)), 0, iw - 1).astype(np.int64)
        offs = np.concatenate((rows * iw * c, cols * c))
        bt = self.tensor((oh + ow,), TYPE_I32, offs)
        z = self.tensor((n, oh, ow, c))
        self.zp[z] = self.zp[x]
        self._op(21, x, bt, z)
        return z

    def lut_table(self, table):
        return self.tensor((256,), TYPE_U8, np.asarray(table, dtype=np.uint8))

    def lut(self, x, table_id, out_zp=None):
        """Code 22: byte-wise 256-entry lookup."""
        z = self.tensor(self.shape(x))
        self.zp[z] = self.zp[x] if out_zp is None else out_zp
        self._op(22, x, table_id, z)
        return z

    def pad(self, x, pads, value=None):
        """Code 23: constant padding, pads = [(before, after)] * 4."""
        s = self.shape(x)
        flat = [v for pr in pads for v in pr]
        bt = self.tensor((8,), TYPE_I32, flat)
        z = self.tensor([s[d] + pads[d][0] + pads[d][1] for d in range(4)])
        self.zp[z] = self.zp[x]
        self._op(23, x, bt, z, (self.zp[x] if value is None else value, 0, 0, 0))
        return z

    def slice(self, x, begin, size):
        """Code 26: slice, p = begin indices."""
        z = self.tensor(size)
        self.zp[z] = self.zp[x]
        self._op(26, x, x, z, tuple(list(begin) + [0] * (4 - len(begin))))
        return z

    def pack(self, ids):
        """Code 19: pack byte outputs in list order."""
        lt = self.tensor((len(ids),), TYPE_I32, ids)
        total = sum(self.tensors[t]["bytes"] for t in ids)
        z = self.tensor((total,))
        self._op(19, ids[0], lt, z)
        return z

    def transpose(self, x, perm):
        """Code 10: permutation of any rank (graph.c:374-390), z.d[i] = x.d[perm[i]]."""
        s = self.shape(x)
        z = self.tensor([s[d] for d in perm], self.tensors[x]["type"])
        self.zp[z] = self.zp.get(x, 0)
        self._op(10, x, x, z, tuple(list(perm) + [0] * (4 - len(perm))))
        return z

    def _product_requant(self, rng, k, yz):
        """Multiplier / shift for a sum of k products of zero-point-shifted int8
        values, spreading the result over ~48 codes; respects the loader's
        k * 255^2 * 2^max(shift, 0) <= 2147483520 bound (graph.c:189)."""
        m = int(rng.multipliers(1)[0])
        s = int(np.ceil(np.log2(48.0 / (np.sqrt(k) * 74.0 * 74.0)))) + int(rng.integers(1, -1, 1)[0])
        s = max(-31, min(s, 15))
        while k * 65025 * (1 << max(s, 0)) > 2147483520:
            s -= 1
        return m, s

    def mul(self, a, b, act="none", yz=None):
        """Code 25: elementwise product (qnn.c:111-116), q = [az, bz, yz, m, shift, lo, hi]."""
        rng = self.rng()
        yz = int(rng.integers(1, -128, 127)[0]) if yz is None else yz
        m, s = self._product_requant(rng, 1, yz)
        lo, hi = clamp_range(act, yz)
        qt = self.tensor((7,), TYPE_I32, [self.zp[a], self.zp[b], yz, m, s, lo, hi])
        z = self.tensor(self.shape(a))
        self.zp[z] = yz
        self._op(25, a, b, z, (qt, 0, 0, 0))
        return z

    def bmm(self, a, b, trans_a=False, trans_b=False, yz=None):
        """Code 27: batched int8 matmul of rank-3 tensors (qnn.c:117-153).
        a is [B][M][K] ([B][K][M] when trans_a), b is [B][K][N] ([B][N][K]
        when trans_b); q = [az, bz, yz, m, shift, trans_a, trans_b]."""
        sa, sb = self.shape(a), self.shape(b)
        mm, k = (sa[2], sa[1]) if trans_a else (sa[1], sa[2])
        n = sb[1] if trans_b else sb[2]
        assert (sb[2] if trans_b else sb[1]) == k and sa[0] == sb[0]
        rng = self.rng()
        yz = int(rng.integers(1, -128, 127)[0]) if yz is None else yz
        m, s = self._product_requant(rng, k, yz)
        qt = self.tensor((7,), TYPE_I32, [self.zp[a], self.zp[b], yz, m, s, int(trans_a), int(trans_b)])
        z = self.tensor((sa[0], mm, n))
        self.zp[z] = yz
        self._op(27, a, b, z, (qt, 0, 0, 0))
        self.macs += sa[0] * mm * n * k
        return z

    def softmax(self, x, beta_scale=None):
        """Code 28: exact int8 softmax over the last axis (qnn.c:87-107) with a
        257-entry table: width, then Q0.31 exp(-d * beta_scale) for d = 0..255."""
        rng = self.rng()
        if beta_scale is None:
            beta_scale = float(0.01 + 0.3 * rng.uniform01(1)[0])
        d = np.arange(256, dtype=np.float64)
        table = np.minimum(np.round(np.exp(-d * beta_scale) * 2.0 ** 31), 2147483647).astype(np.int64)
        table[0] = 2147483647
        bt = self.tensor((257,), TYPE_I32, np.concatenate(([self.shape(x)[-1]], table)))
        z = self.tensor(self.shape(x))
        self.zp[z] = -128
        self._op(28, x, bt, z)
        return z

    def softmax_table(self, x, beta_scale=None):
        """Code 17: table softmax (qnn.c:1082-1087), q = 20 header words
        (q[13] = q[14] = -128, q[15] = 127, q[16] = width) then 256 Q24
        exponentials exp(-d * beta_scale) * 2^24."""
        rng = self.rng()
        if beta_scale is None:
            beta_scale = float(0.01 + 0.3 * rng.uniform01(1)[0])
        d = np.arange(256, dtype=np.float64)
        table = np.round(np.exp(-d * beta_scale) * 2.0 ** 24).astype(np.int64)
        table[0] = 1 << 24
        q = [0] * 20
        q[12], q[13], q[14], q[15], q[16] = self.zp[x], -128, -128, 127, self.shape(x)[-1]
        qt = self.tensor((276,), TYPE_I32, np.concatenate((q, table)))
        z = self.tensor(self.shape(x))
        self.zp[z] = -128
        self._op(17, x, x, z, (qt, 0, 0, 0))
        return z

    # -- serialisation -----------------------------------------------------
    def build(self, output, version=2):
        hdr = struct.pack("<8I", MAGIC, version, len(self.tensors), len(self.ops), len(self.arena),
                          self.input_id, output, int(self.threads == 2))
        desc = b"".join(struct.pack("<12I", t["offset"], t["bytes"], t["type"], len(t["shape"]),
                                    *(list(t["shape"]) + [1] * (4 - len(t["shape"]))), int(t["const"]), 0, 0, 0)
                        for t in self.tensors)
        ops = b"".join(struct.pack("<8I", *o) for o in self.ops)
        return hdr + desc + ops + bytes(self.arena)


def input_bytes(plan):
    """Per-image input bytes of a serialised plan."""
    nt, inp = struct.unpack_from("<I", plan, 8)[0], struct.unpack_from("<I", plan, 20)[0]
    return struct.unpack_from("<I", plan, 32 + 48 * inp + 4)[0]


def output_bytes(plan):
    out = struct.unpack_from("<I", plan, 24)[0]
    return struct.unpack_from("<I", plan, 32 + 48 * out + 4)[0]


def tensor_records(plan):
    nt = struct.unpack_from("<I", plan, 8)[0]
    return [struct.unpack_from("<12I", plan, 32 + 48 * i) for i in range(nt)]


def op_records(plan):
    nt, no = struct.unpack_from("<II", plan, 8)
    base = 32 + 48 * nt
    return [struct.unpack_from("<8I", plan, base + 32 * i) for i in range(no)]


def random_input(plan, images, seed, stream=999):
    """Uniform int8 input for `images` stacked images."""
    return Rng(seed, stream).int8(images * input_bytes(plan))


def op_costs(plan, images):
    """Algorithmic work of each op for `images` stacked images.

    bytes: every input read once, every output written once, plus constants
    (weights, the 12 bytes of bias/multiplier/shift per output channel, tables).
    ops: 2*M*K*N for conv (K the logical kh*kw*ic), 2*M*taps*C for depthwise.
    """
    ts = tensor_records(plan)
    out = []
    for code, a, b, z, p0, p1, p2, p3 in op_records(plan):
        ab, bb, zb = ts[a][1], ts[b][1], ts[z][1]
        const_b = bb if ts[b][8] else images * bb
        act_a = images * ab
        ops = 0
        if code in (14, 15):
            q = np.frombuffer(plan, dtype="<i4", count=20, offset=_arena_offset(plan) + ts[p0][0])
            kh, kw, ic, oc = int(q[0]), int(q[1]), int(q[16]), int(q[17])
            m = images * (zb // oc)
            k = kh * kw * (ic if code == 14 else 1)
            ops = 2 * m * k * oc if code == 14 else 2 * m * k
            weights = oc * k
            nbytes = act_a + images * zb + weights + 12 * oc + (256 if p1 else 0)
        elif code == 16:
            nbytes = act_a + images * zb
        elif code == 18:
            nbytes = act_a + images * bb + images * zb + 2048
        elif code in (5, 22, 21, 23, 26, 24):
            nbytes = act_a + images * zb
        elif code == 20:
            nbytes = act_a + images * bb + images * zb
        elif code == 19:
            nbytes = 2 * images * zb
        else:
            nbytes = act_a + const_b + images * zb
        out.append(dict(code=code, bytes=int(nbytes), ops=int(ops)))
    return out


def _arena_offset(plan):
    nt, no = struct.unpack_from("<II", plan, 8)
    return 32 + 48 * nt + 32 * no
