"""The five seeded INT8 workloads, as batch-1 plans plus an image count.

Every plan is a single-image plan in the reference's format (the reference
loader caps one plan at a 16 MiB arena and 2e9 MACs, graph.h:7-9); batches are
run by stacking images on the leading dimension through the batch entry point.

  pointwise   1x1 conv 56x56x32 -> 64, batch 1, xz -3, yz 5, ReLU6
  dw3s1 / dw3s2 / dw5s1 / dw5s2
              depthwise microbenchmarks, batch 64
  mnv4        MobileNetV4-Conv-Small-shaped classifier, 224x224x3, batch 256
              (the 60-op topology of models/mobilenetv4-small.uqmodel)
  yolo        YOLO26n-shaped detector, 320x320x3, batch 64
  head        1x1 7x7x960 -> 1280, batch 512 (M=25088, K=960, N=1280)
  conv3x3     3x3 s1 80x80x128 -> 128, batch 512 (K=1152)
"""
import numpy as np

from uq_plan import Plan, Rng

# 6/ys for the ReLU6 clamp of the pointwise case; the scale is not given by
# the workload description, so it is fixed here: ys = 0.05 -> q6 = 120.
POINTWISE_Q6 = 120


def pointwise(seed=0, tail_weights=False):
    p = Plan(seed)
    x = p.input((1, 56, 56, 32), zp=-3)
    z = p.conv(x, 64, k=1, act="relu6", yz=5, q6=POINTWISE_Q6, w_sigma=40, bias_sigma=4096,
               shift=(-10, -4), tail_weights=tail_weights)
    return p.build(z), 1


DW_CASES = {
    "dw3s1": dict(hw=112, c=32, k=3, stride=1),
    "dw3s2": dict(hw=112, c=64, k=3, stride=2),
    "dw5s1": dict(hw=28, c=240, k=5, stride=1),
    "dw5s2": dict(hw=56, c=96, k=5, stride=2),
}


def depthwise(case, seed=1, images=64):
    spec = DW_CASES[case]
    p = Plan(seed * 100 + list(DW_CASES).index(case))
    x = p.input((1, spec["hw"], spec["hw"], spec["c"]), zp=int(Rng(seed, 5).integers(1, -128, 127)[0]))
    z = p.depthwise(x, k=spec["k"], stride=spec["stride"], act="relu6", yz=-20, q6=110,
                    w_sigma=40, bias_sigma=2048, shift=(-10, -4))
    return p.build(z), images


def mnv4(seed=2, images=256, calibrate=True):
    """MobileNetV4-Conv-Small-shaped network: stem, fused-IB stages, UIB blocks
    with 3x3/5x5 depthwise, residual adds, global mean, 1x1 head to 1280 and a
    1000-way classifier; same op sequence and shapes as the reference's bundled
    plan, with seeded random constants."""
    p = Plan(seed, threads=2)
    c = dict(calibrate=calibrate)
    x = p.input((1, 224, 224, 3), zp=-13)
    t = p.conv(x, 32, k=3, stride=2, act="relu", yz=-128, **c)            # stem
    t = p.conv(t, 32, k=3, stride=2, act="relu", yz=-128, **c)            # fused IB
    t = p.conv(t, 32, k=1, act="none", **c)
    t = p.conv(t, 96, k=3, stride=2, act="relu", yz=-128, **c)
    t = p.conv(t, 64, k=1, act="none", **c)
    t = p.depthwise(t, k=5, act="none", **c)                               # UIB ExtraDW
    t = p.conv(t, 192, k=1, act="relu", yz=-128, **c)
    t = p.depthwise(t, k=5, stride=2, act="relu", yz=-128, **c)
    x1 = p.conv(t, 96, k=1, act="none", **c)
    for _ in range(4):                                                     # UIB IB, 14x14
        t = p.conv(x1, 192, k=1, act="relu", yz=-128, **c)
        t = p.depthwise(t, k=3, act="relu", yz=-128, **c)
        t = p.conv(t, 96, k=1, act="none", **c)
        x1 = p.add(t, x1)
    t = p.depthwise(x1, k=3, act="none", **c)                              # UIB ConvNext
    t = p.conv(t, 384, k=1, act="relu", yz=-128, **c)
    t = p.conv(t, 96, k=1, act="none", **c)
    x1 = p.add(t, x1)
    t = p.depthwise(x1, k=3, act="none", **c)                              # UIB ExtraDW s2
    t = p.conv(t, 576, k=1, act="relu", yz=-128, **c)
    t = p.depthwise(t, k=3, stride=2, act="relu", yz=-128, **c)
    y = p.conv(t, 128, k=1, act="none", **c)
    t = p.depthwise(y, k=5, act="none", **c)                               # UIB ExtraDW 7x7
    t = p.conv(t, 512, k=1, act="relu", yz=-128, **c)
    t = p.depthwise(t, k=5, act="relu", yz=-128, **c)
    t = p.conv(t, 128, k=1, act="none", **c)
    y = p.add(t, y)
    for expand, k in ((512, 5), (384, 5), (512, 3), (512, 3)):             # UIB IB 7x7
        t = p.conv(y, expand, k=1, act="relu", yz=-128, **c)
        t = p.depthwise(t, k=k, act="relu", yz=-128, **c)
        t = p.conv(t, 128, k=1, act="none", **c)
        y = p.add(t, y)
    t = p.conv(y, 960, k=1, act="relu", yz=-128, **c)
    t = p.mean(t)
    t = p.conv(t, 1280, k=1, act="relu", yz=-128, **c)
    t = p.copy(t)
    t = p.conv(t, 1000, k=1, act="none", **c)
    t = p.copy(t, (1, 1000))
    return p.build(t), images


def _act_table(fn, xs, xz, ys, yz):
    """256-entry int8 activation lookup (index = code + 128), seeded scales."""
    v = np.arange(-128, 128, dtype=np.float64)
    y = fn(xs * (v - xz)) / ys + yz
    return np.clip(np.rint(y), -128, 127).astype(np.int64).astype(np.int8).view(np.uint8)


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


class _Yolo:
    """Builder for the YOLO26n-shaped detector: C3k2 blocks split their 1x1
    output into channel halves with slices, requantise the halves through
    lookups, run bottlenecks with residual adds and concatenate the branches."""

    def __init__(self, p):
        self.p = p
        self.silu = p.lut_table(_act_table(_silu, 0.06, -100, 0.04, -120))

    def conv(self, x, oc, k=1, s=1):
        return self.p.conv(x, oc, k=k, stride=s, act="none", lut=self.silu, calibrate=True)

    def halves(self, t):
        n, h, w, c = self.p.shape(t)
        a = self.p.slice(t, (0, 0, 0, 0), (n, h, w, c // 2))
        b = self.p.slice(t, (0, 0, 0, c // 2), (n, h, w, c // 2))
        return a, b

    def bottleneck(self, x, c, hidden):
        t = self.conv(x, hidden, k=3)
        t = self.conv(t, c, k=3)
        return self.p.add(x, t)

    def c3k(self, x, c):
        h = c // 2
        a = self.conv(x, h)
        for _ in range(2):
            a = self.bottleneck(a, h, h)
        b = self.conv(x, h)
        return self.conv(self.p.concat(a, b), c)

    def c3k2(self, x, c_mid, c_out, inner_c3k=False):
        t = self.conv(x, c_mid)
        a, b = self.halves(t)
        half = c_mid // 2
        inner = self.c3k(b, half) if inner_c3k else self.bottleneck(b, half, half // 2)
        ta = self.p.lut(a, self.p.lut_table(_act_table(lambda z: z, 0.05, 0, 0.05, 3)))
        tb = self.p.lut(b, self.p.lut_table(_act_table(lambda z: z, 0.05, 0, 0.05, -2)))
        cat = self.p.concat(self.p.concat(ta, tb), inner)
        return self.conv(cat, c_out)

    def head(self, x, c_box, n_cls):
        p = self.p
        box = self.conv(self.conv(x, c_box, k=3), c_box, k=3)
        box = p.conv(box, 4, k=1, act="none", calibrate=True)
        cls = p.depthwise(x, k=3, act="none", lut=self.silu, calibrate=True)
        cls = self.conv(cls, c_box)
        cls = p.depthwise(cls, k=3, act="none", lut=self.silu, calibrate=True)
        cls = self.conv(cls, c_box)
        logits = p.conv(cls, n_cls, k=1, act="none", calibrate=True)
        sig = p.lut(logits, p.lut_table(_act_table(_sigmoid, 0.08, 0, 1 / 256, -128)))
        return box, sig


def yolo(seed=3, images=64):
    """YOLO26n-shaped int8 detector at 320x320x3: 3x3 s2 backbone convs, C3k2
    blocks with concat, SPPF max-pools, a neck with nearest 2x upsampling,
    concat and residual adds, and decoupled heads at strides 8/16/32 with
    80-class sigmoid scores (op 22 lookups) plus 4 box values; all six head
    outputs are packed into one output tensor (op 19)."""
    p = Plan(seed, threads=2)
    y = _Yolo(p)
    x = p.input((1, 320, 320, 3), zp=-128)
    t = y.conv(x, 16, k=3, s=2)                       # 160x160
    t = y.conv(t, 32, k=3, s=2)                       # 80x80
    t = y.c3k2(t, 32, 64)
    t = y.conv(t, 64, k=3, s=2)                       # 40x40
    p3 = y.c3k2(t, 64, 128)
    t = y.conv(p3, 128, k=3, s=2)                     # 20x20
    p4 = y.c3k2(t, 128, 128, inner_c3k=True)
    t = y.conv(p4, 256, k=3, s=2)                     # 10x10
    t = y.c3k2(t, 256, 256, inner_c3k=True)
    s0 = y.conv(t, 128)                               # SPPF
    s1 = p.pool(s0, 5, 1, kind="max")
    s2 = p.pool(s1, 5, 1, kind="max")
    s3 = p.pool(s2, 5, 1, kind="max")
    cat = p.concat(p.concat(p.concat(s0, s1), s2), s3)
    p5 = p.add(y.conv(cat, 256), t)
    u = p.resize(p5, 20, 20)                          # neck, top-down
    n4 = y.c3k2(p.concat(u, p4), 128, 128)
    u = p.resize(n4, 40, 40)
    o3 = y.c3k2(p.concat(u, p3), 64, 64)
    d = y.conv(o3, 64, k=3, s=2)                      # bottom-up
    o4 = y.c3k2(p.concat(d, n4), 128, 128)
    d = y.conv(o4, 128, k=3, s=2)
    o5 = y.c3k2(p.concat(d, p5), 256, 256, inner_c3k=True)
    outs = []
    for o in (o3, o4, o5):
        box, cls = y.head(o, 64, 80)
        outs += [box, cls]
    z = p.pack(outs)
    return p.build(z), images


def head(seed=4, images=512):
    p = Plan(seed)
    x = p.input((1, 7, 7, 960), zp=-7)
    z = p.conv(x, 1280, k=1, act="relu6", yz=-100, q6=120, w_sigma=40, bias_sigma=4096, calibrate=True)
    return p.build(z), images


def conv3x3(seed=5, images=512):
    p = Plan(seed)
    x = p.input((1, 80, 80, 128), zp=9)
    z = p.conv(x, 128, k=3, stride=1, act="relu6", yz=-100, q6=120, w_sigma=40, bias_sigma=4096, calibrate=True)
    return p.build(z), images


def lutcopy(seed=6, images=16):
    """Identity 256-entry lookup over 4 MiB per image: a plain streaming copy
    kernel of known size (reads and writes images * 4 MiB), used to calibrate
    the HBM byte counters."""
    p = Plan(seed)
    x = p.input((1, 1024, 1024, 4), zp=0)
    table = p.lut_table(np.arange(256, dtype=np.int64) ^ 128)
    z = p.lut(x, table)
    return p.build(z), images


WORKLOADS = {
    "pointwise": pointwise,
    "dw3s1": lambda **kw: depthwise("dw3s1", **kw),
    "dw3s2": lambda **kw: depthwise("dw3s2", **kw),
    "dw5s1": lambda **kw: depthwise("dw5s1", **kw),
    "dw5s2": lambda **kw: depthwise("dw5s2", **kw),
    "mnv4": mnv4,
    "yolo": yolo,
    "head": head,
    "conv3x3": conv3x3,
    "lutcopy": lutcopy,
}
