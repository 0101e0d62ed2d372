"""Random small plans that exercise every op of the INT8 vision path with
edge-case geometry: odd channel counts, 1xN kernels, strides 1-3, dilation,
explicit and SAME padding, K tails with nonzero weights, positive shifts,
zero multipliers, fused post tables, batch/channel padding, slices, concat on
every axis, resize, pooling, mean, packed outputs, elementwise products,
permutations and attention (batched matmul with either operand transposed,
exact softmax)."""
import numpy as np

from uq_plan import Plan, Rng


def _pick(rng, values):
    return values[int(rng.integers(1, 0, len(values) - 1)[0])]


def _geometry(rng, size, k, stride, dilation):
    """Random explicit padding that leaves at least one output position."""
    before, after = (int(v) for v in rng.integers(2, 0, 2))
    need = (k - 1) * dilation + 1 - size
    return before, max(after, need - before)


def _random_lut(plan, rng):
    return plan.lut_table(rng.int8(256).view(np.uint8))


def conv_op(p, rng, x):
    n, ih, iw, ic = p.shape(x)
    oc = _pick(rng, [1, 2, 3, 4, 5, 8, 16, 17, 32, 40, 64, 96])
    kh, kw = _pick(rng, [1, 1, 2, 3, 3, 5]), _pick(rng, [1, 1, 2, 3, 3, 5])
    sh, sw = _pick(rng, [1, 1, 2, 3]), _pick(rng, [1, 1, 2, 3])
    dil = _pick(rng, [1, 1, 1, 2])
    if kh * kw * ic > 8192:
        kh = kw = 1
    if _pick(rng, [0, 1]):
        padding = "same"
        if sh != sw:
            sw = sh
    else:
        pt, pb = _geometry(rng, ih, kh, sh, dil)
        pl, pr = _geometry(rng, iw, kw, sw, dil)
        padding = (pt, pl, pb, pr)
    act = _pick(rng, ["none", "relu", "relu6"])
    lut = _random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None
    kwargs = dict(k=kh, kw=kw, stride=sh, stride_w=sw, dilation=dil, padding=padding, act=act, q6=int(rng.integers(1, 1, 200)[0]),
                  lut=lut, tail_weights=bool(_pick(rng, [0, 1])), scalar=bool(_pick(rng, [0, 0, 0, 1])),
                  zero_mult=_pick(rng, [0.0, 0.0, 0.3]), w_sigma=_pick(rng, [3, 40, 90]))
    lo = int(rng.integers(1, -24, -1)[0])
    for shift in ((lo, 3), (lo, 0), (-12, -4)):
        try:
            return p.conv(x, oc, shift=shift, **kwargs)
        except ValueError:
            continue
    raise AssertionError("unreachable")


def dw_op(p, rng, x):
    n, ih, iw, c = p.shape(x)
    k = _pick(rng, [1, 2, 3, 3, 5, 5])
    stride = _pick(rng, [1, 1, 2, 3])
    dil = _pick(rng, [1, 1, 2])
    if _pick(rng, [0, 1]):
        padding = "same"
    else:
        pt, pb = _geometry(rng, ih, k, stride, dil)
        pl, pr = _geometry(rng, iw, k, stride, dil)
        padding = (pt, pl, pb, pr)
    lut = _random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None
    lo = int(rng.integers(1, -24, -1)[0])
    for shift in ((lo, 3), (-12, -4)):
        try:
            return p.depthwise(x, k=k, stride=stride, dilation=dil, padding=padding,
                               act=_pick(rng, ["none", "relu", "relu6"]), q6=int(rng.integers(1, 1, 200)[0]),
                               lut=lut, shift=shift, zero_mult=_pick(rng, [0.0, 0.3]),
                               w_sigma=_pick(rng, [3, 40, 90]), bias_sigma=_pick(rng, [0, 2048, 60000]))
        except ValueError:
            continue
    raise AssertionError("unreachable")


def pool_op(p, rng, x):
    n, ih, iw, c = p.shape(x)
    k = _pick(rng, [1, 2, 3, 5])
    stride = _pick(rng, [1, 2, 3])
    if k > min(ih, iw):
        k = min(ih, iw)
    return p.pool(x, k, stride, kind=_pick(rng, ["max", "avg"]), padding=_pick(rng, ["same", "valid"]),
                  act=_pick(rng, ["none", "relu"]))


def pad_op(p, rng, x):
    pads = [tuple(int(v) for v in rng.integers(2, 0, 2)) for _ in range(4)]
    if _pick(rng, [0, 1]):
        pads[0] = (0, 0)
    return p.pad(x, pads, value=int(rng.integers(1, -128, 127)[0]))


def slice_op(p, rng, x):
    s = p.shape(x)
    begin, size = [], []
    for d in s:
        b = int(rng.integers(1, 0, d - 1)[0])
        size.append(int(rng.integers(1, 1, d - b)[0]))
        begin.append(b)
    return p.slice(x, begin, size)


def resize_op(p, rng, x):
    n, ih, iw, c = p.shape(x)
    return p.resize(x, int(rng.integers(1, 1, 2 * ih + 1)[0]), int(rng.integers(1, 1, 2 * iw + 1)[0]))


def add_op(p, rng, x):
    other = p.lut(x, _random_lut(p, rng)) if _pick(rng, [0, 1]) else x
    return p.add(x, other, act=_pick(rng, ["none", "relu", "relu6"]))


def concat_op(p, rng, x):
    other = p.lut(x, _random_lut(p, rng))
    return p.concat(x, other, axis=_pick(rng, [0, 1, 2, 3, 3]))


def mul_op(p, rng, x):
    other = p.lut(x, _random_lut(p, rng)) if _pick(rng, [0, 1]) else x
    return p.mul(x, other, act=_pick(rng, ["none", "relu"]))


def transpose_op(p, rng, x):
    """A 4-D permutation and its inverse, so the chain stays NHWC-shaped."""
    perm = [int(v) for v in np.argsort(rng.uniform01(4))]
    y = p.transpose(x, perm)
    if _pick(rng, [0, 1]):
        y = p.lut(y, _random_lut(p, rng))
    inverse = [perm.index(d) for d in range(4)]
    return p.transpose(y, inverse)


def attention_op(p, rng, x):
    """Self-attention on rank-3 views, as the detector's attention block:
    S = bmm(Q, K^T), P = softmax(S) (exact code 28 or table code 17),
    O = bmm(P, V)."""
    n, h, w, c = p.shape(x)
    q = p.copy(x, (n * h, w, c))
    kq = p.lut(q, _random_lut(p, rng))
    kt_stored = _pick(rng, [0, 1])
    k_op = kq if kt_stored else p.transpose(kq, (0, 2, 1))            # [B][N][K] or [B][K][N]
    ta = _pick(rng, [0, 0, 1])
    a = p.transpose(q, (0, 2, 1)) if ta else q
    scores = p.bmm(a, k_op, trans_a=bool(ta), trans_b=bool(kt_stored))   # [B][w][w]
    probs = p.softmax(scores) if _pick(rng, [0, 0, 1]) == 0 else p.softmax_table(scores)
    v = p.lut(q, _random_lut(p, rng))                                  # [B][w][c]
    out = p.bmm(probs, v)                                              # [B][w][c]
    return p.copy(out, (n, h, w, c))


def _constant_like(p, rng, shape):
    t = p.tensor(shape, values=rng.int8(int(np.prod(shape))))
    p.zp[t] = int(rng.integers(1, -128, 127)[0])
    return t


def constant_operand_op(p, rng, x):
    """A constant tensor in a slot the runtime reads image by image: the
    second operand of add / concat / mul, or the input of a LUT or copy
    (graph.c:72 admits any defined tensor there, constants included)."""
    kind = _pick(rng, ["add", "concat", "mul", "lut", "copy"])
    c = _constant_like(p, rng, p.shape(x))
    if kind == "add":
        return p.add(x, c) if _pick(rng, [0, 1]) else p.add(c, x)
    if kind == "concat":
        return p.concat(x, c, axis=_pick(rng, [0, 1, 2, 3]))
    if kind == "mul":
        return p.mul(x, c)
    y = p.lut(c, _random_lut(p, rng)) if kind == "lut" else p.copy(c)
    return p.add(x, y)


def constant_bmm_op(p, rng, x):
    """bmm with a constant right-hand matrix, as a compiled BATCH_MATMUL with
    a weight buffer (tests/test_modern_ops.py:87-94 pattern)."""
    n, h, w, c = p.shape(x)
    a = p.copy(x, (n * h, w, c))
    tb = _pick(rng, [0, 1])
    cols = _pick(rng, [1, 3, 8, 17, 32, 33])
    b = _constant_like(p, rng, (n * h, cols, c) if tb else (n * h, c, cols))
    z = p.bmm(a, b, trans_b=bool(tb))
    return p.copy(z, (n, h, w, cols))


OPS = [conv_op, conv_op, conv_op, dw_op, dw_op, pool_op, pad_op, slice_op, resize_op, add_op, concat_op,
       mul_op, transpose_op, attention_op]
ATTENTION_OPS = [attention_op, attention_op, transpose_op, mul_op, conv_op, constant_bmm_op]
CONSTANT_OPS = [constant_operand_op, constant_operand_op, constant_bmm_op, conv_op, dw_op]


def random_plan(seed, max_ops=4, ops=None):
    """A small random chain (plan bytes) drawn from `ops` (default: all)."""
    rng = Rng(seed, 424242)
    p = Plan(seed)
    shape = (int(_pick(rng, [1, 1, 2])), int(rng.integers(1, 1, 12)[0]), int(rng.integers(1, 1, 12)[0]),
             int(_pick(rng, [1, 2, 3, 4, 8, 12, 16, 24, 32, 48, 64])))
    t = p.input(shape, zp=int(rng.integers(1, -128, 127)[0]))
    for _ in range(int(rng.integers(1, 1, max_ops)[0])):
        t = _pick(rng, OPS if ops is None else ops)(p, rng, t)
    tail = _pick(rng, ["none", "mean", "pack", "copy"])
    if tail == "mean":
        t = p.mean(t, keepdims=bool(_pick(rng, [0, 1])), scale_ratio=float(0.3 + rng.uniform01(1)[0]))
    elif tail == "pack":
        extra = p.lut(t, _random_lut(p, rng))
        t = p.pack([t, extra])
    elif tail == "copy":
        t = p.copy(t)
    return p.build(t)


def conv_add_plan(seed):
    """A residual block x -> conv -> {lut (the residual), 1x1 conv} -> add,
    the add's operands in either order: the pattern the GPU library runs as
    one launch (the add in the 1x1 conv's epilogue). Channel counts cover
    16-multiples and byte tails; post tables, activations and both
    requantisation ranges vary; the sum is sometimes used further on."""
    rng = Rng(seed, 515151)
    p = Plan(seed)
    shape = (int(_pick(rng, [1, 1, 2])), int(rng.integers(1, 1, 10)[0]), int(rng.integers(1, 1, 10)[0]),
             int(_pick(rng, [16, 32, 48, 64])))
    t = p.input(shape, zp=int(rng.integers(1, -128, 127)[0]))
    c = _pick(rng, [16, 32, 48, 64, 96])
    q6 = int(rng.integers(1, 1, 200)[0])
    h = p.conv(t, c, k=1, act=_pick(rng, ["none", "relu", "relu6"]), q6=q6, shift=(-12, -4))
    residual = p.lut(h, _random_lut(p, rng))
    lut = _random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None
    lo = int(rng.integers(1, -24, -1)[0])
    shift = _pick(rng, [(lo, 3), (-12, -4), (-20, -1)])
    y = p.conv(h, c, k=1, act=_pick(rng, ["none", "relu", "relu6"]), q6=q6, lut=lut, shift=shift,
               zero_mult=_pick(rng, [0.0, 0.0, 0.3]), w_sigma=_pick(rng, [3, 40, 90]),
               tail_weights=bool(_pick(rng, [0, 1])))
    act = _pick(rng, ["none", "relu", "relu6"])
    z = p.add(y, residual, act=act) if _pick(rng, [0, 1]) else p.add(residual, y, act=act)
    if _pick(rng, [0, 1]):
        z = p.conv(z, _pick(rng, [8, 16, 17]), k=1, shift=(-12, -4))
    return p.build(z)


def pointwise_wide_plan(seed):
    """A 1x1 conv over 16384-pixel maps (two images give the GPU's widest
    channel tiles and two row blocks, its register-direct store): channel
    counts with and without a partly used last tile, post tables, activations
    and all requantisation ranges."""
    rng = Rng(seed, 626262)
    p = Plan(seed)
    h, w = _pick(rng, [(128, 128), (64, 256), (256, 64)])
    x = p.input((1, h, w, int(_pick(rng, [16, 32, 64, 96]))), zp=int(rng.integers(1, -128, 127)[0]))
    lo = int(rng.integers(1, -24, -1)[0])
    shift = _pick(rng, [(lo, 3), (-12, -4), (-20, -1)])
    y = p.conv(x, _pick(rng, [64, 80, 96, 112, 128, 192, 256]), k=1, act=_pick(rng, ["none", "relu", "relu6"]),
               q6=int(rng.integers(1, 1, 200)[0]), lut=_random_lut(p, rng) if _pick(rng, [0, 1]) else None,
               shift=shift, w_sigma=_pick(rng, [3, 40, 90]), tail_weights=bool(_pick(rng, [0, 1])))
    return p.build(y)


def gather_plan(seed):
    """YOLO's C3k2 split / table / concat chains and their variants: a conv
    output split in two along the channels (slices of the last axis), each
    half through its own table, the halves concatenated and that concatenated
    with another tensor (on either side); sometimes a half has other readers
    (its slice stays a launch), a table reads a plain tensor, the inner
    concat is of plain tensors, or an op follows. Channel counts that leave
    rows unaligned to 4 and 16 bytes, maps of 1x1 to 9x9; every fifth plan
    YOLO's SPPF chain of three concats."""
    rng = Rng(seed, 919191)
    p = Plan(seed)
    h, w = _pick(rng, [(1, 1), (3, 5), (8, 8), (9, 7), (2, 2)])
    x0 = p.input((1, h, w, int(_pick(rng, [8, 16, 32]))), zp=int(rng.integers(1, -128, 127)[0]))
    c = int(_pick(rng, [2, 5, 12, 16, 32, 48, 64]))
    x = p.conv(x0, c, k=1, act="none", shift=(-12, -4))
    if seed % 5 == 4:
        # YOLO's SPPF: three chained concats of a map and its pooled copies
        # (nested concats, four segments); sometimes a table on the last one.
        y1 = p.pool(x, 5, 1)
        y2 = p.pool(y1, 5, 1)
        y3 = p.pool(y2, 5, 1)
        if _pick(rng, [0, 1]):
            y3 = p.lut(y3, _random_lut(p, rng))
        out = p.concat(p.concat(p.concat(x, y1, axis=3), y2, axis=3), y3, axis=3)
        return p.build(p.conv(out, 16, k=1, act="none", shift=(-12, -4)))
    split = int(rng.integers(1, 1, c - 1)[0]) if c > 2 else 1
    a = p.slice(x, [0, 0, 0, 0], [1, h, w, split])
    b = p.slice(x, [0, 0, 0, split], [1, h, w, c - split])
    shape = int(_pick(rng, [0, 0, 1, 2, 3]))
    if shape == 1:
        # The second half also feeds a conv whose output joins the concat.
        m = p.conv(b, int(_pick(rng, [4, 16, 24])), k=1, act="relu", shift=(-12, -4))
    else:
        m = p.conv(x, int(_pick(rng, [3, 16, 32])), k=1, act="relu", shift=(-12, -4))
    la = p.lut(a, _random_lut(p, rng))
    lb = p.lut(b, _random_lut(p, rng)) if shape != 2 else p.copy(b)
    inner = p.concat(la, lb, axis=3) if shape != 3 else la
    out = p.concat(inner, m, axis=3) if _pick(rng, [0, 1]) else p.concat(m, inner, axis=3)
    if _pick(rng, [0, 0, 1]):
        out = p.conv(out, 16, k=1, act="none", shift=(-12, -4))
    return p.build(out)


def conv_lut_plan(seed):
    """A conv (1x1, 3x3, stride 1 or 2, with or without its own post table)
    whose output feeds only a table lookup, sometimes followed by another op;
    sometimes the conv's output has a second reader (then nothing is fused)."""
    rng = Rng(seed, 959595)
    p = Plan(seed)
    h, w = _pick(rng, [(1, 1), (5, 7), (16, 16), (9, 3)])
    x = p.input((1, h, w, int(_pick(rng, [3, 8, 16, 32, 64]))), zp=int(rng.integers(1, -128, 127)[0]))
    k = int(_pick(rng, [1, 1, 3]))
    y = p.conv(x, int(_pick(rng, [8, 16, 20, 64, 80])), k=k, stride=int(_pick(rng, [1, 2])) if k == 3 else 1,
               act=_pick(rng, ["none", "relu", "relu6"]), q6=int(rng.integers(1, 1, 200)[0]),
               lut=_random_lut(p, rng) if _pick(rng, [0, 1]) else None, shift=(-12, -4),
               w_sigma=_pick(rng, [3, 40, 90]))
    z = p.lut(y, _random_lut(p, rng))
    if _pick(rng, [0, 0, 0, 1]):
        z = p.concat(z, y, axis=3)
    if _pick(rng, [0, 1]):
        z = p.conv(z, 16, k=1, act="none", shift=(-12, -4))
    return p.build(z)


def pack_plan(seed):
    """A pack (code 19) of two to nine outputs of different sizes (tables and
    1x1 convs of one input, rows unaligned to 4 and 16 bytes; nine is past
    what one row gather takes)."""
    rng = Rng(seed, 939393)
    p = Plan(seed)
    h, w = _pick(rng, [(1, 1), (3, 5), (8, 8), (2, 7)])
    x = p.input((1, h, w, int(_pick(rng, [3, 8, 16]))), zp=int(rng.integers(1, -128, 127)[0]))
    outs = []
    for _ in range(int(_pick(rng, [2, 3, 6, 8, 9]))):
        if _pick(rng, [0, 1]):
            outs.append(p.lut(x, _random_lut(p, rng)))
        else:
            outs.append(p.conv(x, int(_pick(rng, [1, 5, 16, 20])), k=1, act="none", shift=(-12, -4)))
    return p.build(p.pack(outs))


def conv_mean_plan(seed):
    """A 1x1 conv followed by the global mean over its output (the classifier
    head the fused conv + mean kernel takes): maps of 1 to 64 pixels, input
    channels 32-256, output channels multiples of 32, post tables,
    activations, all requantisation ranges, the mean's own scale and zero
    point; sometimes an op after the mean, sometimes a second reader of the
    conv's output (then nothing is fused)."""
    rng = Rng(seed, 454545)
    p = Plan(seed)
    h, w = _pick(rng, [(7, 7), (1, 1), (8, 8), (4, 9), (3, 5), (2, 2), (7, 9)])
    x = p.input((1, h, w, int(_pick(rng, [32, 64, 96, 128, 256]))), zp=int(rng.integers(1, -128, 127)[0]))
    lo = int(rng.integers(1, -24, -1)[0])
    shift = _pick(rng, [(lo, 3), (-12, -4), (-20, -1)])
    y = p.conv(x, _pick(rng, [32, 64, 96, 160, 320, 960]), k=1, act=_pick(rng, ["none", "relu", "relu6"]),
               q6=int(rng.integers(1, 1, 200)[0]), lut=_random_lut(p, rng) if _pick(rng, [0, 1]) else None,
               shift=shift, w_sigma=_pick(rng, [3, 40, 90]))
    m = p.mean(y, scale_ratio=float(_pick(rng, [1.0, 0.37, 2.5])), yz=int(rng.integers(1, -20, 20)[0]))
    if _pick(rng, [0, 0, 1]):
        m = p.conv(m, 32, k=1, act="none", shift=(-12, -4))
    if _pick(rng, [0, 0, 0, 1]):
        # A second reader of the conv's output: the pair is not fused.
        m = p.concat(m, p.mean(y), axis=3)
    return p.build(m)


def conv_add_bytes_plan(seed):
    """As conv_add_plan with channel counts that are not multiples of 16 (the
    epilogue's byte path)."""
    rng = Rng(seed, 616161)
    p = Plan(seed)
    shape = (1, int(rng.integers(1, 1, 9)[0]), int(rng.integers(1, 1, 9)[0]), int(_pick(rng, [16, 32])))
    t = p.input(shape, zp=int(rng.integers(1, -128, 127)[0]))
    c = _pick(rng, [3, 5, 8, 12, 17, 20, 36])
    h = p.lut(t, _random_lut(p, rng))
    y = p.conv(h, c, k=1, act=_pick(rng, ["none", "relu"]), shift=(-12, -4))
    r = p.conv(t, c, k=1, act="none", shift=(-12, -4))
    z = p.add(y, r) if _pick(rng, [0, 1]) else p.add(r, y)
    return p.build(z)


def dw_mfma_plan(seed):
    """A depthwise layer the matrix-core kernel takes: 3x3 or 5x5, stride 1
    or 2, 16-64 channels, maps from 3x3 to banded sizes (padded windows over
    40 KiB), SAME or explicit padding, optional post table, both
    requantisation ranges."""
    rng = Rng(seed, 717171)
    p = Plan(seed)
    hw = _pick(rng, [3, 5, 7, 9, 14, 17, 28, 33, 56, 80])
    c = _pick(rng, [16, 32, 48, 64])
    n = 1 if hw >= 56 else _pick(rng, [1, 2])
    x = p.input((n, hw, hw, c), zp=int(rng.integers(1, -128, 127)[0]))
    k = _pick(rng, [3, 5])
    stride = _pick(rng, [1, 2])
    if _pick(rng, [0, 1]):
        padding = "same"
    else:
        pt, pb = _geometry(rng, hw, k, stride, 1)
        padding = (pt, pt, pb, pb)
    lut = _random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None
    lo = int(rng.integers(1, -24, -1)[0])
    for shift in ((lo, 3), (-12, -4), (-20, -1)):
        try:
            y = p.depthwise(x, k=k, stride=stride, padding=padding, act=_pick(rng, ["none", "relu", "relu6"]),
                            q6=int(rng.integers(1, 1, 200)[0]), lut=lut, shift=shift,
                            zero_mult=_pick(rng, [0.0, 0.3]), w_sigma=_pick(rng, [3, 40, 90]),
                            bias_sigma=_pick(rng, [0, 2048, 60000]))
            return p.build(y)
        except ValueError:
            continue
    raise AssertionError("unreachable")


def stem_plan(seed):
    """A stem conv (IC 1-4, kh*kw <= 16, OC a multiple of 16): widths past 128
    output columns (several row segments), strides 1-2, odd sizes."""
    rng = Rng(seed, 818181)
    p = Plan(seed)
    ic = _pick(rng, [1, 2, 3, 4])
    w = _pick(rng, [16, 32, 48, 64, 96, 160, 272])
    h = _pick(rng, [5, 9, 16, 23])
    x = p.input((1, h, w, ic), zp=int(rng.integers(1, -128, 127)[0]))
    k = _pick(rng, [1, 2, 3, 3, 4])
    stride = _pick(rng, [1, 2, 2])
    lut = _random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None
    lo = int(rng.integers(1, -24, -1)[0])
    for shift in ((lo, 3), (-12, -4), (-20, -1)):
        try:
            y = p.conv(x, _pick(rng, [16, 32, 48, 64]), k=k, stride=stride, padding=_pick(rng, ["same", (0, 0, 0, 0)]),
                       act=_pick(rng, ["none", "relu", "relu6"]), q6=int(rng.integers(1, 1, 200)[0]), lut=lut,
                       shift=shift, w_sigma=_pick(rng, [3, 40, 90]), tail_weights=bool(_pick(rng, [0, 1])))
            return p.build(y)
        except ValueError:
            continue
    raise AssertionError("unreachable")


def rows_conv_plan(seed):
    """A spatial conv on 16-channel multiples with OC a multiple of 16: the
    row-staged kernel with its register-direct epilogue, at four row blocks
    (up to 64 channels per slice) or two (96 and 128: six and eight channel
    tiles); widths whose rows do and do not fill a block."""
    rng = Rng(seed, 919191)
    p = Plan(seed)
    ic = _pick(rng, [16, 32])
    w = _pick(rng, [7, 14, 20, 28, 56, 60])
    x = p.input((1, _pick(rng, [4, 9, 14]), w, ic), zp=int(rng.integers(1, -128, 127)[0]))
    lo = int(rng.integers(1, -24, -1)[0])
    for shift in ((lo, 3), (-12, -4)):
        try:
            y = p.conv(x, _pick(rng, [16, 32, 64, 96, 128]), k=_pick(rng, [3, 3, 5]), stride=_pick(rng, [1, 2]),
                       act=_pick(rng, ["none", "relu"]), shift=shift, lut=_random_lut(p, rng) if _pick(rng, [0, 1]) else None,
                       w_sigma=_pick(rng, [3, 40, 90]), tail_weights=bool(_pick(rng, [0, 1])))
            return p.build(y)
        except ValueError:
            continue
    raise AssertionError("unreachable")


def gemm_plan(seed):
    """A conv the large-tile GEMM takes: pointwise over 256-960 channels (K
    not always a multiple of 64) or 3x3/5x5 over 64/128 channels (implicit
    im2col; strides, dilation, SAME and explicit padding), OC from 16 to 400
    in steps of 16 (tails against 128- and 256-channel tiles), pixel counts
    that are not multiples of the 256-pixel tile, post tables, activations
    and all requantisation ranges."""
    rng = Rng(seed, 565656)
    p = Plan(seed)
    pointwise = bool(_pick(rng, [0, 1]))
    if pointwise:
        ic = _pick(rng, [256, 272, 528, 960])
        h, w = _pick(rng, [(7, 7), (9, 13), (16, 16), (5, 37)])
        k, stride, dilation = 1, 1, 1
    else:
        ic = _pick(rng, [64, 128])
        h, w = _pick(rng, [(7, 7), (9, 13), (16, 16), (20, 11)])
        k, stride, dilation = _pick(rng, [3, 3, 5]), _pick(rng, [1, 2]), _pick(rng, [1, 1, 2])
    x = p.input((1, h, w, ic), zp=int(rng.integers(1, -128, 127)[0]))
    if pointwise or _pick(rng, [0, 1]):
        padding = "same"
    else:
        pt, pb = _geometry(rng, h, k, stride, dilation)
        pl, pr = _geometry(rng, w, k, stride, dilation)
        padding = (pt, pl, pb, pr)
    lut = _random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None
    lo = int(rng.integers(1, -24, -1)[0])
    for shift in ((lo, 3), (-12, -4), (-20, -1), (-24, -16)):
        try:
            y = p.conv(x, 16 * int(rng.integers(1, 1, 26)[0]), k=k, stride=stride, dilation=dilation, padding=padding,
                       act=_pick(rng, ["none", "relu", "relu6"]), q6=int(rng.integers(1, 1, 200)[0]), lut=lut,
                       shift=shift, w_sigma=_pick(rng, [3, 20, 40]), bias_sigma=_pick(rng, [0, 4096, 60000]))
            return p.build(y)
        except ValueError:
            continue
    raise AssertionError("unreachable")


def gemm_rows_plan(seed):
    """A conv the row-staged GEMM takes: 128 input channels, stride 1, no
    dilation, 3x3 / 5x5 / 1x3 / 3x1 kernels, SAME or explicit padding, up to
    128 output channels in steps of 16, maps from 3x3 to 80 columns (tiles
    of 512 pixels that start mid-row and end short of it), post tables,
    activations and all requantisation ranges."""
    rng = Rng(seed, 575757)
    p = Plan(seed)
    h, w = _pick(rng, [(3, 3), (7, 7), (9, 13), (20, 11), (24, 80), (33, 40), (5, 64)])
    x = p.input((1, h, w, 128), zp=int(rng.integers(1, -128, 127)[0]))
    kh, kw = _pick(rng, [(3, 3), (3, 3), (5, 5), (1, 3), (3, 1)])
    if _pick(rng, [0, 1]):
        padding = "same"
    else:
        pt, pb = _geometry(rng, h, kh, 1, 1)
        pl, pr = _geometry(rng, w, kw, 1, 1)
        padding = (pt, pl, pb, pr)
    lut = _random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None
    lo = int(rng.integers(1, -24, -1)[0])
    for shift in ((lo, 3), (-12, -4), (-20, -1), (-24, -16)):
        try:
            y = p.conv(x, 16 * int(rng.integers(1, 1, 8)[0]), k=kh, kw=kw, padding=padding,
                       act=_pick(rng, ["none", "relu", "relu6"]), q6=int(rng.integers(1, 1, 200)[0]), lut=lut,
                       shift=shift, w_sigma=_pick(rng, [3, 20, 40]), bias_sigma=_pick(rng, [0, 4096, 60000]))
            return p.build(y)
        except ValueError:
            continue
    raise AssertionError("unreachable")


def dw_band_plan(seed):
    """A depthwise layer for the band kernel: 3x3 or 5x5, stride 1 or 2, 16 to
    240 channels (channel slices of 1, 2, 3, 5, 6 or 15 groups of 16), maps
    from 3x3 to 112x112 (one band or many), SAME or explicit padding,
    optional post table, all requantisation ranges."""
    rng = Rng(seed, 737373)
    p = Plan(seed)
    c = _pick(rng, [16, 32, 48, 64, 80, 96, 240])
    hw = _pick(rng, [3, 5, 7, 14, 17, 28, 56, 112] if c <= 64 else [3, 7, 14, 28, 56])
    x = p.input((1, hw, hw, c), zp=int(rng.integers(1, -128, 127)[0]))
    k = _pick(rng, [3, 5])
    stride = _pick(rng, [1, 2])
    if _pick(rng, [0, 1]):
        padding = "same"
    else:
        pt, pb = _geometry(rng, hw, k, stride, 1)
        padding = (pt, pt, pb, pb)
    lut = _random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None
    lo = int(rng.integers(1, -24, -1)[0])
    for shift in ((lo, 3), (-12, -4), (-20, -1)):
        try:
            y = p.depthwise(x, k=k, stride=stride, padding=padding, act=_pick(rng, ["none", "relu", "relu6"]),
                            q6=int(rng.integers(1, 1, 200)[0]), lut=lut, shift=shift,
                            zero_mult=_pick(rng, [0.0, 0.3]), w_sigma=_pick(rng, [3, 40, 90]),
                            bias_sigma=_pick(rng, [0, 2048, 60000]))
            return p.build(y)
        except ValueError:
            continue
    raise AssertionError("unreachable")


def ib_plan(seed):
    """An inverted bottleneck of the shape the fused kernel takes (behind a
    post table, so that the block input is the library's own buffer): 1x1
    expand from 32 to 256 channels to up to 512, a 3x3 or 5x5 stride-1 SAME
    depthwise, 1x1 project, and a residual add with the block input (either
    operand order) when the channel counts match; maps from 1x1 to 28x28
    within the workgroup's LDS, post tables, activations and all
    requantisation ranges."""
    rng = Rng(seed, 515151)
    p = Plan(seed)
    while True:
        hw = int(_pick(rng, [1, 2, 3, 5, 7, 9, 14, 16, 20, 28]))
        cin = int(_pick(rng, [32, 64, 96, 128, 256]))
        ce = int(_pick(rng, [64, 96, 128, 192, 256, 384, 512]))
        ks = int(_pick(rng, [3, 5]))
        add = bool(_pick(rng, [0, 1, 1]))
        cout = cin if add else int(_pick(rng, [32, 64, 96, 128]))
        P = hw * hw
        lds = (P * (cin + 16) + ce * (hw + ks - 1) ** 2 + P * (ce + 16) + 64 * ce + 32 * cout + 2048 + 768 + 4 * P
               + 4 * ks * (2 if ks > 4 else 1) * ce)
        if lds <= 163840 and P * cout <= ce * (hw + ks - 1) ** 2:
            break
    x = p.input((1, hw, hw, cin), zp=int(rng.integers(1, -128, 127)[0]))
    x = p.lut(x, _random_lut(p, rng))

    def layer(make):
        lo = int(rng.integers(1, -24, -1)[0])
        for shift in ((lo, 3), (-12, -4), (-20, -1)):
            try:
                return make(shift)
            except ValueError:
                continue
        raise AssertionError("unreachable")

    def opts():
        return dict(act=_pick(rng, ["none", "relu", "relu6"]), q6=int(rng.integers(1, 1, 200)[0]),
                    lut=_random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None, w_sigma=_pick(rng, [3, 40, 90]))
    e = layer(lambda shift: p.conv(x, ce, k=1, shift=shift, **opts()))
    d = layer(lambda shift: p.depthwise(e, k=ks, stride=1, padding="same", shift=shift,
                                         bias_sigma=_pick(rng, [0, 2048, 60000]), **opts()))
    z = layer(lambda shift: p.conv(d, cout, k=1, shift=shift, **opts()))
    if add:
        z = p.add(x, z, act=_pick(rng, ["none", "relu", "relu6"])) if _pick(rng, [0, 1]) else \
            p.add(z, x, act=_pick(rng, ["none", "relu", "relu6"]))
    return p.build(z)


def uib_lds(H, W, Ho, Wo, cin, ce, cout, k0, k, s, add, R, rec_lds=1):
    """LDS bytes of the banded bottleneck kernel's workgroup for bands of R
    output rows (its layout: staged input, start-depthwise rows, window
    planes, depthwise rows, records, tables, position tables, tap words;
    rec_lds: the expand and depthwise records in LDS too), 0 when over 160
    KiB or when the output stage does not fit."""
    def up(v):
        return (v + 15) & ~15
    re = (R - 1) * s + k if k else R
    rv = min(re, H)
    pe, po = rv * W, R * Wo
    cols0, cols_p = W + k0 - 1, ((Wo - 1) * s + k if k else 0)
    o = up((cin // 16) * (rv + k0 - 1) * cols0 * 16 if k0 else pe * (cin + 16))
    x1 = o
    o += up(pe * (cin + 16) if k0 else 0)
    e = o
    o += up((ce // 16) * re * cols_p * 16 if k else 0)
    d = o
    o += up((po if k else pe) * (ce + 16)) + 64
    o += (cin * 32 if k0 else 0) + (ce * 32 if rec_lds else 0) + (ce * 32 if k and rec_lds else 0) + cout * 32
    o += (2048 if add else 0) + 1024
    o += up(pe * 4 if k0 else 0) + up(pe * 4 if k else 0) + up(po * 4 if k else 0) + up(po * 4 if add else 0)
    o += up(k0 * (2 if k0 > 4 else 1) * cin * 4) + up(k * (2 if k > 4 else 1) * ce * 4)
    if po * cout > ((d - e) if k else (e - x1)):
        return 0
    return o if o <= 163840 else 0


def dw_window_form(c, oh, ow, k, s):
    """Whether the library keeps a depthwise layer in window form (tap words
    [ky][k > 4 ? 2 : 1][C], the form the fused kernels read): the dot4
    window kernel's plan must fit its 64 KiB of LDS."""
    if c % 4 or k not in (3, 5) or s not in (1, 2):
        return False
    c4, cq = c // 4, 1
    while cq < 16 and c4 % (2 * cq) == 0:
        cq *= 2
    xq_all = (ow + 3) // 4
    tiles_x = (xq_all + 7) // 8
    xw = (xq_all + tiles_x - 1) // tiles_x
    if xw >= 4 and cq > 4:
        cq = 4
    th = 256 // (xw * cq)
    if th < 1:
        return False
    ir = (min(th, oh) - 1) * s + k
    njq = (4 * xw + (4 // s if k > 4 else 0) + 3) // 4
    if ir * njq >= 65536 // njq:
        return False
    return ir * njq * cq * 5 * 16 + k * (2 if k > 4 else 1) * cq * 16 + cq * 4 * 32 + 256 <= 65536


def uib_rows(H, W, Ho, Wo, cin, ce, cout, k0, k, s, add):
    """(R, rec_lds): the output rows per band the banded bottleneck kernel
    takes, the most whose workgroup fits, with the expand and depthwise
    records in LDS when they fit too ((0, 0): nothing fits)."""
    for R in range(Ho, 0, -1):
        for rec_lds in (1, 0):
            if uib_lds(H, W, Ho, Wo, cin, ce, cout, k0, k, s, add, R, rec_lds):
                return R, rec_lds
    return 0, 0


def uib_plan(seed):
    """uib_block's plan."""
    return uib_block(seed)[0]


def uib_block(seed):
    """(plan, rows, out_rows): a universal inverted bottleneck of the shapes the banded fused kernel
    takes (behind a post table, so that the block input is the library's own
    buffer): a 3x3 or 5x5 stride-1 start depthwise (SAME, or explicit pads
    that keep the map), 1x1 expand, a 3x3 or 5x5 depthwise of stride 1 or 2
    (SAME or explicit pads), 1x1 project, and a residual add with the block
    input (either operand order) at stride 1 when the channel counts match;
    blocks without the start depthwise (then at stride 2) or without the
    second one; non-square maps from 3 to 30 rows, one band to many, post
    tables, activations and all requantisation ranges. Both depthwise layers
    in window form (dw_window_form), which the fused kernels need. rows: the
    output rows per band the kernel takes (uib_rows); out_rows: the block's
    output rows."""
    rng = Rng(seed, 626262)
    p = Plan(seed)

    def pads(k):
        if _pick(rng, [0, 1]):
            return "same"
        pt, pl = int(rng.integers(1, 0, k - 1)[0]), int(rng.integers(1, 0, k - 1)[0])
        return (pt, pl, k - 1 - pt, k - 1 - pl)

    while True:
        form = _pick(rng, ["both", "both", "start", "mid"])
        h, w = int(_pick(rng, [3, 5, 7, 9, 14, 17, 28, 30])), int(_pick(rng, [3, 5, 7, 14, 16, 28]))
        cin = int(_pick(rng, [32, 64, 96, 128]))
        ce = int(_pick(rng, [64, 96, 128, 192, 256, 384, 512]))
        k0 = int(_pick(rng, [3, 5])) if form != "mid" else 0
        k = int(_pick(rng, [3, 5])) if form != "start" else 0
        s = 2 if form == "mid" else (int(_pick(rng, [1, 2])) if k else 1)
        add = s == 1 and bool(_pick(rng, [0, 1, 1]))
        cout = cin if add else int(_pick(rng, [32, 64, 96, 128]))
        pad0 = pads(k0) if k0 else None
        pad = (pads(k) if s == 1 else _pick(rng, ["same", (0, 0, 0, 0), (1, 1, 1, 1)])) if k else None
        if k:
            if pad == "same":
                ho, wo = -(-h // s), -(-w // s)
            else:
                ho, wo = (h + pad[0] + pad[2] - k) // s + 1, (w + pad[1] + pad[3] - k) // s + 1
            if ho < 1 or wo < 1 or (s == 1 and (ho, wo) != (h, w)):
                continue
        else:
            ho, wo = h, w
        if (k0 and not dw_window_form(cin, h, w, k0, 1)) or (k and not dw_window_form(ce, ho, wo, k, s)):
            continue
        rows = uib_rows(h, w, ho, wo, cin, ce, cout, k0, k, s, add)[0]
        if rows:
            break
    x = p.input((1, h, w, cin), zp=int(rng.integers(1, -128, 127)[0]))
    x = p.lut(x, _random_lut(p, rng))

    def layer(make):
        lo = int(rng.integers(1, -24, -1)[0])
        for shift in ((lo, 3), (-12, -4), (-20, -1)):
            try:
                return make(shift)
            except ValueError:
                continue
        raise AssertionError("unreachable")

    def opts():
        return dict(act=_pick(rng, ["none", "relu", "relu6"]), q6=int(rng.integers(1, 1, 200)[0]),
                    lut=_random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None, w_sigma=_pick(rng, [3, 40, 90]))
    y = x
    if k0:
        y = layer(lambda shift: p.depthwise(y, k=k0, stride=1, padding=pad0, shift=shift,
                                             bias_sigma=_pick(rng, [0, 2048, 60000]), **opts()))
    e = layer(lambda shift: p.conv(y, ce, k=1, shift=shift, **opts()))
    if k:
        e = layer(lambda shift: p.depthwise(e, k=k, stride=s, padding=pad, shift=shift,
                                             bias_sigma=_pick(rng, [0, 2048, 60000]), **opts()))
    z = layer(lambda shift: p.conv(e, cout, k=1, shift=shift, **opts()))
    if add:
        z = p.add(x, z, act=_pick(rng, ["none", "relu", "relu6"])) if _pick(rng, [0, 1]) else \
            p.add(z, x, act=_pick(rng, ["none", "relu", "relu6"]))
    return p.build(z), rows, ho


def stem_conv_plan(seed):
    """A stem conv (IC 1-4, 32 output channels) followed by a 3x3 stride-2
    conv over its output, the pair the fused stem kernel takes: SAME or
    explicit padding on both, strides 1-2 on the stem, widths from 16 to 96
    input columns, odd heights, post tables, all requantisation ranges, and
    sometimes a post-table op and/or a 1x1 32 -> 32 conv after the pair."""
    rng = Rng(seed, 929292)
    p = Plan(seed)
    ic = _pick(rng, [1, 2, 3, 3, 4])
    w = _pick(rng, [16, 32, 48, 64, 96])
    h = _pick(rng, [7, 9, 16, 23, 30])
    x = p.input((1, h, w, ic), zp=int(rng.integers(1, -128, 127)[0]))
    k = _pick(rng, [2, 3, 3, 4]) if ic < 4 else _pick(rng, [2, 3, 4])
    stride = _pick(rng, [1, 2, 2])
    lo = int(rng.integers(1, -24, -1)[0])

    def layer(make):
        for shift in ((lo, 3), (-12, -4), (-20, -1)):
            try:
                return make(shift)
            except ValueError:
                continue
        raise AssertionError("unreachable")

    def opts():
        return dict(act=_pick(rng, ["none", "relu", "relu6"]), q6=int(rng.integers(1, 1, 200)[0]),
                    lut=_random_lut(p, rng) if _pick(rng, [0, 0, 1]) else None, w_sigma=_pick(rng, [3, 40, 90]))
    s = layer(lambda shift: p.conv(x, 32, k=k, stride=stride, padding=_pick(rng, ["same", (0, 0, 0, 0)]),
                                   shift=shift, **opts()))
    _, sh, sw, _ = p.shape(s)
    if _pick(rng, [0, 1]) and sh >= 3 and sw >= 3:
        padding = "same"
    else:
        pt, pb = _geometry(rng, sh, 3, 2, 1)
        pl, pr = _geometry(rng, sw, 3, 2, 1)
        padding = (pt, pl, pb, pr)
    z = layer(lambda shift: p.conv(s, 32, k=3, stride=2, padding=padding, shift=shift, **opts()))
    if _pick(rng, [0, 1]):
        z = p.lut(z, _random_lut(p, rng))
    # A 1x1 32 -> 32 conv after the pair: fused with it when it reads the
    # 3x3's output directly, a separate launch after a post-table op.
    if _pick(rng, [0, 1, 1]):
        z = layer(lambda shift: p.conv(z, 32, k=1, shift=shift, **opts()))
    return p.build(z)
