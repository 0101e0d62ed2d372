"""Host-side planning of the banded bottleneck kernel (plain C in the library,
callable without a GPU): for random block shapes, the output rows per band
and the workgroup's LDS bytes that uqk_uib_plan picks agree with the layout
restated in plan_fuzz.uib_lds, which the fuzz plans of the GPU tests are
drawn from, and shapes outside the kernel are refused."""
import ctypes as C

import numpy as np

from plan_fuzz import uib_lds, uib_rows
from uq_native import open_library

_I, _P = C.c_int32, C.c_void_p


class UQKUib(C.Structure):
    _fields_ = ([(n, _I) for n in "H W Ho Wo Cin Ce Cout k0 p0t p0l".split()]
                + [(n, _P) for n in "dw0 epi0 lut0".split()]
                + [(n, _I) for n in "m0 yz0 lo0 hi0 xz0".split()]
                + [(n, _P) for n in "we epi_e lut_e".split()]
                + [(n, _I) for n in "kpe e_mode e_yz e_lo e_hi k s pt pl".split()]
                + [(n, _P) for n in "dww epi_d lut_d".split()]
                + [(n, _I) for n in "d_mode d_yz d_lo d_hi d_xz".split()]
                + [(n, _P) for n in "wp epi_p lut_p".split()]
                + [(n, _I) for n in "kpp p_mode p_yz p_lo p_hi has_add add_x_first".split()]
                + [("add_tab", _P)]
                + [(n, _I) for n in "a_m a_s a_yz a_lo a_hi R rec_lds".split()])


def _plan(lib, **kw):
    u = UQKUib(**kw)
    lds = lib.uqk_uib_plan(C.byref(u))
    return lds, u.R, u.rec_lds


def test_uib_plan_matches_layout():
    lib = open_library()
    lib.uqk_uib_plan.restype = C.c_size_t
    rng = np.random.default_rng(5)
    checked = fused = global_records = 0
    for _ in range(3000):
        k0 = int(rng.choice([0, 3, 5]))
        k = int(rng.choice([3, 5])) if k0 == 0 else int(rng.choice([0, 3, 5]))
        s = 2 if k0 == 0 else (int(rng.choice([1, 2])) if k else 1)
        H, W = (int(v) for v in rng.integers(1, 40, 2))
        cin, ce, cout = (32 * int(v) for v in (rng.integers(1, 9), rng.integers(1, 17), rng.integers(1, 9)))
        p0t, p0l = (k0 - 1) // 2, (k0 - 1) // 2
        pt, pl = ((k - 1) // 2, (k - 1) // 2) if k else (0, 0)
        Ho, Wo = ((H + 2 * pt - k) // s + 1, (W + 2 * pl - k) // s + 1) if k else (H, W)
        if Ho < 1 or Wo < 1:
            continue
        add = int(s == 1 and cin == cout and rng.integers(0, 2) == 1)
        lds, R, rec_lds = _plan(lib, H=H, W=W, Ho=Ho, Wo=Wo, Cin=cin, Ce=ce, Cout=cout, k0=k0, p0t=p0t, p0l=p0l,
                                k=k, s=s, pt=pt, pl=pl, has_add=add)
        want = uib_rows(H, W, Ho, Wo, cin, ce, cout, k0, k, s, add)
        assert (R, rec_lds) == want, (H, W, cin, ce, cout, k0, k, s, add)
        assert lds == (uib_lds(H, W, Ho, Wo, cin, ce, cout, k0, k, s, add, R, rec_lds) if R else 0)
        checked += 1
        fused += R > 0
        global_records += R > 0 and not rec_lds
    assert checked > 2000 and 0 < fused < checked and global_records > 0


def test_uib_plan_refuses_outside_shapes():
    lib = open_library()
    lib.uqk_uib_plan.restype = C.c_size_t
    base = dict(H=14, W=14, Ho=14, Wo=14, Cin=96, Ce=384, Cout=96, k0=3, p0t=1, p0l=1, k=0, s=1, has_add=1)
    assert _plan(lib, **base)[0] > 0
    # MobileNetV4's 7x7 ExtraDW block (5x5 start and middle depthwise, 128 ->
    # 512 -> 128 with the add) fits one band with its records read from L2.
    assert _plan(lib, H=7, W=7, Ho=7, Wo=7, Cin=128, Ce=512, Cout=128, k0=5, p0t=2, p0l=2, k=5, s=1, pt=2, pl=2,
                 has_add=1)[1:] == (7, 0)
    for change in (dict(k0=0),                       # neither depthwise
                   dict(Cin=80), dict(Ce=528), dict(Cout=48),   # channel counts
                   dict(Ce=544),                     # Ce > 512
                   dict(k0=7), dict(p0t=3),          # start depthwise kernel and pads
                   dict(Cout=64),                    # an add needs Cin == Cout
                   dict(Ho=7, Wo=7)):                # without a depthwise the map keeps its size
        assert _plan(lib, **dict(base, **change))[:2] == (0, 0), change
    # An add after a stride-2 depthwise is refused.
    assert _plan(lib, **dict(base, k=3, s=2, pt=0, pl=0, Ho=7, Wo=7, Cout=96))[:2] == (0, 0)
