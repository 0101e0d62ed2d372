"""ug_load of libuq_hip.so returns the reference loader's error code
(graph.c:50-216, qnn.c:209-252) for every malformed plan: random mutations of
headers, tensor records, op records, parameter blocks and weights, plus
version-3 lifetime overlaps. Validation runs on the host before any GPU work,
so this test needs no GPU: a plan the reference accepts gets 0 on a GPU host,
24 where no GPU is present, and 19 when it uses ops outside the INT8 path
that the reference runtime also implements (float ops and float / u8 x i8
matmuls, codes 1-4 and 6-9, 11-13).

The reference side is the plain build (no macros); the release build's load
path adds its own preparation steps and is compared on the unmutated plans.
"""
import struct

import numpy as np
import pytest

import uq_plan as P
import uq_workloads as W
from plan_fuzz import ATTENTION_OPS, random_plan
from refs import ref_plain, ref_release
from uq_native import open_library

SUPPORTED = {5, 10, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28}


@pytest.fixture(scope="module")
def libs():
    import ctypes as C
    prod = open_library()
    ref = ref_plain()
    return prod, ref, C


def _load(lib, C, blob):
    buf = C.create_string_buffer(bytes(blob), max(len(blob), 1))
    return lib.ug_load(buf, len(blob))


def _codes(plan):
    nt, no = struct.unpack_from("<II", plan, 8)
    if len(plan) < 32 + 48 * nt + 32 * no:
        return set()
    return {struct.unpack_from("<I", plan, 32 + 48 * nt + 32 * i)[0] for i in range(no)}


def _check(libs, blob):
    prod, ref, C = libs
    want = _load(ref.lib, C, blob)
    got = _load(prod, C, blob)
    if want:
        assert got == want, f"reference {want}, product {got}"
    else:
        allowed = {0, 24} if _codes(blob) <= SUPPORTED else {19}
        assert got in allowed, f"reference accepts; product {got}"
    return want


def _mutate(plan, rng):
    b = bytearray(plan)
    nt, no = struct.unpack_from("<II", b, 8)
    meta = 32 + 48 * nt + 32 * no
    kind = rng.integers(0, 7)
    if kind == 0:                                    # header word
        i = int(rng.integers(0, 8))
        struct.pack_into("<I", b, 4 * i, int(rng.choice([0, 1, 2, 3, 4, nt, nt + 1, no + 1, 1 << 24, 0xFFFFFFFF,
                                                          int(rng.integers(0, 1 << 32))])))
    elif kind == 1:                                  # tensor record word
        t = int(rng.integers(0, nt))
        i = int(rng.integers(0, 12))
        old = struct.unpack_from("<I", b, 32 + 48 * t + 4 * i)[0]
        struct.pack_into("<I", b, 32 + 48 * t + 4 * i,
                         int(rng.choice([0, 1, 2, 5, old + 1, old - 1 if old else 7, old + 128, old * 2, 0xFFFFFFFF])) & 0xFFFFFFFF)
    elif kind == 2:                                  # op record word
        o = int(rng.integers(0, no))
        i = int(rng.integers(0, 8))
        old = struct.unpack_from("<I", b, 32 + 48 * nt + 32 * o + 4 * i)[0]
        struct.pack_into("<I", b, 32 + 48 * nt + 32 * o + 4 * i,
                         int(rng.choice([0, 1, 2, 3, 6, 9, 13, 17, 19, 25, 27, 28, 29, old + 1, nt, 0xFFFFFFFF,
                                         int(rng.integers(0, nt))])) & 0xFFFFFFFF)
    elif kind == 3:                                  # int32 inside a constant (q blocks, tables)
        recs = [struct.unpack_from("<12I", b, 32 + 48 * t) for t in range(nt)]
        consts = [r for r in recs if r[8] and r[2] == 4 and r[1] >= 4]
        if consts:
            r = consts[int(rng.integers(0, len(consts)))]
            j = int(rng.integers(0, min(r[1] // 4, 40)))
            old = struct.unpack_from("<i", b, meta + r[0] + 4 * j)[0]
            struct.pack_into("<i", b, meta + r[0] + 4 * j,
                             int(rng.choice([0, -1, 1, old + 1, old - 1, 16, 200, 5000, -200, 2 ** 31 - 1, -2 ** 31])))
    elif kind == 4:                                  # weight bytes at full scale (breaks bound proofs)
        recs = [struct.unpack_from("<12I", b, 32 + 48 * t) for t in range(nt)]
        consts = [r for r in recs if r[8] and r[2] == 3]
        if consts:
            r = consts[int(rng.integers(0, len(consts)))]
            n = min(r[1], 4096)
            b[meta + r[0]: meta + r[0] + n] = bytes([127] * n)
    elif kind == 5:                                  # length
        return bytes(b[:int(rng.integers(0, len(b)))]) if rng.integers(0, 2) else bytes(b) + b"\0" * int(rng.integers(1, 200))
    else:                                            # version 3 (enables the lifetime-overlap proof)
        struct.pack_into("<I", b, 4, 3)
    return bytes(b)


def _corpus():
    plans = [W.pointwise()[0], W.depthwise("dw5s2")[0]]
    plans += [random_plan(5000 + i) for i in range(24)]
    return plans


CORPUS = None


def _plans():
    global CORPUS
    if CORPUS is None:
        CORPUS = _corpus()
    return CORPUS


def test_unmutated_plans_accepted(libs):
    rel = ref_release()
    for plan in _plans():
        assert _check(libs, plan) == 0
        assert rel.load(plan) == 0


@pytest.mark.parametrize("seed", range(12))
def test_mutated_plans_same_code(libs, seed):
    rng = np.random.default_rng(seed)
    seen = set()
    for plan in _plans():
        for _ in range(25):
            seen.add(_check(libs, _mutate(plan, rng)))
    assert len(seen) >= 3, f"mutations exercised too few codes: {seen}"


def test_short_and_missing_blobs(libs):
    prod, ref, C = libs
    assert prod.ug_load(None, 0) == 10
    for n in (0, 8, 31):
        _check(libs, b"\0" * n)


def test_v3_lifetime_overlap(libs):
    """Two live activations sharing arena bytes: 25; after the first dies: 0."""
    p = P.Plan(4)
    x = p.input((1, 4, 4, 16), zp=0)
    a = p.lut(x, p.lut_table(np.arange(256)))
    b2 = p.lut(a, p.lut_table(np.arange(256)))
    c = p.lut(b2, p.lut_table(np.arange(256)))
    plan = bytearray(p.build(c, version=3))
    recs = P.tensor_records(bytes(plan))
    # alias b2 onto a (both live at op 1): overlap while live
    bad = bytearray(plan)
    struct.pack_into("<I", bad, 32 + 48 * b2, recs[a][0])
    assert _check(libs, bytes(bad)) == 25
    # alias c onto a (a dies at op 1, c is born at op 2): legal reuse
    ok = bytearray(plan)
    struct.pack_into("<I", ok, 32 + 48 * c, recs[a][0])
    assert _check(libs, bytes(ok)) == 0


def test_out_of_scope_ops_rejected_with_19(libs):
    """A plan the reference accepts but that holds a float op (code 4, ReLU on
    int32 here) is refused by the GPU library with 19."""
    p = P.Plan(6)
    x = p.input((4,), zp=0)
    p.tensors[x]["type"] = P.TYPE_I32
    p.tensors[x]["bytes"] = 16
    p.arena.extend(bytes(16))
    z = p.tensor((4,), P.TYPE_I32)
    p._op(4, x, x, z)
    plan = p.build(z)
    prod, ref, C = libs
    assert _load(ref.lib, C, plan) == 0
    assert _load(prod, C, plan) == 19


F32 = 1


def _f32(p, shape, const=False):
    t = p.tensor(shape, P.TYPE_I32, np.zeros(int(np.prod(shape)), np.int32) if const else None)
    p.tensors[t]["type"] = F32
    return t


def _refused_plan(code):
    """A minimal plan holding op `code` that the reference loader accepts
    (graph.c:74-104 for codes 1-13)."""
    p = P.Plan(7)
    if code in (1, 8):                       # float matmul, plain and packed
        x = _f32(p, (2, 3))
        b = _f32(p, (4, 3), const=True)
        z = _f32(p, (2, 4))
    elif code in (6, 9):                     # u8 x i8 matmul with correction, plain and packed
        x = p.tensor((2, 8), P.TYPE_U8)
        b = p.tensor((4, 8), P.TYPE_I8, np.zeros(32, np.int8))
        corr = p.tensor((4,), P.TYPE_I32, np.zeros(4, np.int32))
        z = p.tensor((2, 4), P.TYPE_I32)
    elif code in (2, 3, 4, 13):              # float elementwise, ReLU, softmax
        x = _f32(p, (2, 4))
        b = x
        z = _f32(p, (2, 4))
    elif code == 7:                          # int32 -> float cast
        x = p.tensor((4,), P.TYPE_I32)
        b = x
        z = _f32(p, (4,))
    else:                                    # 11 float im2col, 12 float max pool: 1x1 windows
        x = _f32(p, (1, 4, 4, 1))
        b = p.tensor((12,), P.TYPE_I32, np.array([1, 1, 1, 1, 1, 1, 0, 0, 0, 0, 4, 4], np.int32))
        z = _f32(p, (16, 1)) if code == 11 else _f32(p, (1, 4, 4, 1))
    p.input_id = x
    p.zp[x] = 0
    p._op(code, x, b, z, (3, -2, corr, 1) if code in (6, 9) else (0, 0, 0, 0))
    return p.build(z)


def _header_code_sets():
    """The op codes include/uq_graph.h calls refused (19) and loaded."""
    import re
    from pathlib import Path
    text = (Path(__file__).resolve().parents[1] / "include" / "uq_graph.h").read_text()
    text = " ".join(re.sub(r"\n\s*\*(?!/)", " ", text).split())

    def expand(spec):
        out = set()
        for part in spec.split(","):
            part = part.strip()
            if "-" in part:
                lo, hi = part.split("-")
                out |= set(range(int(lo), int(hi) + 1))
            elif part:
                out.add(int(part))
        return out
    refused = re.search(r"float ops \(codes ([0-9, -]+)\) and the u8 x i8 integer matmuls \(([0-9, ]+)\)", text)
    loaded = re.search(r"loads and runs here: ([0-9, -]+) \(", text)
    assert refused and loaded, "header no longer states the op-code sets"
    return expand(refused.group(1)) | expand(refused.group(2)), expand(loaded.group(1))


def test_header_op_code_sets_match_library(libs):
    """Every code the boundary header calls refused gets 19 on a plan the
    reference accepts; every code it calls loaded is the library's set, and
    the two cover the reference's op codes 1-28."""
    refused, loaded = _header_code_sets()
    assert refused | loaded == set(range(1, 29)) and not refused & loaded
    assert loaded == SUPPORTED
    prod, ref, C = libs
    for code in sorted(refused):
        plan = _refused_plan(code)
        assert _load(ref.lib, C, plan) == 0, f"code {code}: the reference refuses the test plan"
        assert _load(prod, C, plan) == 19, f"code {code}"
    # Loaded codes: every one appears in an accepted corpus plan the library
    # takes (0 with a GPU, 24 without one), never 19.
    seen = set()
    for plan in _plans() + [W.yolo()[0]] + [random_plan(7000 + i, ops=ATTENTION_OPS) for i in range(8)]:
        seen |= _codes(plan)
        assert _load(prod, C, plan) in (0, 24)
    assert loaded <= seen, loaded - seen
