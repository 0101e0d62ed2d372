"""The .uqmodel reader of libuq_hip.so (ug_bundle_plan / ug_load_bundle /
uq_sha256) against the reference's Python container format
(src/unoq_dsp/bundle.py:18-19 header, :66-81 writer, :84-141 loader).

SHA-256 is checked against hashlib (FIPS 180-4 test vectors included). Bundles
are written here exactly as CompiledModel.save writes them (header <8sIII32s>,
manifest, plan, digest of manifest || plan), then corrupted the ways load()
rejects: magic, version, manifest/plan length bounds, truncation or trailing
bytes, checksum, plan magic and plan version. The reference's two shipped
bundles are parsed too where the reference tree is present."""
import ctypes as C
import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest

import uq_workloads as W
from uq_native import open_library

MODELS = Path("/root/reference/models")
HEADER = struct.Struct("<8sIII32s")


@pytest.fixture(scope="module")
def lib():
    return open_library()


def _sha(lib, data):
    out = C.create_string_buffer(32)
    buf = C.create_string_buffer(bytes(data), max(len(data), 1))
    lib.uq_sha256(buf, len(data), out)
    return out.raw


def _bundle(plan, manifest=None, version=1, digest=None, nm=None, np_=None):
    manifest = manifest if manifest is not None else json.dumps({"task": "test"}).encode()
    digest = digest if digest is not None else hashlib.sha256(manifest + plan).digest()
    return HEADER.pack(b"UQMODEL\0", version, len(manifest) if nm is None else nm,
                       len(plan) if np_ is None else np_, digest) + manifest + plan


def _parse(lib, blob):
    buf = C.create_string_buffer(bytes(blob), max(len(blob), 1))
    ptr, n = C.c_void_p(), C.c_uint32()
    rc = lib.ug_bundle_plan(buf, len(blob), C.byref(ptr), C.byref(n))
    if rc:
        return rc, None
    return 0, C.string_at(ptr.value, n.value)


def test_sha256_known_answers(lib):
    # FIPS 180-4 examples (one block, two blocks) and the empty string.
    assert _sha(lib, b"abc").hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert _sha(lib, b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq").hex() == \
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"
    assert _sha(lib, b"").hex() == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"


@pytest.mark.parametrize("n", [1, 55, 56, 63, 64, 65, 119, 120, 127, 128, 1000, 1 << 20])
def test_sha256_matches_hashlib(lib, n):
    data = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    assert _sha(lib, data) == hashlib.sha256(data).digest()


def test_bundle_round_trip(lib):
    plan, _ = W.pointwise()
    rc, got = _parse(lib, _bundle(plan))
    assert rc == 0 and got == plan


def test_bundle_accepts_version3_plan(lib):
    plan, _ = W.pointwise()
    p3 = bytearray(plan)
    struct.pack_into("<I", p3, 4, 3)
    rc, got = _parse(lib, _bundle(bytes(p3)))
    assert rc == 0 and got == bytes(p3)


def test_bundle_header_errors(lib):
    plan, _ = W.pointwise()
    good = _bundle(plan)
    assert _parse(lib, good[:51])[0] == 30                       # truncated header
    assert _parse(lib, b"UQMODEL\1" + good[8:])[0] == 30          # magic
    assert _parse(lib, _bundle(plan, version=2))[0] == 30         # container version
    assert _parse(lib, _bundle(plan, manifest=b""))[0] == 30      # empty manifest
    assert _parse(lib, _bundle(plan, nm=4 * 1024 * 1024 + 1))[0] == 30
    assert _parse(lib, _bundle(plan[:31] if len(plan) > 31 else plan, np_=31))[0] == 30
    assert _parse(lib, _bundle(plan, np_=17 * 1024 * 1024 + 1))[0] == 30
    assert _parse(lib, good[:-1])[0] == 30                        # truncated payload
    assert _parse(lib, good + b"\0")[0] == 30                     # trailing byte


def test_bundle_checksum_errors(lib):
    plan, _ = W.pointwise()
    good = bytearray(_bundle(plan))
    bad = bytearray(good)
    bad[20] ^= 1                                                  # digest bit
    assert _parse(lib, bad)[0] == 31
    for pos in (52, len(good) // 2, len(good) - 1):               # manifest / plan / last byte
        bad = bytearray(good)
        bad[pos] ^= 0x40
        assert _parse(lib, bad)[0] == 31


def test_bundle_plan_header_errors(lib):
    plan, _ = W.pointwise()
    for version in (1, 4):
        p = bytearray(plan)
        struct.pack_into("<I", p, 4, version)
        assert _parse(lib, _bundle(bytes(p)))[0] == 32
    p = bytearray(plan)
    p[0] ^= 1
    assert _parse(lib, _bundle(bytes(p)))[0] == 32


def test_load_bundle_passes_plan_to_loader(lib):
    plan, _ = W.pointwise()
    blob = _bundle(plan)
    buf = C.create_string_buffer(blob, len(blob))
    rc = lib.ug_load_bundle(buf, len(blob))
    assert rc in (0, 24)
    # A plan the loader rejects keeps the loader's code (bad tensor record: 13).
    p = bytearray(plan)
    struct.pack_into("<I", p, 32 + 12, 7)                         # tensor 0 rank 7
    blob = _bundle(bytes(p))
    buf = C.create_string_buffer(blob, len(blob))
    assert lib.ug_load_bundle(buf, len(blob)) == 13


@pytest.mark.parametrize("name", ["mobilenetv4-small.uqmodel", "yolo26n-320.uqmodel"])
def test_reference_bundles(lib, name):
    path = MODELS / name
    if not path.exists():
        pytest.skip("reference models not present")
    data = path.read_bytes()
    magic, version, nm, np_, digest = HEADER.unpack_from(data)
    rc, plan = _parse(lib, data)
    assert rc == 0 and plan == data[52 + nm:]
    manifest = json.loads(data[52:52 + nm])
    nt, no = struct.unpack_from("<II", plan, 8)
    assert manifest["plan_bytes"] == len(plan)
    buf = C.create_string_buffer(data, len(data))
    rc = lib.ug_load_bundle(buf, len(data))
    assert (nt, no) == ((166, 60) if name.startswith("mobilenet") else (577, 234))
    assert rc in (0, 24)
