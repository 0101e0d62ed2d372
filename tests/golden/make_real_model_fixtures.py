"""Copy the reference's shipped MobileNetV4-small bundle
(models/mobilenetv4-small.uqmodel, Apache-2.0, from
timm/mobilenetv4_conv_small.e2400_r224_in1k per models/provenance.json) into
tests/golden/ and score seeded inputs with the reference's own C runtime
(oracle/_ref/libuq_ref_release.so, built from runtime/*.c), writing
tests/golden/mobilenetv4_small_expected.npz (input, output).

The YOLO26n-320 bundle is AGPL-3.0 and stays out of this repository; its
end-to-end parity runs where the reference tree is present.

Runs only where the reference tree and its C build are present:
    python tests/golden/make_real_model_fixtures.py
"""
import ctypes as C
import hashlib
import json
import shutil
import struct
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "unoq-dsp_amd"))
from uq_plan import Rng  # noqa: E402

MODELS = Path("/root/reference/models")
REF = ROOT / "oracle" / "_ref" / "libuq_ref_release.so"
HERE = Path(__file__).resolve().parent
NAME = "mobilenetv4-small.uqmodel"
IMAGES = 4


def main():
    src = MODELS / NAME
    data = src.read_bytes()
    want = {e["file"]: e["sha256"] for e in json.loads((MODELS / "provenance.json").read_text())}[NAME]
    assert hashlib.sha256(data).hexdigest() == want, "bundle does not match its provenance record"
    shutil.copyfile(src, HERE / NAME)
    nm = struct.unpack_from("<I", data, 12)[0]
    plan = data[52 + nm:]
    lib = C.CDLL(str(REF))
    lib.ug_load.argtypes = [C.c_void_p, C.c_uint32]
    lib.ug_run.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32]
    lib.ug_input_bytes.restype = lib.ug_output_bytes.restype = C.c_uint32
    buf = C.create_string_buffer(plan, len(plan))
    assert lib.ug_load(buf, len(plan)) == 0
    ib, ob = lib.ug_input_bytes(), lib.ug_output_bytes()
    # Two noise images, a smooth colour ramp and high-contrast stripes.
    x = Rng(4242, 1).int8(IMAGES * ib)
    hh = ww = 224
    yy, xx = np.mgrid[0:hh, 0:ww]
    ramp = np.stack([xx * 255 // (ww - 1), yy * 255 // (hh - 1), (xx + yy) * 255 // (hh + ww - 2)], -1) - 128
    stripes = np.where(((xx // 14) + (yy // 28)) % 2 == 0, 100, -100)[..., None].repeat(3, -1)
    x[2 * ib:3 * ib] = ramp.astype(np.int8).reshape(-1)
    x[3 * ib:4 * ib] = stripes.astype(np.int8).reshape(-1)
    y = np.empty(IMAGES * ob, np.int8)
    for j in range(IMAGES):
        assert lib.ug_run(x[j * ib:].ctypes.data, ib, y[j * ob:].ctypes.data, ob) == 0
    np.savez_compressed(HERE / "mobilenetv4_small_expected.npz", input=x, output=y)
    print(f"{NAME}: input {ib} B/img, output {ob} B/img, {IMAGES} images, "
          f"top-1 per image {[int(np.argmax(y[j * ob:(j + 1) * ob])) for j in range(IMAGES)]}")


if __name__ == "__main__":
    main()
