"""The C-ABI library loads without a GPU, exports every function declared in
include/uq_graph.h, and answers the not-loaded cases of the reference ABI
(graph.c:263-286: zero sizes, 22 for runs, snapshots and profiles)."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import numpy as np

from uq_native import DEFAULT_LIBRARY, SIGNATURES, open_library

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "uq_graph.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b((?:ug|uq)_\w+)\s*\(", text))


def test_header_and_binding_agree():
    assert declared_functions() == {name for name, _, _ in SIGNATURES}


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(DEFAULT_LIBRARY)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T ((?:ug|uq)_\w+)", out))
    missing = declared_functions() - exported
    assert not missing, missing


def test_not_loaded_behaviour():
    lib = open_library()
    # Loading an invalid blob leaves nothing loaded (ready = 0 on entry).
    assert lib.ug_load(C.create_string_buffer(b"\0" * 64), 64) == 11
    assert lib.ug_input_bytes() == 0 and lib.ug_output_bytes() == 0 and lib.ug_op_count() == 0
    x = np.zeros(16, np.int8)
    assert lib.ug_run(x.ctypes.data, 16, x.ctypes.data, 16) == 22
    assert lib.ug_run_batch(x.ctypes.data, 16, x.ctypes.data, 16, 1) == 22
    assert lib.ug_snapshot(0, x.ctypes.data, 16) == 22
    counters = np.zeros(514, np.uint64)
    assert lib.ug_profile(2, counters.ctypes.data, counters.nbytes) == 22
    assert lib.ug_stream_begin() == 22
    assert lib.ug_stream_end() == 0
