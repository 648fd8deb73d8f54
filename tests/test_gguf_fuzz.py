"""Host AddressSanitizer + UBSan fuzz of the GGUF reader (csrc/gguf.cpp), CPU
only.  `make fuzz-gguf` builds the reader for the host with both sanitizers
and tests/native/gguf_fuzz.c mutates a valid file (truncation, bit flips) and
walks every accessor of each file the reader accepts; any out-of-bounds read,
leak or undefined behaviour ends the run with a sanitizer report.  The file
holds every GGUF KV type (src/gguf.js:7-21), nested and empty arrays, and two
MoE blocks, so mutations reach each branch of the parser (src/gguf.js:37-94)."""
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import synth  # noqa: E402

HIPCC = "/opt/rocm/bin/hipcc"


def _fuzz_file(path):
    layers = [synth.moe_layer(s, H=64, F=32, E=4, K=2) for s in (1, 2)]
    extra = [("t.u8", 0, 7), ("t.i8", 1, -7), ("t.u16", 2, 700), ("t.i16", 3, -700),
             ("t.i32", 5, -70000), ("t.f32", 6, 0.5), ("t.bool", 7, True),
             ("t.u64", 10, 1 << 40), ("t.i64", 11, -(1 << 40)), ("t.f64", 12, 0.25),
             ("t.str", synth.GGUF_STRING, "abc"),
             ("t.arr", 9, (5, [1, 2, 3])), ("t.empty", 9, (4, [])),
             ("t.strs", 9, (synth.GGUF_STRING, ["x", "yz", ""])),
             ("t.nested", 9, (9, [(4, [1, 2]), (6, [0.5])]))]
    data, _ = synth.moe_gguf(layers, K=2, extra_kvs=extra)
    with open(path, "wb") as f:
        f.write(data)
    return len(data)


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_gguf_reader_fuzz_asan_ubsan(tmp_path):
    fuzz_dir = str(tmp_path / "fuzz")
    exe = os.path.join(fuzz_dir, "gguf_fuzz")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "qwenqwen3.js_amd"), "FUZZ_DIR=" + fuzz_dir, exe],
                   check=True, capture_output=True, timeout=300)
    gguf = str(tmp_path / "m.gguf")
    n = _fuzz_file(gguf)
    assert n < 64 << 10
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=24")
    r = subprocess.run([exe, gguf, "40000", "7"], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stderr[-4000:]
    ok, refused = (int(v) for v in r.stdout.split()[1:4:2])
    assert ok + refused == 40000
    # the mutations must exercise both outcomes: files accepted (and walked) and refused
    assert ok > 1000 and refused > 1000, r.stdout
