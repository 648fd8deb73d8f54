"""The C ABI boundary on the CPU: the library builds, loads and exports every
entry point include/qq_moe.h declares; device errors surface as codes and
messages (no silent fallback)."""
import ctypes
import os
import re

import pytest

import qq_hip
from _util import ROOT

HEADER = os.path.join(ROOT, "include", "qq_moe.h")
GGUF_HEADER = os.path.join(ROOT, "include", "qq_gguf.h")
LFM2_HEADER = os.path.join(ROOT, "include", "qq_lfm2.h")
HAS_GPU = os.path.exists("/dev/kfd")


def declared_functions(header=None):
    if header is None:
        return sorted(set(declared_functions(HEADER)) | set(declared_functions(GGUF_HEADER)) |
                      set(declared_functions(LFM2_HEADER)))
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qq_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions(HEADER) == sorted(qq_hip.EXPORTS)
    assert declared_functions(GGUF_HEADER) == sorted(qq_hip.GGUF_EXPORTS)
    assert declared_functions(LFM2_HEADER) == sorted(qq_hip.LFM2_EXPORTS)


def test_every_header_is_covered():
    assert sorted(os.listdir(os.path.join(ROOT, "include"))) == ["qq_gguf.h", "qq_lfm2.h", "qq_moe.h"]


def test_library_exports_every_declared_symbol():
    lib = qq_hip.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_header_constants_match_binding():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define\s+(QQ_[A-Z0-9_]+)\s+(-?\d+)", text))
    assert int(consts["QQ_OK"]) == qq_hip.QQ_OK
    assert int(consts["QQ_TYPE_F32"]) == qq_hip.TYPE_F32
    assert int(consts["QQ_TYPE_Q8_0"]) == qq_hip.TYPE_Q8_0
    assert int(consts["QQ_WAIT_LIMIT_US_DEFAULT"]) == qq_hip.QQ_WAIT_LIMIT_US_DEFAULT


@pytest.mark.skipif(HAS_GPU, reason="checks the no-device error path")
def test_init_without_device_fails_loudly():
    lib = qq_hip.load()
    h = ctypes.c_void_p()
    rc = lib.qq_init(0, ctypes.byref(h))
    assert rc == -3 and not h.value
    assert b"device" in lib.qq_last_error(None)
    with pytest.raises(qq_hip.QQError, match="qq_init"):
        qq_hip.Context(0)


def test_null_context_is_rejected():
    lib = qq_hip.load()
    assert lib.qq_synchronize(None) == -1
    assert lib.qq_timer_start(None) == -1
    assert lib.qq_moe_forward(None, None, None, None, 1, None, None, None, None) == -1
