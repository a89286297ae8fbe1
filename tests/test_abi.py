"""The C-ABI library loads on the CPU host and exports every symbol that
include/funasr_hip.h declares (no device calls)."""
import ctypes
import os
import re

from funasrnet_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "funasr_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fah_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = hip.load()
    names = declared_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name


def test_binding_covers_header():
    assert set(declared_functions()) == set(hip.SIGNATURES)


def test_abi_version_and_error_channel():
    lib = hip.load()
    assert lib.fah_abi_version() == 1
    assert isinstance(lib.fah_last_error(), bytes)
    # A NULL out pointer is rejected before any device work.
    assert lib.fah_context_create(0, None) == hip.ERROR_ARGUMENT
    assert b"NULL" in lib.fah_last_error()


def test_null_handles_are_rejected():
    lib = hip.load()
    assert lib.fah_context_synchronize(None) == hip.ERROR_ARGUMENT
    assert lib.fah_decoder_decode(None, None, 1, None) == hip.ERROR_ARGUMENT
    assert lib.fah_decoder_generate(None, 1, None) == hip.ERROR_ARGUMENT
    assert lib.fah_context_destroy(None) == hip.OK
    assert lib.fah_weight_release(None) == hip.OK
