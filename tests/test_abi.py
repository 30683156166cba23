"""CPU checks of the C-ABI boundary: the library builds and loads, and exports
every entry point include/qwhip.h declares (no device calls are made)."""
import ctypes
import os
import re

import qwenscriber_amd as qa
from qwenscriber_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_entry_points():
    text = open(os.path.join(ROOT, "include", "qwhip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qwh_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_documented_surface():
    names = declared_entry_points()
    for required in ("qwh_linear", "qwh_decode_attention_q8", "qwh_kv_append_q8", "qwh_decoder_step",
                     "qwh_matrix_upload", "qwh_quantize_rows"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(qa.library_path())
    missing = [n for n in declared_entry_points() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert sorted(_lib.SIGNATURES) == declared_entry_points()


def test_abi_version_and_status_names():
    lib = qa.load()
    assert lib.qwh_abi_version() == 0x00010000
    assert lib.qwh_status_string(-7) == b"shape_mismatch"
    assert lib.qwh_status_string(-9) == b"limit_exceeded"


def test_null_arguments_are_rejected_without_a_device():
    lib = qa.load()
    assert lib.qwh_create(0, None) == -1
    assert lib.qwh_destroy(None) == -1
    assert lib.qwh_sync(None) == -1
    assert lib.qwh_linear(None, 1, None, 64, 1, None) == -1
