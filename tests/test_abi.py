"""CPU-side checks of the C ABI: the library loads and exports every symbol
include/pokit_hip.h declares; the Python host layer's argument checks.
No kernel runs here (there is no GPU in this container)."""
import ctypes
import os
import re

import pytest

from pokitlms_amd import _abi

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "pokit_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pk_hip_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_bound_symbols():
    assert declared_symbols() == sorted(_abi.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_version_and_type_table():
    lib = _abi.lib()
    assert lib.pk_hip_version() == b"0.1.0"
    # every type tensor_linear dispatches (src/tensor_linear.cpp:176-187)
    for t in (0, 1, 2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 30):
        assert lib.pk_hip_type_supported(t) == 1
    for t in (4, 5, 9, 15, 16, 99):
        assert lib.pk_hip_type_supported(t) == 0


def header_stats_fields():
    text = open(os.path.join(ROOT, "include", "pokit_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    body = re.search(r"typedef struct pk_hip_stats \{(.*?)\} pk_hip_stats;", text, re.S).group(1)
    names = []
    for decl in body.split(";"):
        decl = decl.strip()
        if decl:
            assert decl.startswith("uint64_t "), decl
            names += [n.strip() for n in decl[len("uint64_t "):].split(",")]
    return names


def test_struct_layouts_match_header():
    # pk_hip_moe_layer: 4 pointers, two uint32, one float (+ tail padding)
    assert ctypes.sizeof(_abi.MoeLayerDesc) == 4 * 8 + 4 + 4 + 4 + 4
    assert ctypes.sizeof(_abi.Options) == 8
    # pk_hip_stats: every field uint64_t, same names in the same order
    assert [n for n, _ in _abi.Stats._fields_] == header_stats_fields()
    assert ctypes.sizeof(_abi.Stats) == 8 * len(header_stats_fields())


def test_null_arguments_are_rejected_without_a_device():
    lib = _abi.lib()
    err = ctypes.create_string_buffer(128)
    # no output handle: INVALID_ARGUMENT before any device call
    assert lib.pk_hip_create(0, None, None, err, 128) == _abi.STATUS_INVALID_ARGUMENT
    assert b"output handle" in err.value
    assert lib.pk_hip_get_stats(None, None) == _abi.STATUS_INVALID_ARGUMENT
    assert lib.pk_hip_matvec(None, None, 0, None, 1, None, err, 128) == \
        _abi.STATUS_INVALID_ARGUMENT
    lib.pk_hip_destroy(None)
    lib.pk_hip_weight_release(None)


def test_error_buffer_is_truncated_and_terminated():
    lib = _abi.lib()
    err = ctypes.create_string_buffer(b"\xff" * 8)
    assert lib.pk_hip_create(0, None, None, err, 8) == _abi.STATUS_INVALID_ARGUMENT
    assert err.raw[7] == 0 and len(err.value) == 7


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_abi, "_lib", None)
    monkeypatch.setattr(_abi, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(ImportError):
        _abi.lib()
