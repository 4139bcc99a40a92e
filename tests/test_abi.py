"""The C-ABI library loads and exports every symbol include/ttrl_hip.h
declares, and the ctypes table matches the header (no GPU calls)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _declared():
    text = (ROOT / "include" / "ttrl_hip.h").read_text()
    return sorted(set(re.findall(r"\b(ttrl_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from ttrl_amd import _lib

    dll = ctypes.CDLL(str(_lib.LIB_PATH))
    names = _declared()
    assert len(names) > 30
    missing = [n for n in names if not hasattr(dll, n)]
    assert not missing, missing


def test_ctypes_table_covers_the_header():
    from ttrl_amd import _lib

    assert set(_declared()) == set(_lib.SIGNATURES)
    _lib.load()  # every signature resolves


def test_library_is_built_for_gfx950_only():
    from ttrl_amd import _lib

    blob = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in blob
    assert b"gfx942" not in blob and b"sm_" not in blob[:0]


def test_errors_are_reported_without_a_device():
    from ttrl_amd import _lib

    out = ctypes.c_int(0)
    rc = _lib.lib().ttrl_conv_out_size(6, 3, 2, 0, ctypes.byref(out))
    assert rc == _lib.TTRL_EINVAL
    assert b"ragged" in _lib.lib().ttrl_last_error()
    rc = _lib.lib().ttrl_conv_out_size(84, 8, 4, 0, ctypes.byref(out))
    assert rc == 0 and out.value == 20
