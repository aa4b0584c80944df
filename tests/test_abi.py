"""The C ABI: libvdnh3.so loads and exports every function declared in include/vdnh3.h."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "vdnh3.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vdnh3_\w+)\s*\(", text)))


def test_header_declares_the_bound_symbols(built_lib):
    from vdn_h3_amd import _lib

    names = declared_functions()
    assert names, "no declarations found"
    assert sorted(_lib.SIGNATURES) == names


def test_library_exports_every_declared_symbol(built_lib):
    from vdn_h3_amd import _lib

    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\b(vdnh3_\w+)\b", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    for name in declared_functions():
        assert getattr(built_lib, name) is not None


def test_version_and_error_channel(built_lib):
    from vdn_h3_amd import _lib

    assert built_lib.vdnh3_abi_version() >= 100
    assert isinstance(_lib.last_error(), str)
