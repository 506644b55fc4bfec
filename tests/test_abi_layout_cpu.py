"""The ctypes argument structs (bmx_amd/_lib.py) against the C headers they
mirror (include/*.h): every struct's size and every field's offset, read from
a small C program that gcc builds against the headers, so that a field added
on one side only cannot pass silently.  And the ctypes stubs shown to a
maintainer in INTEGRATION.md: run as written, they have the shipped layouts."""
import ctypes as ct
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from bmx_amd import _lib

ROOT = Path(__file__).resolve().parents[1]

# ctypes class -> C typedef
STRUCTS = {
    "Geom": "bmx_k2b_geom",
    "DecodeArgs": "bmx_k2b_decode_args",
    "AppendArgs": "bmx_k2b_append_args",
    "DequantArgs": "bmx_k2b_dequant_args",
    "RtnGeom": "bmx_rtn_geom",
    "RtnAppendArgs": "bmx_rtn_append_args",
    "RtnDecodeArgs": "bmx_rtn_decode_args",
    "RtnDequantArgs": "bmx_rtn_dequant_args",
    "SpectralLayout": "bmx_spectral_layout",
    "SpectralAppendArgs": "bmx_spectral_append_args",
    "SpectralDequantArgs": "bmx_spectral_dequant_args",
    "SpectralMergeArgs": "bmx_spectral_merge_args",
    "Fp16DecodeArgs": "bmx_fp16_decode_args",
    "PrefillArgs": "bmx_prefill_args",
}


def _c_layouts(tmp_path):
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "bmx_k2b.h"', '#include "bmx_rtn.h"',
             '#include "bmx_spectral.h"', '#include "bmx_bench.h"', '#include "bmx_prefill.h"', "int main(void) {"]
    for py, c in STRUCTS.items():
        cls = getattr(_lib, py)
        lines.append(f'  printf("{py} sizeof %zu\\n", sizeof({c}));')
        for f in cls._fields_:
            lines.append(f'  printf("{py} {f[0]} %zu\\n", offsetof({c}, {f[0]}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "abi.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "abi"
    subprocess.run(["gcc", "-std=c11", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True,
                   capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        py, field, val = line.split()
        got[(py, field)] = int(val)
    return got


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not found")
def test_ctypes_structs_match_the_headers(tmp_path):
    got = _c_layouts(tmp_path)
    for py in STRUCTS:
        cls = getattr(_lib, py)
        assert got[(py, "sizeof")] == ct.sizeof(cls), f"{py}: sizeof C {got[(py, 'sizeof')]} != ctypes {ct.sizeof(cls)}"
        for f in cls._fields_:
            off = getattr(cls, f[0]).offset
            assert got[(py, f[0])] == off, f"{py}.{f[0]}: offset C {got[(py, f[0])]} != ctypes {off}"


def test_integration_stubs_match_the_shipped_binding():
    """Every ctypes class INTEGRATION.md shows, run as written (in the order
    shown: later classes use earlier ones), has the shipped class's field
    names, size and offsets."""
    text = (ROOT / "INTEGRATION.md").read_text()
    ns = {"ct": ct}
    shown = []
    for m in re.finditer(r"^class (\w+)\(ct\.Structure\):", text, re.M):
        block = text[m.start():text.index("\n\n", m.start())]
        exec(block, ns)   # the document's own stub code
        shown.append(m.group(1))
    assert {"Geom", "DecodeArgs", "RtnGeom", "RtnDecodeArgs"} <= set(shown)
    for py in shown:
        doc, lib = ns[py], getattr(_lib, py)
        assert [f[0] for f in doc._fields_] == [f[0] for f in lib._fields_], py
        assert ct.sizeof(doc) == ct.sizeof(lib), py
        for f in lib._fields_:
            assert getattr(doc, f[0]).offset == getattr(lib, f[0]).offset, f"{py}.{f[0]}"
