"""The C-ABI library loads and exports every entry point its headers declare
(CPU only: no compute calls)."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "minxfmr.cpp_amd" / "lib" / "libminxfmr_hip.so"


def declared(header: Path, prefix: str) -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return set(re.findall(rf"\b({prefix}\w+)\s*\(", text))


def exported(lib: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], check=True, capture_output=True, text=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if " T " in ln}


def test_library_built_and_loads():
    assert LIB.exists(), "run __graft_entry__.build() first"
    import mxhip  # loads via ctypes; raises if missing

    assert mxhip.LIB_PATH == LIB


def test_every_declared_symbol_is_exported():
    syms = exported(LIB)
    decl = declared(ROOT / "include" / "minxfmr_hip.h", "mxh_")
    assert decl, "no declarations parsed"
    missing = decl - syms
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_binding_covers_header():
    import mxhip

    assert set(mxhip.EXPORTED) == declared(ROOT / "include" / "minxfmr_hip.h", "mxh_")
