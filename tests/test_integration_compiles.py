"""The integration guide's changes to the reference compile in the reference.

Every change the guide (the repository's integration document, read from the
path in DOC) asks a maintainer to make to a reference file is written there as
a hunk: a ```cpp block whose first line is
`// >>> <file>:<line> <before|after> | <fragment of that line>`.  This test
applies all of them to a scratch copy of the reference's sources (line
numbers are those of the unmodified files), puts the wrapper header where
the guide puts it (src/backend/hip/hip_backend.h), and compiles the
patched src/backend/backend_runtime.cpp and src/api/minxfmr.cpp with
`g++ -fsyntax-only`: with MINXFMR_ENABLE_HIP (the HIP build) and without it
(the reference as it was).  Warnings on a hunk's own lines fail the test.

CPU only; skipped where the reference tree is not mounted.
"""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
REF = Path("/root/reference")
DOC = ROOT / "INTEGRATION.md"
WRAPPER_H = ROOT / "minxfmr.cpp_amd" / "csrc" / "backend" / "hip_backend.h"

HUNK = re.compile(r"```cpp\n// >>> (?P<path>[\w/.]+):(?P<line>\d+) (?P<where>before|after) \| (?P<frag>[^\n]*)\n"
                  r"(?P<body>.*?)```", re.S)
# the reference builds with these forced includes under GCC (it omits
# <cmath>/<cstdio> and uses MSVC's _stricmp); compiler flags, not edits
REF_FLAGS = ["-std=gnu++17", "-fsyntax-only", "-include", "cmath", "-include", "cstdio", "-include", "strings.h",
             "-D_stricmp=strcasecmp", "-Wno-narrowing"]

pytestmark = pytest.mark.skipif(not (REF / "src" / "api" / "minxfmr.cpp").exists() or shutil.which("g++") is None,
                                reason="reference tree not mounted")


def hunks():
    out = [m.groupdict() for m in HUNK.finditer(DOC.read_text())]
    for h in out:
        h["line"] = int(h["line"])
    return out


def apply(tmp: Path):
    """Scratch tree with every hunk applied; returns {path: [(first, last)
    1-based line ranges of inserted text in the patched file]}."""
    shutil.copytree(REF / "src", tmp / "src")
    shutil.copytree(REF / "include", tmp / "include")
    shutil.copytree(REF / "third_party", tmp / "third_party")  # minxfmr.cpp includes ../../third_party/gguf
    (tmp / "src" / "backend" / "hip").mkdir()
    shutil.copy(WRAPPER_H, tmp / "src" / "backend" / "hip" / "hip_backend.h")
    by_file: dict[str, list] = {}
    for h in hunks():
        by_file.setdefault(h["path"], []).append(h)
    ranges = {}
    for path, hs in by_file.items():
        lines = (tmp / path).read_text().split("\n")
        orig = list(lines)
        seen = set()
        for h in hs:
            key = (h["line"], h["where"])
            assert key not in seen, f"two hunks at {path}:{h['line']} {h['where']}"
            seen.add(key)
            assert h["frag"] in orig[h["line"] - 1], \
                f"{path}:{h['line']} is {orig[h['line'] - 1]!r}, expected to contain {h['frag']!r}"
        # bottom-up so earlier line numbers stay valid
        inserted = []
        for h in sorted(hs, key=lambda h: (h["line"], h["where"] == "after"), reverse=True):
            body = h["body"].rstrip("\n").split("\n")
            at = h["line"] - 1 if h["where"] == "before" else h["line"]
            lines[at:at] = body
            inserted.append((at, len(body)))
        # inserted ranges in the final numbering
        rs = []
        for at, n in inserted:
            shift = sum(m for a, m in inserted if a < at)
            rs.append((at + shift + 1, at + shift + n))
        ranges[path] = rs
        (tmp / path).write_text("\n".join(lines))
    return ranges


def test_every_hunk_is_parsed():
    hs = hunks()
    files = {h["path"] for h in hs}
    assert files == {"src/backend/backend_runtime.h", "src/backend/backend_runtime.cpp", "src/api/minxfmr.cpp"}
    # every ```cpp block of the integration sections is a hunk (nothing unchecked)
    text = DOC.read_text()
    start, end = text.index("## 1. Backend selection"), text.index("## 4. Build switch")
    blocks = re.findall(r"```cpp\n", text[start:end])
    assert len(blocks) == len(hs)
    # the coarse step uses the entry point that carries the first-token swap
    assert any("mxh_model_set_token" in h["body"] for h in hs)


@pytest.mark.parametrize("hip", [True, False], ids=["hip", "reference"])
@pytest.mark.parametrize("src", ["src/backend/backend_runtime.cpp", "src/api/minxfmr.cpp"])
def test_patched_reference_compiles(tmp_path, src, hip):
    ranges = apply(tmp_path)
    cmd = ["g++", *REF_FLAGS, "-Wall", f"-I{tmp_path / 'include'}", f"-I{tmp_path / 'src'}", f"-I{ROOT / 'include'}",
           str(tmp_path / src)]
    if hip:
        cmd.insert(1, "-DMINXFMR_ENABLE_HIP=1")
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    # no warning on an inserted line (the reference's own warnings are its own)
    mine = []
    for path, rs in ranges.items():
        fname = str(tmp_path / path)
        for m in re.finditer(rf"^{re.escape(fname)}:(\d+):\d+: warning: (.*)$", r.stderr, re.M):
            ln = int(m.group(1))
            if any(a <= ln <= b for a, b in rs):
                mine.append(f"{path}:{ln}: {m.group(2)}")
    assert not mine, "\n".join(mine)
