"""The profiling CSVs use the reference's column sets (CPU, no GPU).

enable_profiling writes the operator table of the reference's Profiler and
its command / kernel / operation sidecars (profiler.cpp:127-174, 619-632).
This compares the header lines our runtime writes (the string literals of
myllm_amd/csrc/runtime/profile.cpp) with the reference's, field by field;
skipped where the reference sources are absent.
"""

from __future__ import annotations

import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
REFERENCE = pathlib.Path("/root/reference/profiler.cpp")


def header_lines(source: str) -> list[str]:
    """Every header line: adjacent string literals joined, split at \\n."""
    text = re.sub(r"'(?:[^'\\]|\\.)'", "", source)  # char literals ('"') out of the way
    text = re.sub(r'"\s*\n\s*"', "", text)  # join literals across lines
    out = []
    for lit in re.findall(r'"((?:[^"\\]|\\.)*)"', text):
        if lit.startswith(("record_type,", "command_index,")) and lit.endswith("\\n"):
            out.append(lit[:-2])
    return out


@pytest.mark.skipif(not REFERENCE.exists(), reason="reference sources not present")
def test_profile_headers_match_reference():
    ours = header_lines((ROOT / "myllm_amd" / "csrc" / "runtime" / "profile.cpp").read_text())
    theirs = header_lines(REFERENCE.read_text())
    assert len(theirs) == 4 and len(ours) == 4
    assert sorted(ours) == sorted(theirs)
