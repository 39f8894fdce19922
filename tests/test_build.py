"""Build checks on the CPU: every gfx950 kernel in libpulsarlm_amd.so keeps its
registers in registers. The build (pulsarlm_amd/build.py) saves the compiler's
kernel-resource-usage report per source; a kernel with a nonzero ScratchSize spills
to scratch memory, i.e. extra HBM traffic inside a bandwidth-bound kernel."""

import re
from pathlib import Path

import pytest

BUILD = Path(__file__).resolve().parent.parent / "pulsarlm_amd" / "_build"
REPORTS = sorted(BUILD.glob("*.resources.txt"))


def _kernels(text):
    for block in re.split(r"remark: Function Name: ", text)[1:]:
        name = block.split(" ", 1)[0]
        scratch = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", block)
        yield name, int(scratch.group(1)) if scratch else 0


@pytest.mark.skipif(not REPORTS, reason="library not built in this tree")
def test_no_kernel_spills_to_scratch():
    spilled, total = [], 0
    for rep in REPORTS:
        for name, scratch in _kernels(rep.read_text()):
            total += 1
            if scratch:
                spilled.append((rep.stem, name, scratch))
    assert total > 0
    assert not spilled, spilled


@pytest.mark.skipif(not REPORTS, reason="library not built in this tree")
def test_reports_are_not_older_than_their_sources():
    """A failed rebuild leaves the previous report (and library) behind: every report must
    be at least as new as its source and the shared header."""
    csrc = BUILD.parent / "csrc"
    header = (csrc / "plm_common.hpp").stat().st_mtime
    for rep in REPORTS:
        src = csrc / (rep.name.replace(".resources.txt", "") + ".hip")
        if src.exists():
            assert rep.stat().st_mtime >= max(src.stat().st_mtime, header), f"{rep.name} is older than its sources"
