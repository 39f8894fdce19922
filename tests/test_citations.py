"""The boundary's citations of the reference interface it replaces.

Each C-ABI declaration in include/pulsarlm_amd.h and each C++ drop-in in
pulsarlm_amd/csrc/host/pulsarlm_ops.hpp names the ops.hpp lines of the function it
stands in for. The expected ranges are listed here; where the reference tree is
present (the build container, not the GPU box) the cited lines are also read and must
hold the declaration. CPU only."""

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference/pulsarlm-core/inc/pulsarlm/kernels/ops.hpp"

# function -> (first, last) line of its declaration in ops.hpp
EXPECTED = {
    "repack_int4_marlin_cuda": (306, 311),
    "repack_fp8_marlin_cuda": (313, 314),
    "gemm_int4_marlin_cuda": (316, 323),
    "gemm_fp8_marlin_cuda": (325, 332),
    "route_top_k_cuda": (37, 40),
    "silu_mul_cuda": (42, 43),
    "gemm_int4_cuda": (272, 285),
    "gemm_int4_split_cuda": (287, 297),
}

CITE = re.compile(r"ops\.hpp:(\d+)-(\d+)")


def _read(rel):
    with open(os.path.join(ROOT, rel)) as f:
        return f.read()


def _cited_ranges(text):
    return [(int(a), int(b)) for a, b in CITE.findall(text)]


def _covers(rng, fn):
    lo, hi = EXPECTED[fn]
    return rng[0] <= lo and hi <= rng[1]


@pytest.mark.parametrize("fn", sorted(EXPECTED))
def test_header_cites_each_replaced_function(fn):
    """The header paragraph that says 'Replaces <fn>' cites a range holding fn's lines."""
    text = _read("include/pulsarlm_amd.h")
    paragraphs = re.split(r"\*/", text)
    hits = [p for p in paragraphs if re.search(r"Replaces[^.]*\b%s\b" % fn, p)]
    assert hits, fn
    assert any(_covers(r, fn) for p in hits for r in _cited_ranges(p)), (fn, [_cited_ranges(p) for p in hits])


@pytest.mark.parametrize("fn", sorted(EXPECTED))
def test_host_layer_cites_each_replaced_function(fn):
    text = _read("pulsarlm_amd/csrc/host/pulsarlm_ops.hpp")
    decl = re.search(r"\b%s\(" % fn, text)
    assert decl, fn
    comment = text[max(0, text.rfind(";", 0, decl.start())):decl.start()]
    if not _cited_ranges(comment):  # a block comment shared by the pair of int4 GEMMs
        comment = text[max(0, text.rfind("}", 0, decl.start()), text.rfind(";", 0, text.rfind("//", 0, decl.start()))):decl.start()]
    assert any(_covers(r, fn) for r in _cited_ranges(comment)), (fn, comment)


FILES = ["include/pulsarlm_amd.h", "pulsarlm_amd/csrc/host/pulsarlm_ops.hpp", "pulsarlm_amd/ops.py",
         "INTEGRATION.md", "DESIGN.md"]


@pytest.mark.skipif(not os.path.exists(REF), reason="reference tree not present")
def test_every_cited_range_exists_in_the_reference():
    with open(REF) as f:
        lines = f.read().split("\n")
    for rel in FILES:
        for lo, hi in _cited_ranges(_read(rel)):
            assert 1 <= lo <= hi <= len(lines), (rel, lo, hi, len(lines))


@pytest.mark.skipif(not os.path.exists(REF), reason="reference tree not present")
def test_expected_ranges_hold_the_declarations():
    with open(REF) as f:
        lines = f.read().split("\n")
    for fn, (lo, hi) in EXPECTED.items():
        span = "\n".join(lines[lo - 1:hi])
        assert re.search(r"\b%s\(" % fn, span), (fn, lo, hi)
        # The range ends at the declaration's closing ';'.
        assert lines[hi - 1].rstrip().endswith(";"), (fn, lines[hi - 1])
