"""Every citation of a reference source line (`dir/file.odin:N` or `:N-M`,
also `.metal` / `.sh`) in the sources and documents of this repository names
a file that exists in the reference tree, names it unambiguously (a bare
`forward.odin` could be infer/ or qwen3_5/), and stays within its lines.

The reference tree is read as text only; the test is skipped where it is
absent (the GPU box)."""
import os
import re

import pytest

REF = "/root/reference"
REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCAN = ["odin-infer_amd/csrc", "odin-infer_amd/oi", "odin-infer_amd/odin", "include", "oracle", "tests",
        "DESIGN.md", "INTEGRATION.md", "bench.py", "__graft_entry__.py", "odin-infer_amd/build.py"]
SRC_EXT = re.compile(r"\.(hip|cpp|h|c|py|md|odin)$")
CITE = re.compile(r"(?<![A-Za-z0-9_./-])([A-Za-z0-9_][A-Za-z0-9_./-]*\.(?:odin|metal|sh))"
                  r":(\d+(?:-\d+)?(?:, \d+(?:-\d+)?)*)")


def _reference_files():
    out = {}
    for root, dirs, files in os.walk(REF):
        dirs[:] = [d for d in dirs if not d.startswith(".")]
        for f in files:
            p = os.path.join(root, f)
            with open(p, "rb") as fh:
                data = fh.read()
            out[os.path.relpath(p, REF)] = data.count(b"\n") + (0 if data.endswith(b"\n") else 1)
    return out


def _sources():
    for top in SCAN:
        p = os.path.join(REPO, top)
        if os.path.isfile(p):
            yield p
            continue
        for root, dirs, files in os.walk(p):
            dirs[:] = [d for d in dirs if d not in ("_ref", "__pycache__", "golden")]
            for f in files:
                if SRC_EXT.search(f):
                    yield os.path.join(root, f)


def citations():
    for p in _sources():
        with open(p, errors="replace") as fh:
            for i, line in enumerate(fh, 1):
                for m in CITE.finditer(line):
                    ranges = []
                    for part in m.group(2).split(", "):
                        a, _, b = part.partition("-")
                        ranges.append((int(a), int(b or a)))
                    yield os.path.relpath(p, REPO), i, m.group(1).lstrip("./"), ranges


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference tree not present")
def test_reference_citations_resolve():
    files = _reference_files()
    seen, bad = 0, []
    for src, line, name, ranges in citations():
        seen += 1
        cands = [r for r in files if r == name or r.endswith("/" + name)]
        where = "%s:%d cites %s:%s" % (src, line, name, ranges)
        if not cands:
            bad.append(where + ": no such reference file")
        elif len(cands) > 1:
            bad.append(where + ": ambiguous (%s)" % ", ".join(sorted(cands)))
        else:
            n = files[cands[0]]
            for a, b in ranges:
                if not (1 <= a <= b <= n):
                    bad.append(where + ": lines %d-%d outside the file's %d" % (a, b, n))
    assert seen > 200, "the scan found only %d citations" % seen
    assert not bad, "\n".join(bad)


def test_citation_pattern():
    got = [(m.group(1), m.group(2)) for m in CITE.finditer(
        "x (infer/forward.odin:119-121, 137-139) and `qwen3_5/metal.odin:22`, not a.odin or b.odin: q")]
    assert got == [("infer/forward.odin", "119-121, 137-139"), ("qwen3_5/metal.odin", "22")]
