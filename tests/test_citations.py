"""Every `file.rs:LINE[-LINE]` citation of the reference in this repository
points inside the cited file, and the boundary's optimizer anchors point at
the functions they name.

Runs on the CPU, reading the reference's source files as text; skipped where
the reference checkout is absent (the GPU box has none).
"""
from __future__ import annotations

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.environ.get("NUMRS_REFERENCE", "/root/reference")

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "numrs-core")),
                                reason="reference checkout not present")

# path.ext:a[-b][, c[-d]]...
CITE = re.compile(r"([A-Za-z0-9_/.\-]+\.(?:rs|toml|wgsl|metal)):(\d+)(?:-(\d+))?"
                  r"((?:,\s*\d+(?:-\d+)?)*)")
SCAN_DIRS = ("include", "numrs_amd", "oracle", "tests")
SCAN_FILES = ("DESIGN.md", "INTEGRATION.md", "README.md", "bench.py", "__graft_entry__.py")
SCAN_EXT = (".h", ".hip", ".py", ".c", ".md", "Makefile")


def _reference_files() -> dict[str, list[str]]:
    by_name: dict[str, list[str]] = {}
    for dp, dns, fns in os.walk(REF):
        dns[:] = [d for d in dns if d not in (".git", "target", "node_modules")]
        for f in fns:
            by_name.setdefault(f, []).append(os.path.join(dp, f))
    return by_name


def _lines(path: str, cache: dict[str, list[str]]) -> list[str]:
    if path not in cache:
        with open(path, encoding="utf-8", errors="replace") as fh:
            cache[path] = fh.read().split("\n")
    return cache[path]


def _sources():
    for d in SCAN_DIRS:
        for dp, dns, fns in os.walk(os.path.join(ROOT, d)):
            dns[:] = [x for x in dns if x not in ("__pycache__", "build", "lib", "_ref")]
            for f in fns:
                if f.endswith(SCAN_EXT):
                    yield os.path.join(dp, f)
    for f in SCAN_FILES:
        p = os.path.join(ROOT, f)
        if os.path.exists(p):
            yield p


def test_every_citation_lies_inside_its_file():
    files = _reference_files()
    cache: dict[str, list[str]] = {}
    bad, seen = [], 0
    for src in _sources():
        with open(src, encoding="utf-8", errors="replace") as fh:
            text = fh.read()
        for ln, line in enumerate(text.split("\n"), 1):
            for m in CITE.finditer(line):
                path = m.group(1)
                cands = [c for c in files.get(os.path.basename(path), [])
                         if c.endswith("/" + path.lstrip("./")) or c.endswith(path)]
                if not cands:
                    continue  # not a reference file (or a path this scan cannot resolve)
                ranges = [(int(m.group(2)), int(m.group(3) or m.group(2)))]
                for a, b in re.findall(r"(\d+)(?:-(\d+))?", m.group(4) or ""):
                    ranges.append((int(a), int(b or a)))
                seen += 1
                ok = any(all(1 <= lo <= hi <= len(_lines(c, cache)) for lo, hi in ranges)
                         for c in cands)
                if not ok:
                    bad.append(f"{os.path.relpath(src, ROOT)}:{ln}: {m.group(0)}")
    assert seen > 100, f"only {seen} citations found: the scan is broken"
    assert not bad, "citations outside their file:\n" + "\n".join(bad)


# The optimizer entry points of the boundary and what their anchors must name.
ANCHORS = [
    ("numrs-core/src/autograd/optim/sgd.rs", 87, "fn step"),
    ("numrs-core/src/autograd/optim/sgd.rs", 124, "}"),
    ("numrs-core/src/autograd/optim/sgd.rs", 47, "pub fn new"),
    ("numrs-core/src/autograd/optim/sgd.rs", 71, "pub fn simple"),
    ("numrs-core/src/autograd/optim/sgd.rs", 126, "fn zero_grad"),
    ("numrs-core/src/autograd/optim/adam.rs", 124, "fn step"),
    ("numrs-core/src/autograd/optim/adam.rs", 167, "}"),
    ("numrs-core/src/autograd/optim/adam.rs", 64, "pub fn new"),
    ("numrs-core/src/autograd/optim/adam.rs", 102, "pub fn default"),
    ("numrs-core/src/autograd/optim/adam.rs", 128, "powi"),
    ("numrs-core/src/autograd/optim/adam.rs", 162, "v_hat.sqrt() + self.eps"),
    ("numrs-core/src/autograd/optim/base.rs", 26, "fn apply_weight_decay"),
    ("numrs-core/src/autograd/tensor.rs", 173, "pub fn backward"),
    ("numrs-core/src/autograd/tensor.rs", 218, "fn build_topo"),
    ("numrs-core/src/autograd/tensor.rs", 120, "fn accumulate_gradient"),
    ("numrs-core/src/autograd/backward.rs", 12, "fn unbroadcast"),
    ("numrs-core/src/autograd/backward.rs", 152, "fn relu_backward"),
    ("numrs-core/src/autograd/backward.rs", 239, "fn mse_backward"),
    ("numrs-core/src/autograd/backward.rs", 265, "fn cross_entropy_backward"),
    ("numrs-core/src/autograd/backward.rs", 315, "fn flatten_backward"),
    ("numrs-core/src/autograd/backward.rs", 324, "fn reshape_backward"),
    ("numrs-core/src/autograd/backward.rs", 521, "fn softmax_backward"),
    ("numrs-core/src/ops/model.rs", 550, "pub fn save_checkpoint"),
    ("numrs-core/src/ops/model.rs", 577, "pub fn load_checkpoint"),
]


@pytest.mark.parametrize("path,line,needle", ANCHORS)
def test_boundary_anchor_names_its_function(path, line, needle):
    lines = _lines(os.path.join(REF, path), {})
    assert needle in lines[line - 1], f"{path}:{line} is {lines[line - 1]!r}"


def test_header_cites_the_anchors():
    with open(os.path.join(ROOT, "include", "numrs_hip.h"), encoding="utf-8") as fh:
        h = fh.read()
    for cite in ("optim/sgd.rs:87-124", "optim/adam.rs:124-167", "optim/sgd.rs:47-69",
                 "optim/adam.rs:64-99"):
        assert cite in h, cite
