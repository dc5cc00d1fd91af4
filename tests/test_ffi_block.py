"""The Rust FFI blocks a numrs maintainer would paste into
numrs-core/src/backend/hip/mod.rs (kept in the integration guide at the
repository root) against the C header and the ctypes table: every function
the header declares appears once, with as many parameters as the ctypes
binding passes.  No cargo here, so this is the check that the Rust side
stays in step with the library."""
import collections
import os
import re

from numrs_amd import _lib as L

GUIDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                     "INTEGRATION.md")


def _ffi_functions():
    text = open(GUIDE).read()
    fns = []
    for m in re.finditer(r'extern "C" \{', text):
        end = text.index("\n}", m.start())
        block = re.sub(r"//[^\n]*", "", text[m.start():end])
        fns += re.findall(r"pub fn (numrs_hip_\w+)\s*\((.*?)\)\s*(?:->\s*[^;]+)?;", block, re.S)
    return fns


def test_ffi_blocks_declare_every_header_function_once():
    fns = _ffi_functions()
    names = [f for f, _ in fns]
    dups = [n for n, c in collections.Counter(names).items() if c > 1]
    assert not dups, f"declared twice in the FFI blocks: {dups}"
    header = set(L.header_functions())
    assert not sorted(set(names) - header), "FFI names missing from the header"
    assert not sorted(header - set(names)), f"header functions missing from the FFI blocks: " \
                                            f"{sorted(header - set(names))}"


def test_ffi_arity_matches_ctypes():
    bad = []
    for name, args in _ffi_functions():
        n = len([a for a in args.split(",") if a.strip()])
        if len(L.SIGNATURES[name][1]) != n:
            bad.append((name, n, len(L.SIGNATURES[name][1])))
    assert not bad, f"parameter counts differ (name, FFI, ctypes): {bad}"
