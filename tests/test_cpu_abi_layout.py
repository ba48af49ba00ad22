"""The public header is a drop-in for the reference's: tests/c/abi_layout.c
prints every struct size and field offset and every enum value of
slipstream.h, compiled once against include/slipstream.h and once against
the reference's SlipStream/include/slipstream.h (:32-106, :274-284). Every
line of the reference's output must appear unchanged in ours (ours adds
SS_BACKEND_HIP and extension types, which the program does not print).
Skipped where the reference tree is absent."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INCLUDE = os.path.join(os.environ.get("SS_REFERENCE_DIR", "/root/reference/SlipStream"), "include")


def _dump(tmp_path, include_dir, tag):
    exe = str(tmp_path / ("abi_" + tag))
    subprocess.run(["gcc", "-std=c11", "-Wall", "-I", include_dir, "-o", exe,
                    os.path.join(ROOT, "tests", "c", "abi_layout.c")], check=True)
    return subprocess.run([exe], check=True, capture_output=True, text=True).stdout.splitlines()


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_INCLUDE, "slipstream.h")),
                    reason="reference tree absent")
def test_public_header_layout_matches_reference(tmp_path):
    ref = _dump(tmp_path, REF_INCLUDE, "ref")
    ours = _dump(tmp_path, os.path.join(ROOT, "include"), "ours")
    assert len(ref) > 50
    assert ours == ref
