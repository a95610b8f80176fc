"""A C++ program compiled against include/fmx.h and linked to libfmx.so
(tests/c_abi/fmx_abi_check.cpp, built by the Makefile beside it) runs the
load-time and forward sequence of the reference's C++ server on the
small_dec_t4 layer; its output must match the committed fixture."""
from __future__ import annotations

import pathlib
import subprocess

import numpy as np
import pytest

from helpers import assert_close

ROOT = pathlib.Path(__file__).resolve().parents[1]
PROG = ROOT / "tests" / "c_abi" / "_build" / "fmx_abi_check"
GOLD = ROOT / "tests" / "golden" / "small_dec_t4.npz"


def test_program_links_libfmx():
    """Built by __graft_entry__.build(); resolves libfmx.so from the tree."""
    assert PROG.exists(), f"{PROG} missing: run __graft_entry__.build()"
    out = subprocess.run(["ldd", str(PROG)], capture_output=True, text=True, check=True).stdout
    line = next(ln for ln in out.splitlines() if "libfmx.so" in ln)
    assert "not found" not in line and str(ROOT / "flashmlx_amd") in str(pathlib.Path(line.split("=>")[1].split()[0]).resolve())


@pytest.mark.gpu
def test_program_matches_fixture(gpu, tmp_path):
    y_path, i_path = tmp_path / "y.bin", tmp_path / "inds.bin"
    print("running", PROG, flush=True)
    p = subprocess.run([str(PROG), str(y_path), str(i_path)], capture_output=True, text=True,
                       timeout=120)
    print(p.stdout, p.stderr)
    assert p.returncode == 0, p.stderr
    with np.load(GOLD, allow_pickle=False) as g:
        y_rows, inds, tokens = g["y_rows"], g["inds"], g["tokens"]
    T, k = inds.shape
    y = np.fromfile(y_path, np.uint16).reshape(T, -1)
    np.testing.assert_array_equal(np.fromfile(i_path, np.uint32).reshape(T, k), inds)
    e = assert_close(y[tokens], y_rows, "fmx_abi_check y")
    print(f"C++ program vs fixture: {e}")
