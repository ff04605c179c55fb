"""The C-ABI library loads and exports every symbol include/*.h declares; host-side
validation follows the reference status convention.  No GPU compute is issued."""

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from robolearn_amd import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "robolearn_mi355x.h"


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(rl_[a-z0-9_]+)\s*\(", text)))


def test_header_compiles_as_c():
    compiler = shutil.which("gcc")
    if compiler is None:
        pytest.skip("gcc missing")
    subprocess.run([compiler, "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-x", "c", str(HEADER)], check=True)


def test_library_exports_every_declared_symbol():
    library = _native.load()
    names = declared_symbols()
    assert len(names) >= 60
    for name in names:
        assert hasattr(library, name), name
    # the ctypes declaration table covers the same set
    assert set(names) == set(_native.SIGNATURES)


def test_status_convention_reports_validation_errors():
    with pytest.raises(RuntimeError, match="positive"):
        _native.call("rl_gemm", 0, 0, 0, 1, 1, 0, 4, 4, 1, 1, 4, 0, 1, 4, 0, None, 1, 4, 0, None, 0, 0.0, 0, 1, None,
                     0, None, None, None, None)
    assert "GEMM" in _native.last_error()
    handle = _native.load().rl_plan_create(0, 4, 4, 0, 0, 4, 4, 4, 0, 0, 0)
    assert not handle and "positive" in _native.last_error()


def test_dense_plan_metadata_and_workspace_on_host():
    library = _native.load()
    # input_dtype 1 is the reference's IEEE fp16; 3 (bf16 operands) and 2 (fp32 stored, bf16 compute) are this
    # library's additions
    for input_dtype, precision in ((1, "fp16"), (2, "bf16"), (3, "bf16")):
        plan = _native.create("rl_plan_create_mixed", 1024, 8192, 160, 1, 0, 160, 160, 1024, 0, 0, input_dtype,
                              64 << 20)
        metadata = library.rl_plan_tuning_metadata(plan).decode()
        assert f'"mode":"{precision}"' in metadata
        assert library.rl_plan_workspace(plan) <= 64 << 20
        assert library.rl_plan_destroy(plan) == 0
    assert not library.rl_plan_create_mixed(64, 64, 64, 0, 0, 64, 64, 64, 0, 0, 4, 0)
    assert "input_dtype" in _native.last_error()


def test_exports_have_c_linkage():
    library = ctypes.CDLL(str(_native.library_path()))
    assert library.rl_last_error is not None
