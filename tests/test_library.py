"""The C-ABI library loads and exports every symbol include/mirl.h declares (CPU only, no compute)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mirl.h"
LIB = ROOT / "rl_amd" / "libmirl.so"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mirl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for required in ["mirl_logprob_fwd", "mirl_logprob_bwd", "mirl_clipped_pg",
                     "mirl_grpo_advantage", "mirl_last_error", "mirl_version"]:
        assert required in names


def test_library_exports_every_declared_symbol():
    if not LIB.exists():
        pytest.fail(f"{LIB} not built (run python -m rl_amd.csrc.build)")
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_header():
    from rl_amd import _C

    assert set(_C.SIGNATURES) == set(declared_functions())


def test_version_and_error_calls_need_no_gpu():
    from rl_amd import _C

    lib = _C.load()
    assert lib.mirl_version().decode().startswith("mirl")
    assert lib.mirl_last_error().decode() == ""


def test_invalid_arguments_return_status_not_abort():
    """Host-side validation runs before any device work: bad shapes give a status code."""
    from rl_amd import _C

    lib = _C.load()
    st = lib.mirl_logprob_fwd(None, 7, 1, 1, 10, 10, 10, None, 1, 1, 0, 10, None, None, None)
    assert st != 0
    assert "dtype" in lib.mirl_last_error().decode()
    st = lib.mirl_logprob_fwd(None, 0, 1, 1, 0, 0, 0, None, 1, 1, 0, 10, None, None, None)
    assert st != 0
    assert "shape" in lib.mirl_last_error().decode()
    assert lib.mirl_clipped_pg_workspace_elems(8, 100, 0) > 0
    assert lib.mirl_clipped_pg_workspace_elems(8, 100, 1) == lib.mirl_clipped_pg_workspace_elems(8, 100, 0) + 2400
