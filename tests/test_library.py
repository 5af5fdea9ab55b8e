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


def _prototypes() -> dict:
    """name -> (return type, [parameter types]) for every prototype in the header."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"^\s*#.*$", "", text, flags=re.M)
    out = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w\s\*]*?)\s*\b(mirl_\w+)\s*\(([^)]*)\)\s*;", text):
        ps = [p.strip() for p in params.split(",") if p.strip() and p.strip() != "void"]
        # drop the parameter name: what remains is the type
        types = [re.sub(r"\s*\b\w+$", "", p).replace(" *", "*").strip() for p in ps]
        out[name] = (ret.split()[-1] if ret.strip() else ret, types)
    return out


def _ctype_matches(ctype_name: str, ct) -> bool:
    import ctypes

    if ctype_name.endswith("*"):
        return ct in (ctypes.c_void_p, ctypes.c_char_p) or (
            isinstance(ct, type) and issubclass(ct, ctypes._Pointer))
    scalar = {"int64_t": ctypes.c_int64, "int": ctypes.c_int, "double": ctypes.c_double,
              "float": ctypes.c_float, "uint32_t": ctypes.c_uint32, "int32_t": ctypes.c_int32}
    if ctype_name in scalar:
        return ct is scalar[ctype_name]
    # a struct passed by value
    return isinstance(ct, type) and issubclass(ct, ctypes.Structure) and ct.__name__ != ""


def test_binding_argument_types_follow_the_header():
    """Every entry point's ctypes argument list has the header's arity and, position by
    position, the same kind of type (a changed C signature must change the binding too)."""
    from rl_amd import _C

    protos = _prototypes()
    assert set(protos) == set(_C.SIGNATURES)
    bad = []
    for name, (_, ptypes) in protos.items():
        _, argtypes = _C.SIGNATURES[name]
        if len(argtypes) != len(ptypes):
            bad.append((name, "arity", len(ptypes), len(argtypes)))
            continue
        for k, (pt, ct) in enumerate(zip(ptypes, argtypes)):
            if not _ctype_matches(pt, ct):
                bad.append((name, k, pt, ct))
    assert not bad, bad
