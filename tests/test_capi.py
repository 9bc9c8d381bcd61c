"""CPU checks of the C ABI: the library loads and exports every declared symbol."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from bioemu2_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
_DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(bioemu_\w+)\s*\(", re.M)


def _declared() -> list[str]:
    names: list[str] = []
    for h in sorted((ROOT / "include").glob("*.h")):
        names += _DECL.findall(h.read_text())
    return sorted(set(names))


def test_header_declares_entry_points():
    names = _declared()
    assert "bioemu_trimul_fwd" in names
    assert len(names) >= 4


def test_library_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"native library not built: {_lib.LIB_PATH}")
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in _declared() if not hasattr(handle, n)]
    assert not missing, missing


def test_python_binding_covers_every_declared_symbol():
    assert sorted(_lib.SIGNATURES) == _declared()


def _declared_arity() -> dict[str, int]:
    """Parameter count of every declared entry point, parsed from include/*.h."""
    text = "\n".join(h.read_text() for h in sorted((ROOT / "include").glob("*.h")))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(bioemu_\w+)\s*\(([^;{]*?)\)\s*;", text, re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_binding_arity_matches_header():
    arity = _declared_arity()
    assert set(arity) == set(_lib.SIGNATURES)
    for name, (_, argtypes) in _lib.SIGNATURES.items():
        assert len(argtypes) == arity[name], (name, len(argtypes), arity[name])


def test_host_only_queries():
    lib = _lib.lib()
    assert b"gfx950" in lib.bioemu_version()
    n = 768
    np_ = 768  # already a multiple of the 256 contraction tile
    folded = 2 * 128 * 128 * 2 + 2 * 128 * 4  # folded output weights and biases
    assert lib.bioemu_trimul_workspace_bytes(1, n, 128) == 3 * 128 * np_ * np_ * 2 + folded
    assert lib.bioemu_trimul_workspace_bytes(0, n, 128) == 0
    # folded fc1 | fc2 ([1024][128] bf16) and their bias pairs ([1024][2] bf16)
    assert lib.bioemu_transition_pair_workspace_bytes(128, 512) == 1024 * 128 * 2 + 1024 * 4
    assert lib.bioemu_transition_pair_workspace_bytes(64, 256) == 512 * 64 * 2 + 512 * 4
    assert lib.bioemu_transition_pair_workspace_bytes(64, 128) == 256 * 64 * 2 + 256 * 4
    assert lib.bioemu_transition_pair_workspace_bytes(128, 384) == 0
    assert lib.bioemu_transition_pair_workspace_bytes(384, 1536) == 0


def test_invalid_arguments_rejected_without_gpu():
    """Argument validation runs on the host before any launch."""
    lib = _lib.lib()
    rc = lib.bioemu_trimul_fwd(*([None] * 12), None, 0, 1, 16, 128, 1, 0, None)
    assert rc == -1
    assert b"null" in lib.bioemu_last_error()
    rc = lib.bioemu_trimul_fwd(*([None] * 12), None, 0, 1, 16, 64, 1, 0, None)
    assert rc == -2


def test_integration_doc_argtypes_match_binding():
    """Every `lib.<entry>.argtypes = ...` line of the integration guide at the repository root declares the
    binding's signature."""
    text = (ROOT / "INTEGRATION.md").read_text().replace("\\\n", " ")
    found = re.findall(r"lib\.(bioemu_\w+)\.argtypes\s*=\s*([^\n]+)", text)
    assert found
    for name, expr in found:
        got = eval(expr, {"ctypes": ctypes})   # the document's own expression, ctypes only
        assert got == _lib.SIGNATURES[name][1], (name, got)
