"""The C-ABI library loads and exports every function include/bpdecode_hip.h
declares (no device calls)."""

from __future__ import annotations

import re
import subprocess
from pathlib import Path

from bpdecode_amd import _lib

ROOT = Path(__file__).resolve().parent.parent


def declared() -> set[str]:
    text = (ROOT / "include" / "bpdecode_hip.h").read_text()
    return set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(bpd_\w+)\s*\(", text, re.M))


def test_header_declarations_are_exported():
    names = declared()
    assert len(names) >= 20
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (bpd_\w+)", out))
    assert names <= exported, sorted(names - exported)


def test_every_declaration_has_a_binding():
    lib = _lib.lib()
    assert lib.bpd_abi_version() == _lib.ABI_VERSION
    for name in declared():
        assert name in _lib._SIGNATURES, name
        assert getattr(lib, name) is not None


def test_error_path_reports_message():
    import torch

    with __import__("pytest").raises(RuntimeError, match="overflow"):
        _lib.check(_lib.lib().bpd_host_dense_apply_mask(
            torch.zeros(1, 1, dtype=torch.float16).data_ptr(), _lib.DTYPE_F16, 1, 1, 1,
            torch.zeros(1, 1, dtype=torch.int32).data_ptr(), 1,
            torch.zeros(1, dtype=torch.int32).data_ptr(), None, -1e9))
