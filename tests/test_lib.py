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


def test_fsa_entry_points_validate_before_launching():
    """The walking-kernel entry points reject bad arguments on the host (no
    device call is made on these paths)."""
    import ctypes as C

    import torch

    lib = _lib.lib()
    trans = torch.zeros(4, dtype=torch.int32)
    u8 = torch.ones(2, dtype=torch.uint8)
    offs = torch.tensor([0, 1, 2], dtype=torch.int32)
    sym = torch.zeros(2, dtype=torch.uint8)
    ok = _lib.FsaTableC(trans.data_ptr(), 2, 2, 1, u8.data_ptr(), u8.data_ptr(), offs.data_ptr(),
                        sym.data_ptr(), 2, -1)
    st = torch.zeros(1, dtype=torch.int32)
    lg = torch.zeros(1, 2, dtype=torch.float16)
    # null table, unknown dtype, a fill value that overflows float16
    assert lib.bpd_fsa_apply_mask(None, lg.data_ptr(), _lib.DTYPE_F16, 1, 2, st.data_ptr(), None,
                                  0.0, None, None) != 0
    assert lib.bpd_fsa_apply_mask(C.byref(ok), lg.data_ptr(), 99, 1, 2, st.data_ptr(), None, 0.0,
                                  None, None) != 0
    assert "unknown logits dtype" in lib.bpd_last_error().decode()
    assert lib.bpd_fsa_apply_mask(C.byref(ok), lg.data_ptr(), _lib.DTYPE_F16, 1, 2, st.data_ptr(),
                                  None, -1e9, None, None) == _lib.ERR_OVERFLOW
    # a dead state outside the table and a short logits stride
    bad = _lib.FsaTableC(trans.data_ptr(), 2, 2, 5, u8.data_ptr(), u8.data_ptr(), offs.data_ptr(),
                         sym.data_ptr(), 2, -1)
    assert lib.bpd_fsa_compute_mask(C.byref(bad), st.data_ptr(), None, 1, None, None, None) != 0
    assert "dead state" in lib.bpd_last_error().decode()
    assert lib.bpd_fsa_apply_mask(C.byref(ok), lg.data_ptr(), _lib.DTYPE_F16, 1, 1, st.data_ptr(),
                                  None, 0.0, None, None) != 0
    # unknown token dtype; zero rows is a no-op that touches nothing
    assert lib.bpd_fsa_advance(C.byref(ok), st.data_ptr(), None, None, 0, st.data_ptr(), 7, 1,
                               st.data_ptr(), 0, None, None) != 0
    # queued writes need a slot map and write_back, and at most 256 per launch
    assert lib.bpd_fsa_advance(C.byref(ok), st.data_ptr(), None, st.data_ptr(), 1, st.data_ptr(),
                               _lib.INDEX_I32, 1, st.data_ptr(), 1, None, None) != 0
    assert "queued writes" in lib.bpd_last_error().decode()
    assert lib.bpd_fsa_advance(C.byref(ok), st.data_ptr(), st.data_ptr(), st.data_ptr(), 300,
                               st.data_ptr(), _lib.INDEX_I32, 1, st.data_ptr(), 1, None, None) != 0
    assert lib.bpd_fsa_apply_mask(C.byref(ok), None, _lib.DTYPE_F32, 0, 2, None, None, 0.0, None,
                                  None) == 0
    assert lib.bpd_fsa_advance(C.byref(ok), None, None, None, 0, None, _lib.INDEX_I32, 0, None, 0,
                               None, None) == 0
