"""ctypes binding of ``libbpdecode_hip.so`` (the C ABI in include/bpdecode_hip.h).

Loading is lazy and strict: if the library is missing or stale the first
operator call raises, naming the build step; nothing falls back to another
implementation.  Error codes become exceptions the way the reference's
torch ops raise them: an out-of-range index is an :class:`IndexError`,
anything else a :class:`RuntimeError`.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libbpdecode_hip.so"
ABI_VERSION = 9

OK, ERR_INVALID, ERR_HIP, ERR_OVERFLOW, ERR_UNSUPPORTED = 0, 1, 2, 3, 4
DTYPE_F32, DTYPE_F16, DTYPE_BF16, DTYPE_F64 = 0, 1, 2, 3
INDEX_I32, INDEX_I64, INDEX_I64_LOW32 = 0, 1, 2
MAX_FUSED_PENDING = 256  # BPD_MAX_FUSED_PENDING
FLAG_STATE_RANGE, FLAG_TOKEN_RANGE = 1, 2
PDA_MAX_CONFIGS = 8
PDA_MAX_DEPTH = 32
PDA_CONFIG_WORDS = 2 + PDA_MAX_CONFIGS + PDA_MAX_CONFIGS * PDA_MAX_DEPTH
SOFT_MEMBER_CHUNK, SOFT_MEMBER_CAP_MAX = 4096, 1024  # BPD_SOFT_MEMBER_CHUNK / _CAP_MAX
SOFT_PRIOR_SCRATCH_BYTES = 16 << 20  # BPD_SOFT_PRIOR_SCRATCH_BYTES

_DTYPE_CODE = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}
_DENSE_DTYPE_CODE = {**_DTYPE_CODE, torch.float64: DTYPE_F64}
_INDEX_CODE = {torch.int32: INDEX_I32, torch.int64: INDEX_I64}

vp, i32, i64, f64, f32, sz = C.c_void_p, C.c_int32, C.c_int64, C.c_double, C.c_float, C.c_size_t
cint = C.c_int


class PdaTableC(C.Structure):
    _fields_ = [
        ("num_states", i32), ("root_start", i32), ("root_accept", i32), ("num_edges", i32),
        ("accept", vp), ("live", vp), ("edge_offsets", vp), ("edge_kind", vp),
        ("edge_lo", vp), ("edge_hi", vp), ("edge_dst", vp), ("edge_callee", vp),
    ]


class PdaFramesC(C.Structure):
    _fields_ = [("num_lists", i32), ("words", i32), ("keys", vp), ("slots", vp), ("trans", vp),
                ("allowed", vp), ("seed_off", vp), ("seeds", vp)]


class TokenBytesC(C.Structure):
    _fields_ = [("vocab_size", i32), ("eos_id", i32), ("offsets", vp), ("bytes", vp), ("order", vp),
                ("runs", vp), ("frames", C.POINTER(PdaFramesC)), ("pack_tag", C.c_uint64)]


class FsaTableC(C.Structure):
    _fields_ = [
        ("trans", vp), ("num_states", i32), ("num_symbols", i32), ("dead", i32),
        ("accept", vp), ("live", vp), ("tok_offsets", vp), ("tok_symbols", vp),
        ("vocab", i64), ("eos_id", i32), ("trans16", vp), ("tok_records", vp),
    ]


class SoftClassesC(C.Structure):
    _fields_ = [
        ("num_classes", i32), ("num_members", i32), ("num_pieces", i32), ("num_pairs", i32),
        ("class_off", vp), ("class_tok", vp), ("class_piece", vp), ("piece_off", vp),
        ("state_off", vp), ("pair_class", vp), ("pair_next", vp), ("token_class", vp),
        ("token_class16", vp), ("chunk_members", vp), ("chunk_cap", i32),
    ]


_SIGNATURES = {
    "bpd_last_error": (C.c_char_p, []),
    "bpd_abi_version": (cint, []),
    "bpd_dense_apply_mask": (cint, [vp, cint, i64, i64, i64, vp, i32, vp, vp, vp, i64, f64, vp, vp]),
    "bpd_dense_apply_mask_bits": (cint, [vp, cint, i64, i64, i64, vp, i64, i32, vp, vp, vp, i64, f64,
                                         vp, vp]),
    "bpd_dense_advance": (cint, [vp, i32, i64, vp, vp, vp, i64, vp, cint, i64, vp, cint, vp, vp]),
    "bpd_dense_compute_mask": (cint, [vp, i32, i64, vp, vp, i64, vp, vp, vp]),
    "bpd_build_reachability": (cint, [vp, i32, i32, vp, vp, vp]),
    "bpd_host_build_reachability": (cint, [vp, i32, i32, vp, vp]),
    "bpd_build_tok_next": (cint, [vp, i32, i32, i32, vp, vp, vp, vp, i64, i32, vp, i32, vp, vp]),
    "bpd_fsa_apply_mask": (cint, [C.POINTER(FsaTableC), vp, cint, i64, i64, vp, vp, f64, vp, vp]),
    "bpd_fsa_compute_mask": (cint, [C.POINTER(FsaTableC), vp, vp, i64, vp, vp, vp]),
    "bpd_fsa_advance": (cint, [C.POINTER(FsaTableC), vp, vp, vp, i64, vp, cint, i64, vp, cint, vp,
                                vp]),
    "bpd_host_dense_apply_mask": (cint, [vp, cint, i64, i64, i64, vp, i32, vp, vp, f64]),
    "bpd_host_dense_apply_mask_bits": (cint, [vp, cint, i64, i64, i64, vp, i64, i32, vp, vp, f64]),
    "bpd_host_dense_advance": (cint, [vp, i32, i64, vp, vp, vp, cint, i64, vp, cint]),
    "bpd_host_dense_compute_mask": (cint, [vp, i32, i64, vp, vp, i64, vp]),
    "bpd_host_build_tok_next": (cint, [vp, i32, i32, i32, vp, vp, vp, vp, i64, i32, vp, i32, vp]),
    "bpd_stage_int64": (cint, [vp, vp, i64, vp]),
    "bpd_pda_init": (cint, [C.POINTER(PdaTableC), vp]),
    "bpd_pda_feed": (cint, [C.POINTER(PdaTableC), vp, C.c_char_p, i64]),
    "bpd_host_frame_classify": (cint, [vp, i32, vp, vp, i32, i32, vp, vp, vp, vp, vp, i32]),
    "bpd_host_frame_lists": (cint, [C.POINTER(PdaTableC), i32, vp, vp, vp]),
    "bpd_frame_classify": (cint, [vp, i32, vp, vp, i32, i32, vp, vp, vp, vp, vp, vp]),
    "bpd_frame_classify_blocks": (i32, [i32]),
    "bpd_pda_workspace_bytes": (sz, [i64, i32]),
    "bpd_pda_apply_mask": (cint, [C.POINTER(PdaTableC), C.POINTER(TokenBytesC), vp, vp, vp,
                                  i64, vp, cint, i64, f64, vp, sz, vp]),
    "bpd_pda_compute_mask": (cint, [C.POINTER(PdaTableC), C.POINTER(TokenBytesC), vp, vp, i64,
                                    vp, vp, sz, vp]),
    "bpd_pda_advance": (cint, [C.POINTER(PdaTableC), C.POINTER(TokenBytesC), vp, vp, vp, cint,
                               i64, vp, vp, vp, vp, vp, sz, vp]),
    "bpd_host_pda_apply_mask": (cint, [C.POINTER(PdaTableC), C.POINTER(TokenBytesC), vp, vp, vp,
                                       i64, vp, cint, i64, f64]),
    "bpd_host_pda_compute_mask": (cint, [C.POINTER(PdaTableC), C.POINTER(TokenBytesC), vp, vp,
                                         i64, vp]),
    "bpd_host_pda_advance": (cint, [C.POINTER(PdaTableC), C.POINTER(TokenBytesC), vp, vp, vp,
                                    cint, i64, vp, vp, vp]),
    "bpd_soft_workspace_bytes": (sz, [i64, i32, i32]),
    "bpd_soft_build_lookahead": (cint, [vp, i32, i64, vp, vp, i32, i32, vp, vp, sz, vp]),
    "bpd_soft_apply": (cint, [vp, cint, i64, i64, i64, vp, i32, vp, vp, f32, vp, vp]),
    "bpd_host_soft_classes": (cint, [vp, i32, i64, C.POINTER(SoftClassesC)]),
    "bpd_soft_prior_workspace_bytes": (sz, [i64, i64, i32, i32]),
    "bpd_soft_prior": (cint, [vp, i64, i64, i64, i32, vp, vp, i32, vp, vp, C.POINTER(SoftClassesC),
                              i32, f32, vp, sz, vp, vp]),
    "bpd_soft_prior_noalloc": (cint, [vp, i64, i64, i64, i32, vp, vp, i32, vp, vp,
                                      C.POINTER(SoftClassesC), i32, f32, vp, vp]),
    "bpd_host_soft_prior": (cint, [vp, i64, i64, i64, vp, i32, vp, vp, i32, vp, vp, i32, f32]),
    "bpd_host_soft_build_lookahead": (cint, [vp, i32, i64, vp, vp, i32, i32, vp]),
    "bpd_host_soft_apply": (cint, [vp, cint, i64, i64, i64, vp, i32, vp, vp, f32]),
}

_lib = None


def lib():
    """The loaded library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m bpdecode_amd.build` "
                "(or __graft_entry__.build())"
            )
        handle = C.CDLL(str(LIB_PATH), mode=C.RTLD_GLOBAL)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        got = handle.bpd_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name} ABI {got} != expected {ABI_VERSION}; rebuild it")
        _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(rc: int) -> None:
    if rc == OK:
        return
    msg = lib().bpd_last_error().decode(errors="replace")
    if rc == ERR_INVALID and msg.startswith("index "):
        raise IndexError(msg)
    raise RuntimeError(msg)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype, dense: bool = False) -> int:
    """Logits dtype code; ``dense`` admits float64 (the tok_next mask only)."""
    code = (_DENSE_DTYPE_CODE if dense else _DTYPE_CODE).get(dt)
    if code is None:
        names = "float32, float16, bfloat16" + (", float64" if dense else "")
        raise RuntimeError(f"logits dtype {dt} is not supported ({names})")
    return code


def index_code(dt: torch.dtype, low32: bool = False) -> int:
    """Token dtype code; ``low32`` reads int64 ids as their low 32 bits (the
    ``tokens.to(torch.int32)`` the reference's batch classes apply)."""
    code = _INDEX_CODE.get(dt)
    if code is None:
        raise RuntimeError(f"token ids must be int32 or int64, got {dt}")
    return INDEX_I64_LOW32 if (low32 and code == INDEX_I64) else code


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


def on_device(t: torch.Tensor) -> bool:
    return t.device.type == "cuda"


def debug_checks() -> bool:
    return os.environ.get("BPDECODE_CHECK", "0") not in ("", "0")
