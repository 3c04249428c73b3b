"""``torch.ops.bpdecode.*``: the reference's operator schemas, re-registered
over ``libbpdecode_hip.so``.

The seven schemas are the strings of bindings/torch_ops.cpp:427-459 and keep
their argument meaning, dtype checks and in-place contracts (torch_ops.cpp:
109-229, 307-425); like the reference they are registered for
``CompositeExplicitAutograd`` and branch on the device internally.  Two dense
operators are added for the ``tok_next`` path: ``dense_apply_mask_`` and
``dense_advance_state``.  Device tensors run the HIP kernels on torch's
current stream; CPU tensors run the library's host entry points.  Importing
this module registers the operators (as importing ``bpdecode._C`` does).
"""

from __future__ import annotations

import torch

from . import ops
from ._lib import PDA_CONFIG_WORDS
from .grammar import device as _gdev

_SCHEMAS = (
    "build_reachability(Tensor trans, Tensor accept, int num_symbols) -> Tensor",
    "apply_mask_(Tensor(a!) logits, Tensor trans, Tensor accept, Tensor live, int num_symbols, "
    "int dead, Tensor offsets, Tensor symbols, int eos_id, Tensor states, float neg_inf) "
    "-> Tensor(a!)",
    "compute_mask(Tensor trans, Tensor accept, Tensor live, int num_symbols, int dead, "
    "Tensor offsets, Tensor symbols, int eos_id, Tensor states) -> Tensor",
    "advance_state(Tensor trans, Tensor accept, Tensor live, int num_symbols, int dead, "
    "Tensor offsets, Tensor symbols, int eos_id, Tensor states, Tensor token_ids) -> Tensor",
    "pda_init(Tensor accept, Tensor live, Tensor edge_offsets, Tensor edge_kind, "
    "Tensor edge_lo, Tensor edge_hi, Tensor edge_dst, Tensor edge_callee, int root_start, "
    "int root_accept) -> Tensor",
    "pda_apply_mask_(Tensor(a!) logits, Tensor accept, Tensor live, Tensor edge_offsets, "
    "Tensor edge_kind, Tensor edge_lo, Tensor edge_hi, Tensor edge_dst, Tensor edge_callee, "
    "int root_start, int root_accept, Tensor tok_offsets, Tensor tok_bytes, int eos_id, "
    "Tensor configs, float neg_inf) -> Tensor(a!)",
    "pda_advance_state(Tensor(a!) configs, Tensor accept, Tensor live, Tensor edge_offsets, "
    "Tensor edge_kind, Tensor edge_lo, Tensor edge_hi, Tensor edge_dst, Tensor edge_callee, "
    "int root_start, int root_accept, Tensor tok_offsets, Tensor tok_bytes, int eos_id, "
    "Tensor token_ids) -> Tensor",
    "dense_apply_mask_(Tensor(a!) logits, Tensor tok_next, Tensor states, float neg_inf) "
    "-> Tensor(a!)",
    "dense_advance_state(Tensor tok_next, Tensor states, Tensor tokens) -> Tensor",
)

_KEY = "CompositeExplicitAutograd"


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


# grammar bundles are long-lived: wrap (and, for the walking kernels, merge
# the symbol classes of) each one once, keyed by the identity and version of
# its tensors
_FSA_CACHE: dict = {}
_PDA_CACHE: dict = {}


def _tensor_key(*parts) -> tuple:
    return tuple((p.data_ptr(), p.numel(), p.dtype, p.device, p._version) if p is not None else None
                 for p in parts)


def _fsa(trans, accept, live, num_symbols, dead, offsets, symbols, eos_id) -> ops.FsaTensors:
    key = _tensor_key(trans, accept, live, offsets, symbols) + (int(num_symbols), int(dead), int(eos_id))
    hit = _FSA_CACHE.get(key)
    if hit is not None:
        return hit[0]
    fsa = ops.FsaTensors(
        trans=trans.to(torch.int32), accept=accept.to(torch.uint8), live=live.to(torch.uint8),
        num_symbols=int(num_symbols), dead=int(dead), offsets=offsets.to(torch.int32),
        symbols=symbols.to(torch.int32), eos_id=int(eos_id),
    )
    if len(_FSA_CACHE) > 64:
        _FSA_CACHE.clear()
    _FSA_CACHE[key] = (fsa, (trans, accept, live, offsets, symbols))
    return fsa


def _pda(accept, live, eo, ek, elo, ehi, ed, ec, root_start, root_accept,
         tok_offsets=None, tok_bytes=None, eos_id=-1) -> _gdev.PdaTensors:
    parts = (accept, live, eo, ek, elo, ehi, ed, ec, tok_offsets, tok_bytes)
    key = _tensor_key(*parts) + (int(root_start), int(root_accept), int(eos_id))
    hit = _PDA_CACHE.get(key)
    if hit is not None:
        return hit
    if tok_offsets is None:
        tok_offsets = torch.zeros(1, dtype=torch.int32, device=accept.device)
        tok_bytes = torch.zeros(0, dtype=torch.uint8, device=accept.device)
    g = _gdev.PdaTensors(
        num_states=int(accept.numel()), root_start=int(root_start), root_accept=int(root_accept),
        accept=accept.contiguous(), live=live.contiguous(), edge_offsets=eo.contiguous(),
        edge_kind=ek.contiguous(), edge_lo=elo.contiguous(), edge_hi=ehi.contiguous(),
        edge_dst=ed.contiguous(), edge_callee=ec.contiguous(),
        tok_offsets=tok_offsets.contiguous(), tok_bytes=tok_bytes.contiguous(),
        vocab_size=int(tok_offsets.numel() - 1), eos_id=int(eos_id),
    )
    g.c_table()  # validates the grammar arrays
    if len(_PDA_CACHE) > 64:
        _PDA_CACHE.clear()
    _PDA_CACHE[key] = g
    return g


def _pda_check_configs(configs: torch.Tensor) -> None:
    _check(configs.dtype == torch.int32, "configs must be int32")
    _check(configs.dim() == 2 and configs.size(1) == PDA_CONFIG_WORDS,
           f"configs must be [batch, {PDA_CONFIG_WORDS}]")
    _check(configs.is_contiguous(), "configs must be contiguous")


# --- FSA ops (torch_ops.cpp:95-229) --------------------------------------------
def build_reachability(trans, accept, num_symbols):
    """torch_ops.cpp:95-107 (host only there); device tensors run the
    reachability kernel."""
    return ops.build_reachability(trans, accept, int(num_symbols))


def apply_mask_(logits, trans, accept, live, num_symbols, dead, offsets, symbols, eos_id, states,
                neg_inf):
    _check(logits.dim() == 2 and logits.dtype == torch.float32, "logits must be float32 [batch, vocab]")
    _check(states.dtype == torch.int32, "states must be int32")
    _check(states.numel() == logits.size(0), "one state per logits row")
    _check(offsets.numel() - 1 == logits.size(1), "offsets imply a different vocab size")
    fsa = _fsa(trans, accept, live, num_symbols, dead, offsets, symbols, eos_id)
    return ops.apply_mask_(logits, fsa, states, float(neg_inf))


def compute_mask(trans, accept, live, num_symbols, dead, offsets, symbols, eos_id, states):
    fsa = _fsa(trans, accept, live, num_symbols, dead, offsets, symbols, eos_id)
    return ops.compute_mask(fsa, states)


def advance_state(trans, accept, live, num_symbols, dead, offsets, symbols, eos_id, states,
                  token_ids):
    _check(states.dtype == torch.int32 and token_ids.dtype == torch.int32,
           "states / token_ids must be int32")
    _check(token_ids.numel() == states.numel(), "one token id per state")
    fsa = _fsa(trans, accept, live, num_symbols, dead, offsets, symbols, eos_id)
    return ops.advance_state(fsa, states, token_ids)


# --- PDA ops (torch_ops.cpp:307-425) -------------------------------------------
def pda_init(accept, live, eo, ek, elo, ehi, ed, ec, root_start, root_accept):
    g = _pda(accept.cpu(), live.cpu(), eo.cpu(), ek.cpu(), elo.cpu(), ehi.cpu(), ed.cpu(), ec.cpu(),
             root_start, root_accept)
    return g.init_config().clone().to(accept.device)


def pda_apply_mask_(logits, accept, live, eo, ek, elo, ehi, ed, ec, root_start, root_accept,
                    tok_offsets, tok_bytes, eos_id, configs, neg_inf):
    _check(logits.dim() == 2 and logits.dtype == torch.float32, "logits must be float32 [batch, vocab]")
    _pda_check_configs(configs)
    _check(configs.size(0) == logits.size(0), "one config-set per logits row")
    g = _pda(accept, live, eo, ek, elo, ehi, ed, ec, root_start, root_accept, tok_offsets,
             tok_bytes, eos_id)
    _check(g.vocab_size == logits.size(1), "tok_offsets imply a different vocab size")
    return _gdev.pda_mask_(logits, g, configs, neg_inf=float(neg_inf))


def pda_advance_state(configs, accept, live, eo, ek, elo, ehi, ed, ec, root_start, root_accept,
                      tok_offsets, tok_bytes, eos_id, token_ids):
    _pda_check_configs(configs)
    _check(token_ids.dtype == torch.int32 and token_ids.numel() == configs.size(0),
           "token_ids must be int32, one per config-set")
    g = _pda(accept, live, eo, ek, elo, ehi, ed, ec, root_start, root_accept, tok_offsets,
             tok_bytes, eos_id)
    ok, _ = _gdev.pda_step(configs, g, token_ids)
    return ok


# --- dense ops (the tok_next branches of ops.py:271 and :301) --------------------
def dense_apply_mask_(logits, tok_next, states, neg_inf):
    return ops.dense_mask_(logits, tok_next, states, neg_inf=float(neg_inf))


def dense_advance_state(tok_next, states, tokens):
    return ops.dense_advance(tok_next, states, tokens)


_IMPLS = (build_reachability, apply_mask_, compute_mask, advance_state, pda_init, pda_apply_mask_,
          pda_advance_state, dense_apply_mask_, dense_advance_state)


def _register() -> torch.library.Library | None:
    if hasattr(torch.ops.bpdecode, "apply_mask_"):
        return None  # already registered in this process
    lib = torch.library.Library("bpdecode", "DEF")
    for schema, fn in zip(_SCHEMAS, _IMPLS):
        lib.define(schema)
        lib.impl(schema.split("(", 1)[0], fn, _KEY)
    return lib


_LIBRARY = _register()
