"""bpdecode_amd -- the batched constrained-decoding step of bpdecode, built for
AMD Instinct MI355X (gfx950).

The public API mirrors the reference package: ``batch`` (ConstraintBatch,
GrammarCache, MaskCache), ``ops`` (FsaTensors and the mask / commit / soft
operators), ``grammar`` (GBNF, JSON Schema, the device PDA and
CFGConstraintBatch), ``hf`` / ``vllm`` adapters, and the host front-end
(regex -> DFA, vocabularies).  All per-step computation runs in
``libbpdecode_hip.so``.  The reference's per-sequence CPU constraints
(RegexConstraint, TokenDFA, CFGConstraint and its unbounded PDA) are not part
of this build: the batch classes serve CPU tensors through the library's host
entry points.
"""

from __future__ import annotations

from .fsa import (
    FsaTable,
    TokenSymbols,
    advance_state_batch,
    apply_mask,
    build_reachability,
    compute_mask,
    fsa_from_dfa,
    step,
    token_symbols,
)
from .regex import DFA, RegexSyntaxError, compile_regex
from .tokenizer import DEFAULT_MODEL, Vocabulary

__version__ = "0.1.0"

__all__ = [
    "DEFAULT_MODEL", "DFA", "FsaTable", "RegexSyntaxError", "TokenSymbols", "Vocabulary",
    "advance_state_batch",
    "apply_mask", "build_reachability", "compile_regex", "compute_mask", "fsa_from_dfa", "step",
    "token_symbols", "__version__",
]
