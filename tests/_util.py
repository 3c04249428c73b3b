"""Shared helpers of the test-suite (not a test module)."""

from __future__ import annotations

import numpy as np
import torch

from bpdecode_amd.ops import FsaTensors
from bpdecode_amd.tokenizer import Vocabulary
from oracle import dense as OD

TOY_VOCAB = Vocabulary.from_tokens(
    ["a", "b", "c", "ab", "ba", "0", "1", "12", "-", ".", "aa", "", "caf", "\xc3", "\xe9", "é", "<eos>"],
    eos_id=16,
)
TOY_PATTERNS = ["[01]+", "a+b*", "(ab)+", "-?[0-9]+(\\.[0-9]+)?", "a|bc|12", "[a-c]*", "caf(e|é)"]

PDA_VOCAB = Vocabulary.from_tokens(
    ["(", ")", "x", "y", "{", "}", "a", "b", ":", "0", "1", ",", "<eos>", "((", "x)", "", "{a", ":0,",
     "\"", "[1", "[", "]", "tr", "ue", "nul", "l", "-", "2.5", "e9", " ", "\"ab\"", "\\n"],
    eos_id=12,
)


def oracle_table(fsa: FsaTensors) -> np.ndarray:
    """tok_next from the oracle's restatement of build_token_transitions."""
    return OD.build_token_transitions(
        fsa.trans.cpu().numpy(), fsa.accept.cpu().numpy(), fsa.live.cpu().numpy(), fsa.num_symbols,
        fsa.offsets.cpu().numpy(), fsa.symbols.cpu().numpy(), fsa.eos_id,
    )


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.cpu().contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32).numpy().copy()


def reachable(tok_next: np.ndarray, start: int) -> list[int]:
    seen, todo = {start}, [start]
    while todo:
        for d in np.unique(tok_next[todo.pop()]):
            if d >= 0 and int(d) not in seen:
                seen.add(int(d))
                todo.append(int(d))
    return sorted(seen)
