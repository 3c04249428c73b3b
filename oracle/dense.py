"""TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

numpy restatement of the reference's dense tok_next path:

* :func:`build_token_transitions`  ops.py:143-197 (== fsa.step entry for entry,
  fsa.py:155-174): walk each token's symbol classes from each start state;
  ``-1`` when the end state is not live (the absorbing dead state is never
  live); EOS column ``s`` for accepting ``s`` else ``-1``.
* :func:`apply_mask_bits`  ops.py:271-276: an entry is rejected iff the row's
  state is negative or ``tok_next[state, t] == -1``; rejected entries take the
  fill value's bit pattern, others keep their bits.
* :func:`advance`  ops.py:301-306: ``-1`` for a negative state else
  ``tok_next[state, t]`` with torch's negative-index wrap; int64 ids index
  in full (``token_ids.long()``), or by their low 32 bits with ``low32``
  (the ``tokens.to(torch.int32)`` of batch.py:213 / device.py:278).
* :func:`compute_mask_bits`  packed LSB-first allow bits.
The fill value's bit pattern is taken from ATen's own scalar conversion (the
reference's masked_fill_ arithmetic), including its overflow error.
"""

from __future__ import annotations

import numpy as np
import torch

_TORCH_BITS = {torch.float32: (torch.int32, np.uint32), torch.float16: (torch.int16, np.uint16),
               torch.bfloat16: (torch.int16, np.uint16), torch.float64: (torch.int64, np.uint64)}


def fill_bits(dtype: torch.dtype, value: float) -> int:
    """Bit pattern ATen stores for ``value`` in a ``dtype`` tensor."""
    ibits, npt = _TORCH_BITS[dtype]
    t = torch.zeros(1, dtype=dtype).masked_fill_(torch.ones(1, dtype=torch.bool), value)
    return int(t.view(ibits).numpy().astype(npt)[0])


def build_token_transitions(trans, accept, live, num_symbols, offsets, symbols, eos_id, rows=None):
    trans = np.asarray(trans, dtype=np.int64)
    accept = np.asarray(accept, dtype=bool)
    live = np.asarray(live, dtype=bool)
    offsets = np.asarray(offsets, dtype=np.int64)
    symbols = np.asarray(symbols, dtype=np.int64)
    S = accept.size
    V = offsets.size - 1
    starts = np.arange(S, dtype=np.int64) if rows is None else np.asarray(rows, dtype=np.int64)
    lengths = offsets[1:] - offsets[:-1]
    cur = np.repeat(starts[:, None], V, axis=1)
    for k in range(int(lengths.max()) if V else 0):
        active = np.nonzero(lengths > k)[0]
        sym = symbols[offsets[active] + k]
        cur[:, active] = trans[cur[:, active] * num_symbols + sym[None, :]]
    out = np.where(live[cur], cur, -1).astype(np.int32)
    if eos_id is not None and 0 <= eos_id < V:
        out[:, eos_id] = np.where(accept[starts], starts, -1)
    return out


def apply_mask_bits(logit_bits: np.ndarray, tok_next: np.ndarray, states, fill: int) -> np.ndarray:
    s = np.asarray(states, dtype=np.int64)
    rejected = tok_next[np.clip(s, 0, None)] == -1
    rejected |= (s < 0)[:, None]
    logit_bits[rejected] = fill
    return logit_bits


def apply_mask(logits: torch.Tensor, tok_next, states, neg_inf: float = float("-inf")) -> torch.Tensor:
    """In place on a CPU tensor via its raw bits."""
    ibits, npt = _TORCH_BITS[logits.dtype]
    fill = fill_bits(logits.dtype, neg_inf)
    bits = logits.view(ibits).numpy().view(npt)
    apply_mask_bits(bits, np.asarray(tok_next), np.asarray(states), fill)
    return logits


def advance(tok_next: np.ndarray, states, tokens, low32: bool = True) -> np.ndarray:
    s = np.asarray(states, dtype=np.int64)
    t = np.asarray(tokens)
    t = (t.astype(np.int32) if low32 else t).astype(np.int64)
    V = tok_next.shape[1]
    if t.size and (t.max() >= V or t.min() < -V):
        raise IndexError("token index out of range")
    t = np.where(t < 0, t + V, t)
    nxt = tok_next[np.clip(s, 0, None), t]
    return np.where(s < 0, -1, nxt).astype(np.int32)


def compute_mask_bits(tok_next: np.ndarray, states) -> np.ndarray:
    s = np.asarray(states, dtype=np.int64)
    allowed = (tok_next[np.clip(s, 0, None)] != -1) & (s >= 0)[:, None]
    B, V = allowed.shape
    W = (V + 31) // 32
    pad = np.zeros((B, W * 32), dtype=np.uint64)
    pad[:, :V] = allowed
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    return (pad.reshape(B, W, 32) * weights).sum(axis=2).astype(np.uint32)
