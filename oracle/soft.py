"""TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

float64 numpy restatement of the soft lookahead:

* :func:`build_lookahead`  ops.py:200-236 (uniform counts):
  ``logZ_0 = 0`` on live states else ``-inf``;
  ``logZ_{j+1}(s) = logsumexp_t logZ_j(tok_next[s, t])`` (``logaddexp(., 0)``
  for accepting ``s``), ``-inf`` off the live set; ``k-1`` rounds;
  ``out[s, t] = logZ_{k-1}(tok_next[s, t])``, ``-inf`` on rejected tokens,
  EOS column 0 for accepting ``s`` else ``-inf``.
* :func:`apply_soft`  ops.py:239-259.
* :func:`prior_lookahead`  the per-row model-prior variant: with
  ``logpi_b = log_softmax(logits_b)``,
  ``logZ_{j+1,b}(s) = logsumexp_t [logpi_b(t) + logZ_{j,b}(tok_next[s, t])]
  ⊕ [accept s] logpi_b(eos)`` and
  ``out[b, t] = logpi_b(t) + alpha * logZ_{k-1,b}(tok_next[s_b, t])`` on
  allowed tokens (EOS: ``logpi_b(eos)`` when ``s_b`` accepts), ``-inf``
  elsewhere.  With ``logpi == 0`` the recurrence is exactly the uniform one.
* :func:`prior_lookahead_torch`  the same prior variant as an fp32 torch
  program on CPU tensors, op for op the reference's build_lookahead /
  apply_soft_ sequence (ops.py:200-259: an ``[S, V]`` gather of ``logZ``
  through ``tok_next``, ``logsumexp`` over the vocabulary, ``logaddexp`` for
  accepting states) with the row's log-softmax added to every gathered
  term: the timed CPU baseline of the prior lookahead.
"""

from __future__ import annotations

import numpy as np
from scipy.special import logsumexp

NEG = -np.inf


def _gather(logz: np.ndarray, tn: np.ndarray) -> np.ndarray:
    return np.where(tn >= 0, logz[np.clip(tn, 0, None)], NEG)


def build_lookahead(tok_next, live, accept, eos, k):
    tn = np.asarray(tok_next, dtype=np.int64)
    live = np.asarray(live, dtype=bool)
    accept = np.asarray(accept, dtype=bool)
    S, V = tn.shape
    logz = np.where(live, 0.0, NEG)
    for _ in range(max(k - 1, 0)):
        with np.errstate(divide="ignore"):
            nxt = logsumexp(_gather(logz, tn), axis=1)
        nxt = np.where(accept, np.logaddexp(nxt, 0.0), nxt)
        logz = np.where(live, nxt, NEG)
    out = _gather(logz, tn)
    if eos is not None and 0 <= eos < V:
        out[:, eos] = np.where(accept, 0.0, NEG)
    return out


def apply_soft(logits: np.ndarray, lookahead: np.ndarray, states, alpha: float) -> np.ndarray:
    s = np.asarray(states, dtype=np.int64)
    bias = lookahead[np.clip(s, 0, None)].copy()
    bias[s < 0] = NEG
    dis = np.isneginf(bias)
    out = logits.astype(np.float64).copy()
    if alpha != 0.0:
        out += alpha * np.where(dis, 0.0, bias)
    out[dis] = NEG
    return out


def prior_lookahead(logits, tok_next, live, accept, eos, states, k, alpha):
    x = np.asarray(logits, dtype=np.float64)
    tn = np.asarray(tok_next, dtype=np.int64)
    live = np.asarray(live, dtype=bool)
    accept = np.asarray(accept, dtype=bool)
    S, V = tn.shape
    logpi = x - logsumexp(x, axis=1, keepdims=True)
    out = np.full_like(logpi, NEG)
    for b, s in enumerate(np.asarray(states, dtype=np.int64)):
        lp = logpi[b]
        logz = np.where(live, 0.0, NEG)
        for _ in range(max(k - 1, 0)):
            with np.errstate(divide="ignore"):
                nxt = logsumexp(lp[None, :] + _gather(logz, tn), axis=1)
            if 0 <= eos < V:
                nxt = np.where(accept, np.logaddexp(nxt, lp[eos]), nxt)
            logz = np.where(live, nxt, NEG)
        if s < 0:
            continue
        row = _gather(logz, tn[s])
        out[b] = np.where(np.isneginf(row), NEG, lp + alpha * np.where(np.isneginf(row), 0.0, row))
        if 0 <= eos < V:
            out[b, eos] = lp[eos] if accept[s] else NEG
    return out


def prior_lookahead_torch(logits, tok_next, live, accept, eos, states, k, alpha, rows=None):
    """fp32 torch restatement of :func:`prior_lookahead` (see the module
    header); ``rows`` limits the work to those row indices (the others stay
    ``-inf``).  Returns a float32 CPU tensor."""
    import torch

    x = torch.as_tensor(logits, dtype=torch.float32)
    tn = torch.as_tensor(tok_next).long()
    live = torch.as_tensor(live).bool()
    accept = torch.as_tensor(accept).bool()
    S, V = tn.shape
    neg = torch.tensor(float("-inf"))
    rejected = tn < 0
    idx = tn.clamp(min=0)
    has_eos = eos is not None and 0 <= eos < V
    out = torch.full(x.shape, float("-inf"), dtype=torch.float32)
    st = torch.as_tensor(states).long()
    for b in (range(x.shape[0]) if rows is None else rows):
        lp = torch.log_softmax(x[b], dim=0)
        logz = torch.where(live, torch.zeros(S), neg.expand(S))
        for _ in range(max(k - 1, 0)):
            cand = torch.where(rejected, neg, logz[idx] + lp)  # [S, V]
            nxt = torch.logsumexp(cand, dim=1)
            if has_eos:
                nxt = torch.where(accept, torch.logaddexp(nxt, lp[eos]), nxt)
            logz = torch.where(live, nxt, neg.expand(S))
        s = int(st[b])
        if s < 0:
            continue
        row = torch.where(rejected[s], neg, logz[idx[s]])
        dis = torch.isneginf(row)
        out[b] = torch.where(dis, neg, lp + alpha * row.masked_fill(dis, 0.0))
        if has_eos:
            out[b, eos] = lp[eos] if bool(accept[s]) else neg
    return out
