"""Per-sequence constraint interface (interface.py of the reference)."""

from __future__ import annotations

import math
from abc import ABC, abstractmethod
from typing import Protocol, runtime_checkable

NEG_INF = -math.inf


@runtime_checkable
class Constraint(Protocol):
    @property
    def vocab_size(self) -> int: ...

    def reset(self) -> None: ...

    def accepts(self, token_id: int) -> bool: ...

    def advance(self, token_id: int) -> None: ...

    def is_complete(self) -> bool: ...

    def fill_mask(self, out) -> None: ...


class BaseConstraint(ABC):
    """Mask helpers shared by the per-sequence constraints."""

    @property
    @abstractmethod
    def vocab_size(self) -> int: ...

    @abstractmethod
    def reset(self) -> None: ...

    @abstractmethod
    def accepts(self, token_id: int) -> bool: ...

    @abstractmethod
    def advance(self, token_id: int) -> None: ...

    @abstractmethod
    def is_complete(self) -> bool: ...

    @abstractmethod
    def allowed_ids(self) -> frozenset[int]: ...

    def fill_mask(self, out) -> None:
        allowed = self.allowed_ids()
        for i in range(len(out)):
            out[i] = i in allowed

    def apply_(self, scores):
        allowed = self.allowed_ids()
        for i in range(len(scores)):
            if i not in allowed:
                scores[i] = NEG_INF
        return scores

    def __call__(self, input_ids, scores):
        import torch

        if isinstance(scores, torch.Tensor):
            allowed = self.allowed_ids()
            block = torch.ones(scores.shape[1], dtype=torch.bool, device=scores.device)
            if allowed:
                block[torch.tensor(sorted(allowed), device=scores.device)] = False
            for row in range(scores.shape[0]):
                scores[row][block] = NEG_INF
            return scores
        for row in scores:
            self.apply_(row)
        return scores
