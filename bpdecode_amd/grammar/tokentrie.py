"""Byte trie of a vocabulary, walked against the host :class:`PDA`
(grammar/tokentrie.py of the reference): a depth-first walk feeds one byte per
edge and prunes a subtree as soon as the config-set empties."""

from __future__ import annotations

from ..tokenizer import Vocabulary


class _Node:
    __slots__ = ("children", "token_id")

    def __init__(self) -> None:
        self.children: dict[int, _Node] = {}
        self.token_id: int | None = None


class TokenTrie:
    def __init__(self, root: _Node, eos_id: int | None) -> None:
        self._root = root
        self._eos_id = eos_id

    @classmethod
    def build(cls, vocab: Vocabulary) -> TokenTrie:
        root = _Node()
        for tid, tb in enumerate(vocab.token_bytes):
            if tid == vocab.eos_id:
                continue
            node = root
            for b in tb:
                node = node.children.setdefault(b, _Node())
            node.token_id = tid
        return cls(root, vocab.eos_id)

    def allowed(self, pda) -> set[int]:
        out: set[int] = set()
        snap = pda.configs
        stack = [(self._root, snap)]
        while stack:
            node, cfgs = stack.pop()
            if node.token_id is not None:
                out.add(node.token_id)
            for b, child in node.children.items():
                pda.set_configs(cfgs)
                if pda.advance_byte(b):
                    stack.append((child, pda.configs))
        pda.set_configs(snap)
        if self._eos_id is not None and pda.is_complete():
            out.add(self._eos_id)
        return out


_CACHE: dict[int, TokenTrie] = {}


def token_trie(vocab: Vocabulary) -> TokenTrie:
    trie = _CACHE.get(id(vocab))
    if trie is None:
        trie = _CACHE[id(vocab)] = TokenTrie.build(vocab)
    return trie
