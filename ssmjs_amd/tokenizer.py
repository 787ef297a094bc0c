"""Pluggable tokenizer contract (src/session/tokenizer.ts:11-18) and a byte-level stub.

The reference's default BPETokenizer downloads Qwen2.5-Coder vocab files over the network
(session.ts:26-27,341-343); this backend takes an injected tokenizer instead, as the
reference allows through MambaSessionOptions.tokenizer (session.ts:326-334).
"""
from __future__ import annotations

from typing import List, Protocol


class Tokenizer(Protocol):
    vocabSize: int

    def encode(self, text: str) -> List[int]: ...

    def decode(self, tokens: List[int]) -> str: ...


class ByteTokenizer:
    """UTF-8 bytes as ids 0..255, padded up to `vocab_size` ids (ids >= 256 decode to '')."""

    def __init__(self, vocab_size: int = 256):
        if vocab_size < 256:
            raise ValueError("ByteTokenizer needs vocab_size >= 256")
        self.vocabSize = vocab_size

    def encode(self, text: str) -> List[int]:
        return list(text.encode("utf-8"))

    def decode(self, tokens: List[int]) -> str:
        return bytes(t for t in tokens if 0 <= t < 256).decode("utf-8", errors="replace")
