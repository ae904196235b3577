"""Byte-level tokenizer: one token per UTF-8 byte plus BOS/EOS/PAD
(vllmlite/tokenizer.py:9-59). The HuggingFace tokenizer of the reference
downloads by name and is not available offline; `get_tokenizer` raises for it."""

from __future__ import annotations

from typing import List, Tuple

BOS = 256
EOS = 257
PAD = 258
VOCAB_SIZE = 261


class ByteTokenizer:
    bos_id = BOS
    eos_id = EOS
    pad_id = PAD
    vocab_size = VOCAB_SIZE
    name = "byte"

    def encode(self, text: str, add_bos: bool = True) -> List[int]:
        ids = list(text.encode("utf-8"))
        return [BOS] + ids if add_bos else ids

    def decode(self, ids: List[int]) -> str:
        return bytes(i for i in ids if i < 256).decode("utf-8", errors="replace")

    def decode_stream(self, ids: List[int], already: int) -> Tuple[str, int]:
        """Decode ids[already:], holding back an unfinished multi-byte UTF-8
        character (tokenizer.py:28-58). Returns (text_delta, new_already)."""
        tail = ids[already:]
        raw = bytes(i for i in tail if i < 256)
        if not raw:
            return "", len(ids)
        cut = len(raw)
        for back in range(1, min(4, len(raw)) + 1):
            b = raw[-back]
            if b < 0x80:
                break
            if b >= 0xC0:
                need = 2 if b < 0xE0 else 3 if b < 0xF0 else 4
                if back < need:
                    cut = len(raw) - back
                break
        text = raw[:cut].decode("utf-8", errors="replace")
        consumed = used = 0
        for tid in tail:
            if consumed >= cut:
                break
            if tid < 256:
                consumed += 1
            used += 1
        return text, already + used


def get_tokenizer(name=None):
    if not name or name == "byte":
        return ByteTokenizer()
    raise ValueError(f"tokenizer {name!r} needs a download; only the byte tokenizer is available")
