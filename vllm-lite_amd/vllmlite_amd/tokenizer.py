"""Byte-level tokenization: one token per UTF-8 byte, then the specials BOS
256, EOS 257 and PAD 258 in a 261-entry vocabulary (the ids the reference's
model and workload use, vllmlite/tokenizer.py:9-22).

Streaming detokenization keeps one incremental UTF-8 decoder per request:
each step feeds that step's new byte tokens (specials are dropped) and gets
back the text they complete; a multi-byte character split across steps is
held inside the decoder until its last byte arrives. The HuggingFace
tokenizer of the reference loads by model name from the network and is not
available offline.
"""

from __future__ import annotations

import codecs
from typing import List

BOS = 256
EOS = 257
PAD = 258
VOCAB_SIZE = 261

_Utf8 = codecs.getincrementaldecoder("utf-8")
_BYTE = [bytes((i,)) for i in range(256)]


class ByteTokenizer:
    bos_id = BOS
    eos_id = EOS
    pad_id = PAD
    vocab_size = VOCAB_SIZE
    name = "byte"

    def encode(self, text: str, add_bos: bool = True) -> List[int]:
        body = list(text.encode("utf-8"))
        return [BOS, *body] if add_bos else body

    def decode(self, ids: List[int]) -> str:
        return bytes(t for t in ids if t < 256).decode("utf-8", errors="replace")

    def stream_decoder(self):
        """A callable new_ids -> text completed by them."""
        dec = _Utf8(errors="replace")

        def feed(new: List[int]) -> str:
            if len(new) == 1:  # a decode step's one token
                t = new[0]
                return dec.decode(_BYTE[t]) if 0 <= t < 256 else ""
            return dec.decode(bytes(t for t in new if t < 256))
        return feed


def get_tokenizer(name=None):
    if not name or name == "byte":
        return ByteTokenizer()
    raise ValueError(f"tokenizer {name!r} loads from the network; only the byte tokenizer "
                     "is available")
