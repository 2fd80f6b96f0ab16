"""CPU restatement of the request's text side. TEST INFRASTRUCTURE ONLY:
imported by tests, never by the product library.

- encode (protocol.mm:558-579; vendor tokenization_yue2.py:27-28): NFC by
  ``unicodedata.normalize``, pieces by the reference pattern run through the
  ``regex`` module, byte pair merges by tiktoken's published loop (join the
  adjacent pair whose concatenation has the lowest rank, leftmost first,
  until none is in the vocabulary; a piece in the vocabulary is one token).
  ``\\s`` / ``\\S`` are written out as ICU's class ``[\\t\\n\\f\\r\\p{Z}]``
  (the native reference's NSRegularExpression is ICU); the vendor path's
  tiktoken uses the White_Space property instead, which adds U+000B and
  U+0085 (``VENDOR_PATTERN``).
- decode (protocol.mm:580-591): pieces joined, ``bytes.decode(errors="replace")``.
- the prompt layout: instruction, SongRequest.text, token_prefixes,
  negative_prefix, guidance, chunk_ranges (protocol.mm:200-369; vendor
  protocol.py:104-145).
"""
from __future__ import annotations

import base64
import unicodedata

import regex

EOD, ABC_START, ABC_END, MUSIC_START = 151643, 151847, 151848, 151851

_S = r"[\t\n\f\r\p{Z}]"
_NS = r"[^\t\n\f\r\p{Z}]"
ICU_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}|"
               r" ?[^" + _S[1:-1] + r"\p{L}\p{N}]+[\r\n]*|" + _S + r"*[\r\n]+|" + _S + r"+(?!"
               + _NS + r")|" + _S + r"+")
VENDOR_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+"
                  r"[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")

INSTRUCTIONS = {
    "off": "Generate music with codec tokens from the given conditions.",
    "melody": "Generate a melody-only ABC transcription without chord symbols, then generate "
              "music with codec tokens from the given conditions.",
    "full": "Generate a chord-annotated ABC transcription, then generate music with codec "
            "tokens from the given conditions.",
}


def write_vocabulary(path, pieces):
    """A qwen.tiktoken file: one "base64(piece) rank" line per piece."""
    with open(path, "wb") as f:
        for rank, piece in enumerate(pieces):
            f.write(base64.b64encode(piece) + b" " + str(rank).encode() + b"\n")


def read_vocabulary(path):
    ranks = {}
    for line in open(path, "rb").read().splitlines():
        if line:
            piece, rank = line.split()
            ranks[base64.b64decode(piece)] = int(rank)
    return ranks


def pieces(text, pattern=ICU_PATTERN):
    """Pre-tokenizer pieces of NFC text (str)."""
    return regex.findall(pattern, text)


def bpe(word: bytes, ranks):
    if word in ranks:
        return [ranks[word]]
    parts = [word[i:i + 1] for i in range(len(word))]
    while len(parts) > 1:
        best, at = None, -1
        for i in range(len(parts) - 1):
            r = ranks.get(parts[i] + parts[i + 1])
            if r is not None and (best is None or r < best):
                best, at = r, i
        if best is None:
            break
        parts[at:at + 2] = [parts[at] + parts[at + 1]]
    return [ranks[p] for p in parts]


def encode(text: str, ranks, pattern=ICU_PATTERN):
    out = []
    for piece in pieces(unicodedata.normalize("NFC", text), pattern):
        out += bpe(piece.encode("utf-8"), ranks)
    return out


def decode(ids, ranks):
    inverse = {r: p for p, r in ranks.items()}
    specials = [b"<|endoftext|>", b"<|im_start|>", b"<|im_end|>", b"<R>", b"<S>", b"<X>",
                b"<mask>", b"<sep>"] + [b"<extra_%d>" % i for i in range(200)]
    specials[204:206] = [b"<abc>", b"</abc>"]
    for i, s in enumerate(specials):
        inverse[EOD + i] = s
    return b"".join(inverse[t] for t in ids if t in inverse).decode("utf-8", errors="replace")


def request_text(style, lyrics, cot):
    return f"{INSTRUCTIONS[cot]}\n[Tags]\n{style}\n[Lyrics]\n{lyrics}\n"


def token_prefixes(style, lyrics, cot, ranks, abc=None, abc_ids=None):
    base = [EOD] + encode(request_text(style, lyrics, cot), ranks)
    if cot == "off":
        return base + [ABC_START, ABC_END, MUSIC_START]
    if abc_ids is None:
        if abc is None:
            return base + [ABC_START]
        abc_ids = encode(abc, ranks)
    return base + [ABC_START] + list(abc_ids) + [ABC_END, MUSIC_START]


def negative_prefix(cot, ranks, abc_ids=None):
    base = [EOD] + encode(INSTRUCTIONS[cot], ranks)
    if cot == "off":
        return base + [MUSIC_START]
    return base + [ABC_START] + list(abc_ids) + [ABC_END, MUSIC_START]


CONTEXT = 24576


def chunk_ranges(frames, prefix_tokens, context=CONTEXT):
    """The acoustic stage's frame chunks (vendor protocol.py:141-145)."""
    size = min((context - prefix_tokens - 3) // 2, CONTEXT)
    if frames < 1 or size < 1:
        raise ValueError("Empty codec or prefix leaves no acoustic context")
    return [(a, min(a + size, frames)) for a in range(0, frames, size)]
