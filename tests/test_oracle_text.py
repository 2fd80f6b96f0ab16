"""Pins of the oracle's text side (oracle/text_ref.py) before it judges the
library: its byte pair merges against an independent implementation (the
HF ``tokenizers`` BPE model over the same vocabulary, pair merges in rank
order, vocabulary words taken whole) and hand-worked cases; its two
patterns against each other (ICU \\s and White_Space differ only on U+000B
and U+0085); the prompt layout against the reference's own protocol tests
(vendor test_protocol.py:26-39). NFC and the pattern engine are library
routines (``unicodedata``, ``regex``)."""
import random
import unicodedata

import pytest

import text_ref
import text_util
from text_ref import ABC_END, ABC_START, EOD, MUSIC_START


def byte_level():
    """GPT-2's reversible byte -> printable character map (HF ByteLevel)."""
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    out, extra = {}, 0
    for b in range(256):
        if b in keep:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + extra)
            extra += 1
    return out


def random_text(rng, n):
    alphabet = (list("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789")
                + list(" \t\n\r\x0b\x0c'\".,;:!?-_[](){}|/\\#@~") +
                [" ", " ", "　", "\u0085", "ſ", "é", "ß", "ç", "ñ", "ø",
                 "́", "̈", "̣", "漢", "字", "한", "글", "١", "½", "Ⅻ", "😀",
                 "🎵", "‍", "️", "א", "ب", "क", "ि"])
    return "".join(rng.choice(alphabet) for _ in range(n))


@pytest.fixture(scope="module")
def hf_model():
    tokenizers = pytest.importorskip("tokenizers")
    m = byte_level()
    to_str = (lambda bs: "".join(m[b] for b in bs))
    pieces = text_util.vocabulary_pieces()
    merges = text_util.merges()
    vocab = {to_str(p): r for r, p in enumerate(pieces) if b"\xff" not in p or len(p) == 1}
    model = tokenizers.models.BPE(vocab=vocab, merges=[(to_str(a), to_str(b)) for a, b in merges],
                                  ignore_merges=True)
    return model, to_str


def test_bpe_matches_hf_pair_merges(hf_model, text_vocab):
    model, to_str = hf_model
    _, ranks = text_vocab
    rng = random.Random(3)
    texts = list(text_util.SAMPLES) + [random_text(rng, 200) for _ in range(50)]
    import make_text_vocab
    texts += make_text_vocab.CORPUS
    checked = 0
    for text in texts:
        for piece in text_ref.pieces(unicodedata.normalize("NFC", text)):
            word = piece.encode("utf-8")
            want = [t.id for t in model.tokenize(to_str(word))]
            assert text_ref.bpe(word, ranks) == want, piece
            checked += 1
    assert checked > 3000


def test_bpe_hand_worked():
    ranks = {b"a": 0, b"b": 1, b"c": 2, b"ab": 3, b"bc": 4, b"abc": 5, b"aa": 6}
    assert text_ref.bpe(b"abc", ranks) == [5]          # the piece is a token
    assert text_ref.bpe(b"abca", ranks) == [5, 0]      # ab (3) before bc (4), then abc
    assert text_ref.bpe(b"bca", ranks) == [4, 0]
    assert text_ref.bpe(b"aaa", ranks) == [6, 0]       # equal ranks: leftmost first
    assert text_ref.bpe(b"cab", ranks) == [2, 3]
    # a token reachable only through a pair that is not in the table stays split
    ranks2 = {b"x": 0, b"y": 1, b"z": 2, b"xyz": 3}
    assert text_ref.bpe(b"xyzx", ranks2) == [0, 1, 2, 0]


def test_icu_and_white_space_patterns_differ_only_on_vt_and_nel():
    rng = random.Random(9)
    for _ in range(300):
        text = random_text(rng, 120)
        icu = text_ref.pieces(text, text_ref.ICU_PATTERN)
        vendor = text_ref.pieces(text, text_ref.VENDOR_PATTERN)
        if "\x0b" not in text and "\x85" not in text:
            assert icu == vendor, text
        assert "".join(icu) == text  # the pieces cover the text
    # ICU: U+000B is not \s, so it joins the punctuation run
    assert text_ref.pieces("!\x0b!", text_ref.ICU_PATTERN) == ["!\x0b!"]
    assert text_ref.pieces("!\x0b!", text_ref.VENDOR_PATTERN) == ["!", "\x0b", "!"]
    assert text_ref.pieces("x\x85", text_ref.ICU_PATTERN) == ["x", "\x85"]


def test_pattern_known_pieces():
    p = text_ref.pieces
    assert p("Hello world's end") == ["Hello", " world", "'s", " end"]
    assert p("I'VE it'S 'ſx") == ["I", "'VE", " it", "'S", " '", "ſx"]
    assert p("a  b") == ["a", " ", " b"]
    assert p("x \n\n  y") == ["x", " \n\n", " ", " y"]
    assert p("2024!!\n\nok") == ["2", "0", "2", "4", "!!\n\n", "ok"]
    assert p("end   ") == ["end", "   "]


def test_prefix_layout_follows_the_reference_tests(text_vocab):
    _, ranks = text_vocab
    ids = [17, 19, 23]
    for cot in ("full", "melody"):
        positive = text_ref.token_prefixes("STYLE", "LYRIC", cot, ranks, abc_ids=ids)
        negative = text_ref.negative_prefix(cot, ranks, ids)
        tail = [ABC_START, 17, 19, 23, ABC_END, MUSIC_START]
        assert positive[-6:] == negative[-6:] == tail
        assert negative == [EOD] + text_ref.encode(text_ref.INSTRUCTIONS[cot], ranks) + tail
        assert positive != negative
    off = text_ref.token_prefixes("a", "b", "off", ranks)
    assert off[-3:] == [ABC_START, ABC_END, MUSIC_START]
    assert ABC_START not in text_ref.negative_prefix("off", ranks)
    assert text_ref.token_prefixes("a", "b", "full", ranks)[-1] == ABC_START


def test_decode_is_python_replacement_decoding(text_vocab):
    _, ranks = text_vocab
    euro = "€".encode()
    split = [ranks[euro[:1]], ranks[euro[1:2]]]  # a cut three-byte character
    assert text_ref.decode(split, ranks) == "�"
    assert text_ref.decode([ranks[b"a"], EOD, ABC_START, 10 ** 7, -1], ranks) == "a<|endoftext|><abc>"


def test_chunk_ranges_hand_worked():
    # (context - prefix - 3) // 2 frames per chunk, capped at the context
    assert text_ref.chunk_ranges(10, 24570) == [(i, i + 1) for i in range(10)]  # 3 // 2 = 1
    assert text_ref.chunk_ranges(5000, 100) == [(0, 5000)]                       # 12236 per chunk
    assert text_ref.chunk_ranges(30000, 0) == [(0, 12286), (12286, 24572), (24572, 30000)]
    assert text_ref.chunk_ranges(7, 10, context=20) == [(0, 3), (3, 6), (6, 7)]  # 7 // 2 = 3
    for frames, prefix in ((0, 10), (5, 24572), (5, 30000)):
        with pytest.raises(ValueError, match="Empty codec or prefix leaves no acoustic context"):
            text_ref.chunk_ranges(frames, prefix)
