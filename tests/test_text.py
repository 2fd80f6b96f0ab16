"""The library's text side (host code in libyuear, no GPU) against the
oracle (oracle/text_ref.py): NFC over every code point, the pre-tokenizer's
pieces, encode / decode, the vocabulary loader's checks, the prompt layout
and SongRequest validation, with the reference's error types and messages
(protocol.mm:123-357, 428-591). The library's Unicode tables come from
Python's unicodedata; code points unassigned there are left out of the
pattern comparison (the ``regex`` module may know newer assignments)."""
import random
import unicodedata

import pytest

import text_ref
import text_util
from text_ref import ABC_END, ABC_START, EOD, MUSIC_START


@pytest.fixture(scope="module")
def yuear():
    import yuear as y
    return y


@pytest.fixture(scope="module")
def tok(yuear, text_vocab):
    t = yuear.Tokenizer(text_vocab[0])
    yield t
    t.close()


def assigned(cp):
    return not (0xD800 <= cp <= 0xDFFF) and unicodedata.category(chr(cp)) != "Cn"


def random_unicode(rng, n):
    pools = [range(0x20, 0x7F), range(0xA0, 0x250), range(0x300, 0x370), range(0x370, 0x530),
             range(0x1100, 0x1200), range(0x1E00, 0x2000), range(0x2000, 0x2070),
             range(0x3000, 0x3100), range(0xAC00, 0xAC40), range(0x4E00, 0x4E40),
             range(0x1F300, 0x1F400)]
    out = []
    while len(out) < n:
        cp = rng.choice(rng.choice(pools))
        if assigned(cp):
            out.append(chr(cp))
        if rng.random() < 0.15:
            out.append(rng.choice(" \n\r\t'"))
    return "".join(out)


def test_nfc_every_code_point(yuear):
    text = "".join(chr(cp) for cp in range(0x110000) if not 0xD800 <= cp <= 0xDFFF)
    assert yuear.text_nfc(text) == unicodedata.normalize("NFC", text)


def test_nfc_sequences(yuear):
    rng = random.Random(2)
    marks = [chr(c) for c in range(0x300, 0x370)] + ["ཱ", "ི", "ְ", "ุ",
                                                      "゙", "゚", "᷀", "⃐"]
    bases = list("aeiouAEIOUnNcCsSzZ") + ["Α", "ι", "Е", "ᄀ", "ᅡ",
                                          "ᆨ", "가", "か", "ハ", "େ",
                                          "ା", "ဥ", "ီ"]
    for _ in range(2000):
        s = "".join(rng.choice(bases) + "".join(rng.choice(marks)
                                               for _ in range(rng.randrange(4)))
                    for _ in range(rng.randrange(1, 6)))
        for form in ("NFD", "NFKD"):
            s2 = unicodedata.normalize(form, s)
            assert yuear.text_nfc(s2) == unicodedata.normalize("NFC", s2), ascii(s2)


def test_pieces_every_assigned_code_point(yuear):
    cps = [cp for cp in range(0x110000) if assigned(cp)]
    text = "".join(chr(cp) for cp in cps)
    nfc = unicodedata.normalize("NFC", text)
    assert yuear.text_pieces(text) == text_ref.pieces(nfc)


def test_pieces_random_and_samples(yuear):
    rng = random.Random(4)
    import make_text_vocab
    texts = text_util.SAMPLES + make_text_vocab.CORPUS + [random_unicode(rng, 300)
                                                           for _ in range(300)]
    for text in texts:
        assert yuear.text_pieces(text) == text_ref.pieces(unicodedata.normalize("NFC", text)), \
            ascii(text)


def test_encode_decode_match_oracle(tok, text_vocab):
    _, ranks = text_vocab
    rng = random.Random(6)
    import make_text_vocab
    texts = text_util.SAMPLES + make_text_vocab.CORPUS + [random_unicode(rng, 400)
                                                           for _ in range(200)]
    for text in texts:
        ids = tok.encode(text)
        assert ids == text_ref.encode(text, ranks), ascii(text)
        assert tok.decode(ids) == text_ref.decode(ids, ranks) == unicodedata.normalize("NFC", text)
    # arbitrary id runs: cut multi-byte characters, specials, fillers, out of range
    specials = list(range(EOD, EOD + 208)) + [MUSIC_START, 184000, -5, 10 ** 8]
    for _ in range(300):
        ids = [rng.choice([rng.randrange(0, 1300), rng.randrange(0, EOD), rng.choice(specials)])
               for _ in range(rng.randrange(0, 40))]
        assert tok.decode(ids) == text_ref.decode(ids, ranks), ids


def test_encode_long_pieces(tok, text_vocab):
    _, ranks = text_vocab
    for text in (" " * 5000, "a" * 3000, "ab" * 2000 + "\n" * 100, "漢" * 1000, "!?" * 1500):
        assert tok.encode(text) == text_ref.encode(text, ranks)


def test_encode_rejects_invalid_utf8(tok, yuear):
    for data in (b"\xff", b"abc\xc3", b"\xc0\xaf", b"\xed\xa0\x80", b"\xf4\x90\x80\x80",
                 b"\xe2\x82", b"\x80x"):
        with pytest.raises(yuear.TextDecodeError, match="Invalid UTF-8 text"):
            tok.encode(data)
    assert tok.encode(b"a\x00b") == tok.encode("a") + tok.encode("\x00") + tok.encode("b")


def write(path, lines):
    path.write_bytes(b"".join(line + b"\n" for line in lines))
    return str(path)


def test_loader_checks(tmp_path, yuear, text_vocab):
    lines = open(text_vocab[0], "rb").read().splitlines()
    with pytest.raises(FileNotFoundError):
        yuear.Tokenizer(tmp_path / "missing.tiktoken")
    bad = "Invalid checkpoint-native qwen.tiktoken vocabulary"
    for broken in (b"YQ== 5 extra", b"YQ==", b"YQ== x5", b"YQ== 151643", b"YQ== -1",
                   b"YQ== 99999999999", b"   "):
        with pytest.raises(ValueError, match=bad):
            yuear.Tokenizer(write(tmp_path / "v.tiktoken", lines[:7] + [broken] + lines[8:]))
    for broken in (b"Y!== 7", b"YQ 7", b"= 7", b"==== 7"):
        with pytest.raises(ValueError, match="Invalid base64 vocabulary token"):
            yuear.Tokenizer(write(tmp_path / "v.tiktoken", lines[:7] + [broken] + lines[8:]))
    count = r"Expected checkpoint-native qwen.tiktoken \(151643 ordinary tokens\)"
    with pytest.raises(ValueError, match=count):  # one token short
        yuear.Tokenizer(write(tmp_path / "v.tiktoken", lines[:-1]))
    with pytest.raises(ValueError, match=count):  # a piece listed twice
        yuear.Tokenizer(write(tmp_path / "v.tiktoken", lines[:7] + [lines[6].split()[0] + b" 7"]
                              + lines[8:]))
    # blank lines, CRLF endings, + signs and leading zeros are accepted
    ok = [b""] + [line + b"\r" for line in lines[:5]] + [lines[5].split()[0] + b" +0005"] + lines[6:]
    t = yuear.Tokenizer(write(tmp_path / "v.tiktoken", ok))
    assert t.encode("hello") == yuear.Tokenizer(text_vocab[0]).encode("hello")
    t.close()


def test_missing_byte_token(tmp_path, yuear, text_vocab):
    lines = open(text_vocab[0], "rb").read().splitlines()
    # the byte 'q' replaced by another filler: text with 'q' cannot be encoded
    filler = b"\xff\xff\xff\xff"
    import base64
    lines[ord("q")] = base64.b64encode(filler) + b" %d" % ord("q")
    t = yuear.Tokenizer(write(tmp_path / "v.tiktoken", lines))
    with pytest.raises(ValueError, match="Vocabulary is missing a byte token"):
        t.encode("quiet")
    t.close()


@pytest.mark.parametrize("cot", ["off", "melody", "full"])
def test_prefixes_match_oracle(tok, yuear, text_vocab, cot):
    _, ranks = text_vocab
    style, lyrics = "female vocal, pop", "[verse]\nI've been walking\r\n  down this road\n"
    abc = "X:1\nK:C\n\"C\"CDEF|GABc|\n"
    req = yuear.SongRequest(style, lyrics, cot=cot)
    assert yuear.token_prefixes(req, tok) == text_ref.token_prefixes(style, lyrics, cot, ranks)
    ids = text_ref.encode(abc, ranks)
    assert yuear.token_prefixes(req, tok, ids) == text_ref.token_prefixes(style, lyrics, cot,
                                                                          ranks, abc_ids=ids)
    if cot != "off":
        with_abc = yuear.SongRequest(style, lyrics, cot=cot, abc=abc)
        assert yuear.token_prefixes(with_abc, tok) == text_ref.token_prefixes(
            style, lyrics, cot, ranks, abc=abc)
        assert yuear.negative_prefix(req, tok, ids) == text_ref.negative_prefix(cot, ranks, ids)
        assert yuear.negative_prefix(req, tok, []) == text_ref.negative_prefix(cot, ranks, [])
        with pytest.raises(ValueError, match="Symbolic CFG must retain the exact positive-branch"):
            yuear.negative_prefix(req, tok)
        with pytest.raises(ValueError, match="ABC IDs must remain inside the ordinary text"):
            yuear.token_prefixes(req, tok, [5, EOD])
        with pytest.raises(ValueError, match="ABC IDs must remain inside the ordinary text"):
            yuear.negative_prefix(req, tok, [-1])
    else:
        assert yuear.negative_prefix(req, tok) == text_ref.negative_prefix(cot, ranks)
        assert yuear.token_prefixes(req, tok, [EOD + 5]) == yuear.token_prefixes(req, tok)


def test_prefixes_follow_the_reference_tests(tok, yuear):
    # vendor test_protocol.py:26-39 with this tokenizer
    for cot in ("full", "melody"):
        r = yuear.SongRequest("STYLE", "LYRIC", cot=cot, cfg_scale=1.2)
        ids = [17, 19, 23]
        positive = yuear.token_prefixes(r, tok, ids)
        negative = yuear.negative_prefix(r, tok, ids)
        assert positive[-6:] == negative[-6:] == [ABC_START, 17, 19, 23, ABC_END, MUSIC_START]
        assert negative == [EOD] + tok.encode(text_ref.INSTRUCTIONS[cot]) + negative[-6:]
        assert positive != negative
    r = yuear.SongRequest("a", "b", cot="off")
    assert yuear.token_prefixes(r, tok)[-3:] == [ABC_START, ABC_END, MUSIC_START]
    assert ABC_START not in yuear.negative_prefix(r, tok)


def test_request_validation_and_guidance(yuear, tok):
    ok = yuear.SongRequest("a", "b")
    ok.validate()
    assert ok.guidance == 1.0
    assert yuear.SongRequest("a", "b", cot="off").guidance == 1.01
    assert yuear.SongRequest("a", "b", cfg_scale=3.5).guidance == 3.5
    cases = [
        (dict(cot="sideways"), "cot must be off, melody or full"),
        (dict(seed=2 ** 63), r"seed must be an integer in \[0, 2\*\*63\)"),
        (dict(id=""), "id must be a filename-safe identifier"),
        (dict(id="-x"), "id must be a filename-safe identifier"),
        (dict(id="a/b"), "id must be a filename-safe identifier"),
        (dict(id="a" * 181), "id must be a filename-safe identifier"),
        (dict(cot="off", abc="X:1"), "External ABC requires nonempty text and cot=melody/full"),
        (dict(abc=" \n\t　\x1c\x85"), "External ABC requires nonempty text"),
        (dict(cfg_scale=20.5), r"cfg_scale must be finite and in \[0,20\]"),
        (dict(cfg_scale=float("nan")), r"cfg_scale must be finite and in \[0,20\]"),
        (dict(cfg_scale=-0.1), r"cfg_scale must be finite and in \[0,20\]"),
    ]
    for kw, msg in cases:
        with pytest.raises(ValueError, match=msg):
            yuear.SongRequest("a", "b", **kw).validate()
    yuear.SongRequest("a", "b", id="A9_.-x" + "b" * 174, abc=" x ", cfg_scale=20).validate()
    with pytest.raises(ValueError, match="cot must be off, melody or full"):
        yuear.token_prefixes(yuear.SongRequest("a", "b", cot="x"), tok)


def test_chunk_ranges_match_oracle(yuear):
    rng = random.Random(8)
    cases = [(10, 24570, 24576), (5000, 100, 24576), (30000, 0, 24576), (7, 10, 20), (1, 0, 5),
             (2 ** 31 - 1, 0, 24576)]
    cases += [(rng.randrange(1, 100000), rng.randrange(0, 24576), rng.randrange(5, 24577))
              for _ in range(300)]
    for frames, prefix, context in cases:
        try:
            want = text_ref.chunk_ranges(frames, prefix, context)
        except ValueError:
            with pytest.raises(ValueError, match="Empty codec or prefix leaves no acoustic"):
                yuear.chunk_ranges(frames, prefix, context)
            continue
        if frames > 10 ** 6:  # the oracle's list is long; compare ends and count
            got = yuear.chunk_ranges(frames, prefix, context)
            assert (got[0], got[-1], len(got)) == (want[0], want[-1], len(want))
            continue
        assert yuear.chunk_ranges(frames, prefix, context) == want, (frames, prefix, context)
    for frames, prefix in ((0, 10), (5, 24572), (5, 30000), (-3, 0)):
        with pytest.raises(ValueError, match="Empty codec or prefix leaves no acoustic context"):
            yuear.chunk_ranges(frames, prefix)
