"""The test vocabulary: a checkpoint-native qwen.tiktoken built from the
merge fixture (tests/golden/text_merges.txt, made by make_text_vocab.py):
ranks 0-255 the single bytes, then the merged pieces in training order,
then filler pieces holding the byte 0xFF (never in valid UTF-8) up to the
151643 ordinary tokens the loader requires."""
import base64
import os

import text_ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def merges():
    out = []
    with open(os.path.join(GOLDEN, "text_merges.txt")) as f:
        for line in f:
            a, b = line.split()
            out.append((base64.b64decode(a), base64.b64decode(b)))
    return out


def vocabulary_pieces():
    pieces = [bytes([b]) for b in range(256)] + [a + b for a, b in merges()]
    pieces += [b"\xff" + i.to_bytes(3, "big") for i in range(text_ref.EOD - len(pieces))]
    return pieces


# Text the tests encode: the training corpus plus lines it never saw.
SAMPLES = [
    "Generate a chord-annotated ABC transcription, then generate music with codec tokens "
    "from the given conditions.\n[Tags]\nfemale vocal, pop\n[Lyrics]\n[verse]\nHello\n",
    "I'VE GOT IT'S THEY'LL we're You'D 'Ll 'ſ 'ſt ' s '  x'x 'xyz '123 '''",
    "tabs\t\tand\x0cform\x0bfeed\u0085next line para nbsp　ideo",
    "punct!\x0b!? \x85\x85 ;\x0b\n\x0b\x0b  \x85 end\x85",
    "  leading\n\n\n  trailing  \r\n\r\n\t \n",
    "multi    space\n   \n\t\tindent\r\r\n\n\rmix",
    "numbers 1234567890 ١٢٣ ⅫⅩ ½ ²³ 𝟘𝟙",
    "é ǟ ḍ̇ q̣̇ Å Å Ω Å",
    "한국어 각 한글",
    "emoji 👩‍👩‍👧‍👦 🇯🇵 ❤️‍🔥 🏳️‍🌈 x‍y",
    "ABC X:1\nK:C\n\"Am\"A2c2 e2a2|\"F\"f4 \"G\"g4:|\n",
    "¡¿«»—–…•·° ©® ™ § ¶ † ‡ ‰ ′ ″ ‹ › € £ ¥",
    "mixed漢字kana仮名ひらがなカタカナ123abc",
    "",
    " ",
    "\n",
    "a",
    "zzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzzz",
]
