"""Writes text_merges.txt: the merged pieces (base64, in rank order from 256)
of a small byte pair vocabulary trained on the corpus below -- instructions,
tags, lyrics in several scripts and ABC notation -- for the tokenizer tests.
The tests complete it to the 151643 ordinary tokens a checkpoint-native
qwen.tiktoken holds (ranks 0-255 the single bytes, then these merges, then
filler pieces containing the byte 0xFF, which valid UTF-8 never holds).

Training: pieces by the reference pattern over NFC text; repeatedly join
the most frequent adjacent pair (ties: shorter concatenation, then lowest
bytes), down to pairs seen once. No two pairs may make the same token (the
script fails otherwise), so every token has one creating pair and a rank
above both halves: rank order and pair-merge order agree.

Run from the repository root: python3 tests/golden/make_text_vocab.py
"""
import base64
import collections
import os
import sys
import unicodedata

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import text_ref  # noqa: E402

MERGES = 1500

CORPUS = [
    text_ref.INSTRUCTIONS["off"], text_ref.INSTRUCTIONS["melody"], text_ref.INSTRUCTIONS["full"],
    "[Tags]\nfemale vocal, pop, piano, bright, 120 bpm, emotional, acoustic guitar\n",
    "[Tags]\nmale vocal, rock, electric guitar, drums, bass, energetic, anthem\n",
    "[Tags]\njazz, saxophone, smooth, late night, swing, upright bass\n",
    "[Lyrics]\n[verse]\nI've been walking down this road tonight\nThe city's lights are burning bright\n",
    "[chorus]\nWe'll sing until the morning comes, we're young and we're alive\n",
    "[verse]\nShe'd never known the way it'd feel, they'll never know the truth\n",
    "[bridge]\nHold on, hold on, don't let me go, I'm falling into you\n",
    "You're the reason that I'm still here, you're the light inside my heart\n",
    "Nobody knows the trouble I've seen, nobody knows but me\n",
    "Dancing in the rain again, singing in the sun, oh oh oh\n",
    "La la la la, na na na, hey hey hey, yeah yeah yeah\n",
    "[verse]\n春风吹过山岗 我在远方歌唱\n你的笑容 像星光一样\n",
    "[chorus]\n爱你到永远 不离不弃\n我们一起 走过四季\n",
    "[verse]\n夜空に輝く星たちよ 私の願いを聞いて\n君と歩いた道を 忘れないよ\n",
    "[chorus]\n사랑해요 영원히 너만을\n우리 함께 노래해\n",
    "Café au lait, naïve façade, crème brûlée, déjà vu, Ångström, Øresund\n",
    "Ünter den Linden, schön, Straße, Grüße, Mädchen, Fräulein\n",
    "¿Dónde está la música? ¡Canta conmigo, corazón!\n",
    "Привет, мир! Песня о любви и надежде\n",
    "Γεια σου κόσμε, τραγούδι της αγάπης\n",
    "مرحبا بالعالم أغنية الحب\n",
    "שלום עולם שיר אהבה\n",
    "नमस्ते दुनिया प्यार का गीत\n",
    "🎵🎶 music 🎸🥁 love ❤️ 2024 🎤\n",
    "X:1\nT:Morning Song\nM:4/4\nL:1/8\nQ:1/4=120\nK:G\n",
    '"G"GABc d2B2|"C"c2e2 "D"d2A2|"G"B2G2 "Em"E2G2|"Am"A4 "D"D4|\n',
    '"G"g2fe d2B2|"C"cBAG "D"FGAd|"G"B2G2 "D"A2F2|"G"G8:|\n',
    "X:2\nT:Waltz\nM:3/4\nL:1/4\nK:D\n|:D F A|d3|c B A|B2 A|F G A|D3:|\n",
    "V:1\n[V:1] z4 | C2 E2 G2 c2 | B,2 D2 G2 B2 |]\n",
    "X:1\r\nK:C\r\n\"C\"CDEF|\r\n\"G\"GABc|\r\n",
    "w: Twin-kle twin-kle lit-tle star how I won-der what you are\n",
    "1, 2, 3, 4, 10, 25, 100, 2024, 3.14159, 1/8, 4/4, 6/8\n",
    "    indented    spaces  and\ttabs\t\tand\n\nnewlines\r\n\r\n  \n",
    "THE END... (fade out) -- [outro] ~ * # @ & % $ !?\n",
    "It's IT'S it'S 'tis 're 've 'm 'll 'd we'VE they'RE\n",
]


def train(corpus, merges):
    words = collections.Counter()
    for text in corpus:
        for piece in text_ref.pieces(unicodedata.normalize("NFC", text)):
            words[piece.encode("utf-8")] += 1
    seqs = {w: [bytes([b]) for b in w] for w in words}
    vocab = {bytes([b]) for b in range(256)}
    out = []
    while len(out) < merges:
        pairs = collections.Counter()
        for w, count in words.items():
            s = seqs[w]
            for a, b in zip(s, s[1:]):
                pairs[(a, b)] += count
        if not pairs:
            break
        (a, b), count = min(pairs.items(), key=lambda kv: (-kv[1], len(kv[0][0] + kv[0][1]),
                                                           kv[0][0] + kv[0][1], kv[0][0]))
        token = a + b
        assert token not in vocab, token
        vocab.add(token)
        out.append((a, b))
        for w, s in seqs.items():
            i, merged = 0, []
            while i < len(s):
                if i + 1 < len(s) and s[i] == a and s[i + 1] == b:
                    merged.append(token)
                    i += 2
                else:
                    merged.append(s[i])
                    i += 1
            seqs[w] = merged
    return out


def main():
    merges = train(CORPUS, MERGES)
    with open(os.path.join(HERE, "text_merges.txt"), "w") as f:
        for a, b in merges:
            f.write(f"{base64.b64encode(a).decode()} {base64.b64encode(b).decode()}\n")
    print(f"{len(merges)} merges")


if __name__ == "__main__":
    main()
