"""Synthetic Qwen2-style tokenizer files for the tests: a CPT1 vocabulary with merges trained
on a small multilingual corpus, and the UNI1 table of code point classes.

The layouts are the reference's (written by tools/convert_tokenizer_qwen.py:91-103, read by
engine/tokenizers/tokenizer.c:13-58 and tokenizer_qwen.c:32-48):
  CPT1: u32 "CPT1", u32 1, u32 n_vocab, u32 n_merges; n_vocab x (u16 length, raw bytes);
        n_merges x (u32 left id, u32 right id, u32 merged id), rank = position.
  UNI1: u32 "UNI1", u32 n; n x (u32 lo, u32 hi, u32 class) covering every code point, class 1
        for a letter (Unicode category L*), 2 for a number (N*), 0 otherwise (surrogates too).
The special tokens sit where Qwen2.5's do, from id 151643 (<|endoftext|>, <|im_start|> 151644,
<|im_end|> 151645, ...); the ids between the trained tokens and the specials are filler
tokens of several bytes that no merge produces.

The merges come from byte-pair training (count adjacent pairs over the corpus's pre-token
chunks, merge the most frequent, repeat), so the vocabulary behaves like a real one: long
words become one token, rare ones split.

Also here, for the tests: the Qwen2 pre-tokenizer as the reference states it, written as a
regular expression for the `regex` module, and the textbook BPE loop (tokenizer.c:73-106:
the lowest merge rank first, the leftmost of equal ranks)."""
import os
import struct
import unicodedata

import numpy as np

SPECIAL_FIRST = 151643
SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<|object_ref_start|>",
            "<|object_ref_end|>", "<|box_start|>", "<|box_end|>", "<|quad_start|>",
            "<|quad_end|>", "<|vision_start|>", "<|vision_end|>", "<|vision_pad|>",
            "<|image_pad|>", "<|video_pad|>", "<tool_call>", "</tool_call>", "<|fim_prefix|>",
            "<|fim_middle|>", "<|fim_suffix|>", "<|fim_pad|>", "<|repo_name|>", "<|file_sep|>"]
N_VOCAB = SPECIAL_FIRST + len(SPECIALS)          # 151665, Qwen2.5's tokenizer size
TOK_FILE, UNI_FILE = "qwen2.5-tokenizer.bin", "qwen2.5-unicode.bin"

# The reference's split (engine/tokenizers/tokenizer_qwen.c:7-13 and its code at 116-170), in
# the `regex` module's syntax. Whitespace is the six ASCII characters of the reference's
# is_sp_cp. Where the code differs from Qwen2's published pattern the code is followed: its
# newline rule takes [ \t\v\f]* then a newline and then the REST of the whitespace run.
_WS, _WS_NOT_NL = r"[ \t\n\r\v\f]", r"[ \t\v\f]"
PATTERN = (r"'(?i:s|t|re|ve|m|ll|d)"
           r"|[^\r\n\p{L}\p{N}]?\p{L}+"
           r"|\p{N}"
           rf"| ?(?:(?!{_WS})[^\p{{L}}\p{{N}}])+[\r\n]*"
           rf"|{_WS_NOT_NL}*[\r\n]{_WS}*"
           rf"|{_WS}+(?!(?!{_WS}).)"
           rf"|{_WS}+")

CORPUS = """\
The quick brown fox jumps over the lazy dog. It's what they'll say, isn't it? We've been here;
I'm sure you'd agree. THE QUICK BROWN FOX'S TAIL. Don't stop -- keep going!!! (really...)
def forward(self, x):\n    return self.proj(x) + 1  # residual\n\n\tif x > 0:\n\t\treturn -1
Zwölf Boxkämpfer jagen Viktor quer über den großen Sylter Deich. Ça va très bien, merci.
Съешь же ещё этих мягких французских булок да выпей чаю. Γαζέες καὶ μυρτιὲς δὲν θὰ βρῶ.
我能吞下玻璃而不伤身体。日本語のテキストも少し。한국어 문장입니다. 数字１２３ and ٣٤٥ and 12345.
Emoji: 😀🎉 and symbols © ® ™ € £ ¥ — “quotes” ‘single’ «guillemets».
    indented line with trailing spaces   \n\r\nwindows line\r\n  \n\nlast line 2026-12-02 10:30
"""


def class_of(cp):
    """0 other, 1 letter, 2 number (the UNI1 classes)."""
    if 0xD800 <= cp <= 0xDFFF:
        return 0
    c = unicodedata.category(chr(cp))
    return 1 if c[0] == "L" else 2 if c[0] == "N" else 0


def class_ranges():
    cls = np.fromiter((class_of(cp) for cp in range(0x110000)), np.uint8, 0x110000)
    cut = np.flatnonzero(np.diff(cls)) + 1
    lo = np.concatenate([[0], cut])
    hi = np.concatenate([cut - 1, [0x10FFFF]])
    return np.stack([lo, hi, cls[lo]], 1).astype(np.uint32)


def pretokenize(text, specials=()):
    """The chunks of text (a str): a special token is recognised at a chunk start only, the
    lowest id first (tokenizer_qwen.c:91-99, 109-110)."""
    import regex
    pat = regex.compile(PATTERN)
    out, k = [], 0
    while k < len(text):
        sp = next((s for s in specials if text.startswith(s, k)), None)
        if sp is not None:
            out.append(("special", sp))
            k += len(sp)
            continue
        m = pat.match(text, k)
        end = m.end() if m and m.end() > k else k + 1
        out.append(("chunk", text[k:end]))
        k = end
    return out


def bpe_textbook(ids, rank):
    """Merge the lowest-rank adjacent pair, the leftmost of equal ranks, until none merges."""
    ids = list(ids)
    while True:
        best = None
        for i in range(len(ids) - 1):
            r = rank.get((ids[i], ids[i + 1]))
            if r is not None and (best is None or r[0] < best[0]):
                best = (r[0], i, r[1])
        if best is None:
            return ids
        _, i, out = best
        ids[i:i + 2] = [out]


class Vocab:
    """A trained vocabulary: tokens (list of bytes, id order) and merges [(a, b, out)]."""

    def __init__(self, n_merges=1200, seed=11, drop_bytes=()):
        rng = np.random.default_rng(seed)
        order = [int(b) for b in rng.permutation(256) if int(b) not in drop_bytes]
        self.tokens = [bytes([b]) for b in order]
        self.byte_id = {b: i for i, b in enumerate(order)}
        self.merges = []
        words = {}
        for kind, s in pretokenize(CORPUS):
            w = tuple(self.byte_id[b] for b in s.encode() if b in self.byte_id)
            if len(w) > 1:
                words[w] = words.get(w, 0) + 1
        index, seen = {}, set()
        for _ in range(n_merges):
            pairs = {}
            for w, c in words.items():
                for p in zip(w, w[1:]):
                    pairs[p] = pairs.get(p, 0) + c
            if not pairs:
                break
            best = max(pairs.items(), key=lambda kv: (kv[1], -kv[0][0], -kv[0][1]))[0]
            new = self.tokens[best[0]] + self.tokens[best[1]]
            if new not in index:
                index[new] = len(self.tokens)
                self.tokens.append(new)
            out = index[new]
            if best not in seen:                  # a pair formed again keeps its first rank
                seen.add(best)
                self.merges.append((best[0], best[1], out))
            merged = {}
            for w, c in words.items():
                nw, i = [], 0
                while i < len(w):
                    if i + 1 < len(w) and (w[i], w[i + 1]) == best:
                        nw.append(out)
                        i += 2
                    else:
                        nw.append(w[i])
                        i += 1
                merged[tuple(nw)] = merged.get(tuple(nw), 0) + c
            words = merged
        self.n_trained = len(self.tokens)
        self.tokens += [b"\xef\xbf\xbdfill%06d" % i for i in range(SPECIAL_FIRST - len(self.tokens))]
        self.tokens += [s.encode() for s in SPECIALS]
        self.rank = {(a, b): (r, o) for r, (a, b, o) in reversed(list(enumerate(self.merges)))}

    def encode(self, text):
        """text (str) to ids by pretokenize + bpe_textbook, each chunk cut to 512 bytes."""
        ids = []
        for kind, s in pretokenize(text, SPECIALS):
            if kind == "special":
                ids.append(SPECIAL_FIRST + SPECIALS.index(s))
                continue
            b = s.encode()[:512]
            ids += bpe_textbook([self.byte_id[x] for x in b if x in self.byte_id], self.rank)
        return ids

    def write(self, d):
        """Both files into directory d; returns d."""
        os.makedirs(d, exist_ok=True)
        with open(os.path.join(d, TOK_FILE), "wb") as f:
            f.write(struct.pack("<4I", 0x31545043, 1, len(self.tokens), len(self.merges)))
            for t in self.tokens:
                f.write(struct.pack("<H", len(t)) + t)
            for m in self.merges:
                f.write(struct.pack("<3I", *m))
        rg = class_ranges()
        with open(os.path.join(d, UNI_FILE), "wb") as f:
            f.write(struct.pack("<2I", 0x31494E55, len(rg)) + rg.astype("<u4").tobytes())
        return d
