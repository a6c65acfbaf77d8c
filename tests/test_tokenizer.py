"""The tokenizer behind cp_chat (include/cptok.h) on the CPU, against the reference's own
tokenizer (engine/tokenizers/tokenizer.c + tokenizer_qwen.c compiled from source into
oracle/_ref) and against an independent statement of the same rules (tests/tok_files.py: the
split as a regular expression, the textbook BPE loop).

The files are synthetic (tests/tok_files.py): no Qwen2.5 tokenizer.json is available here, and
the reference holds no recorded tokenizer vectors (its tools/verify_qwen_tokenizer.py reads a
trace that is not in the tree). Bar: identical ids."""
import ctypes
import os

import numpy as np
import pytest

import cachepotato_amd as C
from tests import tok_files as TF

TEXTS = [
    "",
    "Hello, world!",
    "<|im_start|>user\nWhat's 2+2? /no_think<|im_end|>\n<|im_start|>assistant\n",
    "<|im_start|><|im_end|><|endoftext|>",
    "I'LL be there; she'S here, they'Re gone, we'VE won, I'M in, he'D go, don'T",
    "'s's 'x ''ll '",
    "numbers 12345 and ٣٤٥ and １２３ and ½ ⅷ",
    "   leading spaces, trailing spaces   ",
    "a  b   c    d\t\te\n\nf\r\n\r\ng \n h\n  \n  x",
    "punctuation!!!\n\n... ?!?\n  --> ==> (x) [y] {z}\n",
    "tabs\tand\vvertical\fform feeds",
    "Zwölf Boxkämpfer jagen Viktor quer über den großen Sylter Deich.",
    "Съешь же ещё этих мягких французских булок. 我能吞下玻璃而不伤身体。",
    "emoji 😀🎉👍🏽 mixed with text😀text",
    "x" * 700,
    " " * 600 + "y",
    "a" + "é" * 300,
    "def f(x):\n    return x ** 2  # square\n",
    "<tool_call>{\"name\": \"f\"}</tool_call>",
    "<|im_start",
    "!<|im_end|>",
    "word<|im_end|>",
    "\n<|im_start|>",
]


@pytest.fixture(scope="module")
def vocab(tmp_path_factory):
    v = TF.Vocab()
    v.dir = v.write(str(tmp_path_factory.mktemp("tok")))
    return v


class Ours:
    def __init__(self, d):
        L = C.lib()
        L.cpt_load.restype = ctypes.c_void_p
        L.cpt_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
        L.cpt_free.argtypes = [ctypes.c_void_p]
        L.cpt_encode.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int]
        L.cpt_vocab_size.argtypes = [ctypes.c_void_p]
        L.cpt_token_bytes.argtypes = [ctypes.c_void_p, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_void_p),
                                      ctypes.POINTER(ctypes.c_size_t)]
        self.L = L
        self.err = ctypes.create_string_buffer(256)
        self.h = L.cpt_load(os.path.join(d, TF.TOK_FILE).encode(),
                            os.path.join(d, TF.UNI_FILE).encode(), self.err, 256)

    def encode(self, text, max_ids=1 << 16):
        b = text if isinstance(text, bytes) else text.encode()
        out = np.zeros(max(max_ids, 1), np.int32)
        n = self.L.cpt_encode(self.h, b, out.ctypes.data, max_ids)
        return out[:n].tolist()

    def token(self, i):
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        if self.L.cpt_token_bytes(self.h, i, ctypes.byref(p), ctypes.byref(n)):
            return None
        return ctypes.string_at(p.value, n.value) if n.value else b""

    def close(self):
        self.L.cpt_free(self.h)


class RefTok:
    """The reference's tokenizer: tokenizer_load + tokenizer_qwen_load_unicode +
    tokenizer_qwen_encode from oracle/_ref/libref.so. Its class table is process-global.
    Its special tokens get a terminating NUL (ref_tok_terminate_specials): the encoder takes
    strlen() of those unterminated entries (tokenizer_qwen.c:110), which without it reads
    whatever follows them on this process's heap."""

    def __init__(self, d):
        from oracle.bindings import REF_SO
        if not os.path.exists(REF_SO):
            pytest.skip("oracle/_ref/libref.so is not built")
        L = ctypes.CDLL(REF_SO)
        L.tokenizer_qwen_encode.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p,
                                            ctypes.c_int]
        self.L = L
        self.t = ctypes.create_string_buffer(2048)       # struct Tokenizer is 1056 bytes
        assert L.tokenizer_qwen_load_unicode(os.path.join(d, TF.UNI_FILE).encode()) == 0
        assert L.tokenizer_load(self.t, os.path.join(d, TF.TOK_FILE).encode()) == 0
        assert L.ref_tok_terminate_specials(self.t) == TF.N_VOCAB - TF.SPECIAL_FIRST

    def encode(self, text, max_ids=1 << 16):
        b = text if isinstance(text, bytes) else text.encode()
        out = np.zeros(max(max_ids, 1), np.int32)
        n = self.L.tokenizer_qwen_encode(self.t, b, out.ctypes.data, max_ids)
        return out[:n].tolist()


@pytest.fixture(scope="module")
def ours(vocab):
    o = Ours(vocab.dir)
    assert o.h, o.err.value
    yield o
    o.close()


@pytest.fixture(scope="module")
def ref(vocab):
    return RefTok(vocab.dir)


def fuzz_texts(n, seed, valid=False):
    """Text mixing every class the rules distinguish, as bytes: ASCII letters and digits,
    the six whitespace characters, apostrophes and contraction letters, punctuation, multi-byte
    letters / digits / symbols / emoji, special-token pieces, and invalid UTF-8 (lone
    continuation bytes, lead bytes without their continuation, 0xF8-0xFF), never a NUL."""
    rng = np.random.default_rng(seed)
    atoms = [b"a", b"Z", b"q", b"7", b"0", b" ", b" ", b"  ", b"\t", b"\n", b"\r", b"\v", b"\f",
             b"'", b"'s", b"'LL", b"'re", b"'d", b"!", b"?", b"...", b"#", b"(", b")", b"-",
             "é".encode(), "ß".encode(), "д".encode(), "界".encode(), "٣".encode(),
             "１".encode(), "€".encode(), "😀".encode(), "—".encode(), b"<|im_start|>",
             b"<|im_end|>", b"<|", b"|>", b"<tool_call>", b"\x80", b"\xbf", b"\xc3", b"\xe4\xb8",
             b"\xf0\x9f", b"\xf8", b"\xff", b"\xc0\x80", b"the", b" the", b"ing", b"self"]
    if valid:
        atoms = [a for a in atoms if _utf8(a)]
    out = []
    for _ in range(n):
        k = int(rng.integers(1, 60))
        out.append(b"".join(atoms[int(i)] for i in rng.integers(0, len(atoms), k)))
    return out


def _utf8(b):
    try:
        b.decode("utf-8")
        return True
    except UnicodeDecodeError:
        return False


def test_files_load(ours, vocab):
    assert ours.L.cpt_vocab_size(ours.h) == TF.N_VOCAB
    for i in (0, 255, vocab.n_trained - 1, TF.SPECIAL_FIRST + 2, TF.N_VOCAB - 1):
        assert ours.token(i) == vocab.tokens[i]
    assert ours.token(TF.N_VOCAB) is None and ours.token(-1) is None


@pytest.mark.parametrize("i", range(len(TEXTS)))
def test_encode_matches_reference(ours, ref, i):
    assert ours.encode(TEXTS[i]) == ref.encode(TEXTS[i])


@pytest.mark.parametrize("i", range(len(TEXTS)))
def test_encode_matches_restatement(ours, vocab, i):
    """Against the regex split + textbook BPE: a different formulation of the same rules, so
    an edge both C codes get wrong the same way still shows."""
    import regex
    for ch in set(TEXTS[i]):           # the regex module's classes agree with the table's
        cp = ord(ch)
        want = TF.class_of(cp)
        assert (regex.match(r"\p{L}", ch) is not None) == (want == 1), ch
        assert (regex.match(r"\p{N}", ch) is not None) == (want == 2), ch
    assert ours.encode(TEXTS[i]) == vocab.encode(TEXTS[i])


def test_encode_matches_reference_on_fuzz(ours, ref):
    bad = [t for t in fuzz_texts(400, 5) if ours.encode(t) != ref.encode(t)]
    assert not bad, bad[:3]


def test_encode_matches_reference_on_cut_sequences(ours, ref):
    """Texts ending inside a multi-byte sequence, for every lead byte: a lead byte opens the
    longest sequence that still fits (an F0 lead with two bytes left is read as three bytes),
    and a lone lead byte at the end is a code point of its own value."""
    rng = np.random.default_rng(9)
    bad = []
    for lead in range(0xC0, 0x100):
        for tail in (b"", b"\x9f", b"\x9f\x98", b"\x9f\x98\x80"):
            for pre in (b"", b"a", b" ", b"'", b"7", b"\n"):
                t = pre + bytes([lead]) + tail
                if ours.encode(t) != ref.encode(t):
                    bad.append(t)
    for t in fuzz_texts(1500, 12):
        cut = t[:int(rng.integers(1, len(t) + 1))]
        if cut and ours.encode(cut) != ref.encode(cut):
            bad.append(cut)
    assert not bad, bad[:3]


def test_unordered_unicode_table_is_refused(ours, vocab, tmp_path):
    """The class lookup bisects the ranges, so they must be ordered and disjoint."""
    raw = bytearray(open(os.path.join(vocab.dir, TF.UNI_FILE), "rb").read())
    raw[8:20], raw[20:32] = raw[20:32], raw[8:20]          # swap the first two ranges
    p = tmp_path / "uni_swapped"
    p.write_bytes(bytes(raw))
    err = ctypes.create_string_buffer(256)
    tok = os.path.join(vocab.dir, TF.TOK_FILE)
    assert not ours.L.cpt_load(tok.encode(), str(p).encode(), err, 256)
    assert b"not ordered" in err.value


def test_encode_matches_restatement_on_valid_fuzz(ours, vocab):
    for t in fuzz_texts(300, 6, valid=True):
        assert ours.encode(t) == vocab.encode(t.decode()), t


def test_round_trip_bytes(ours, vocab):
    """Every byte has a token here, so the tokens' bytes concatenate back to the text (for
    chunks within the 512-byte cut)."""
    for t in TEXTS[:14] + fuzz_texts(100, 7):
        b = t if isinstance(t, bytes) else t.encode()
        assert b"".join(ours.token(i) for i in ours.encode(b)) == b


def test_long_chunk_is_cut(ours, vocab):
    """A chunk is encoded from its first 512 bytes only (tokenizer.c:77)."""
    ids = ours.encode("x" * 700)
    assert sum(len(ours.token(i)) for i in ids) == 512


def test_max_ids(ours, ref):
    t = TEXTS[2] + TEXTS[11]
    full = ours.encode(t)
    for m in (1, 2, 5, len(full) - 1, len(full), len(full) + 3):
        assert ours.encode(t, m) == ref.encode(t, m) == full[:m]
    assert ours.encode(t, 0) == []


def test_missing_byte_tokens_are_dropped(tmp_path):
    """Bytes with no single-byte token are skipped (tokenizer.c:79-82)."""
    v = TF.Vocab(drop_bytes=(ord("q"), 0xC3))
    v.write(str(tmp_path))
    o = Ours(str(tmp_path))
    try:
        t = "quick Qué"
        got = o.encode(t)
        assert got == v.encode(t)
        assert b"".join(o.token(i) for i in got) == t.encode().replace(b"q", b"").replace(b"\xc3", b"")
    finally:
        o.close()


def test_bad_files_are_refused(ours, vocab, tmp_path):
    L = ours.L
    err = ctypes.create_string_buffer(256)
    tok, uni = os.path.join(vocab.dir, TF.TOK_FILE), os.path.join(vocab.dir, TF.UNI_FILE)
    raw = open(tok, "rb").read()
    cases = {"magic": b"XPT1" + raw[4:], "version": raw[:4] + b"\x02" + raw[5:],
             "truncated": raw[:len(raw) // 2], "merges cut": raw[:-5]}
    for name, data in cases.items():
        p = tmp_path / name
        p.write_bytes(data)
        assert not L.cpt_load(str(p).encode(), uni.encode(), err, 256), name
        assert err.value, name
    p = tmp_path / "uni"
    p.write_bytes(open(uni, "rb").read()[:100])
    assert not L.cpt_load(tok.encode(), str(p).encode(), err, 256)
    assert b"truncated" in err.value
    assert not L.cpt_load(b"/nonexistent/x", uni.encode(), err, 256)
    assert b"cannot open" in err.value
