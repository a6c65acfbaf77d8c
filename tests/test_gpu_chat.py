"""cp_chat through the public API (include/cachepotato.h) on the GPU against the reference's
own cp_chat (engine/api/cachepotato.c:315-378, compiled from source into oracle/_ref and run
in a child process): the same model file, the same tokenizer files, the same turns.

The model is the small synthetic geometry with the full vocabulary (151936 ids, so the ChatML
special tokens are rows of the embedding) and 128 experts (the reference's cp_open binds that
many: qwen3_moe.c:474). The tokenizer files are synthetic (tests/tok_files.py). Bar: for every
turn, the return code, every byte handed to the callback (token by token) and the cp_turn
counts and stop reason are identical."""
import os
import zlib

import numpy as np
import pytest

import cachepotato_amd as C
from cachepotato_amd import qwen3 as Q
from tests import tok_files as TF
from tests.test_v4 import SMALL, _tables

pytestmark = pytest.mark.gpu

CHAT = dict(SMALL, n_experts=128, vocab=151936)
MAX_CTX = 256
IM_END = 151645
# [message, max_new, stop after this many tokens (0: never)]: a turn that ends at max_new, a
# follow-up appended to it that the callback stops, one that finds too little room and
# restarts the conversation, and one that runs into the end of the context
TURNS = [["Hello there! What's 2+2?", 24, 0],
         ["And what about 3+3? Explain it step by step.", 16, 5],
         ["A third message, long enough that the conversation has to restart.", 150, 0],
         ["Now fill the context to its very end.", 400, 0]]


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def tok_dir(tmp_path_factory):
    return TF.Vocab().write(str(tmp_path_factory.mktemp("tok")))


def model_fd(name):
    return Q.memfd_model(Q.bind(C.lib()), CHAT, name)


def ours(path, tdir, turns, env=None):
    old = {k: os.environ.get(k) for k in (env or {})}
    os.environ.update(env or {})
    try:
        m = Q.Model(C.lib(), path, max_ctx=MAX_CTX, tokenizer_dir=tdir)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k)
            else:
                os.environ[k] = v
    out = []
    try:
        for msg, max_new, stop_after in turns:
            say(f"  ours: turn {msg[:24]!r} max_new {max_new}")
            rc, got, t = m.chat(msg, max_new, stop_after)
            out.append({"rc": rc, "tokens": [g.hex() for g in got],
                        "prompt_tokens": t.prompt_tokens, "context_tokens": t.context_tokens,
                        "generated_tokens": t.generated_tokens,
                        "context_reset": t.context_reset, "stop": t.stop,
                        "prefill_s": t.prefill_s, "decode_s": t.decode_s})
    finally:
        m.close()
    return out


def compare(got, want):
    keys = ("rc", "prompt_tokens", "context_tokens", "generated_tokens", "context_reset", "stop")
    for i, (g, w) in enumerate(zip(got, want)):
        gt, wt = g["tokens"], w["tokens"]
        same = next((j for j in range(min(len(gt), len(wt))) if gt[j] != wt[j]),
                    min(len(gt), len(wt)))
        say(f"  turn {i}: ours {[g[k] for k in keys]} ref {[w[k] for k in keys]}; callback "
            f"tokens identical for {same} of {len(wt)}; ours decode {g['decode_s'] * 1e3:.1f} "
            f"ms, reference {w['decode_s'] * 1e3:.1f} ms")
    assert len(got) == len(want)
    for g, w in zip(got, want):
        assert g["tokens"] == w["tokens"]
        assert [g[k] for k in keys] == [w[k] for k in keys]


def test_chat_turns_match_reference(cpg, tok_dir):
    from oracle.refrun import spawn_chat
    fd, path = model_fd("chat")
    try:
        got = ours(path, tok_dir, TURNS)
        want = spawn_chat(fd, tok_dir, TURNS, MAX_CTX)
    finally:
        os.close(fd)
    compare(got, want)
    stops = [w["stop"] for w in want]
    assert stops == [1, 3, 1, 2]            # max tokens, caller, max tokens, context
    assert [w["context_reset"] for w in want] == [0, 0, 1, 1]
    assert all(g["prefill_s"] > 0 and g["decode_s"] > 0 for g in got)


def test_chat_enqueued_equals_graph(cpg, tok_dir):
    """The layers enqueued kernel by kernel (CP_NO_GRAPH=1) give the same turns as the
    captured layers graph, byte for byte."""
    fd, path = model_fd("chat_graph")
    try:
        a = ours(path, tok_dir, TURNS[:2])
        b = ours(path, tok_dir, TURNS[:2], env={"CP_NO_GRAPH": "1"})
    finally:
        os.close(fd)
    for x, y in zip(a, b):
        assert x["tokens"] == y["tokens"] and x["context_tokens"] == y["context_tokens"]


def patch_im_end_row(fd, path, X, D):
    """Make <|im_end|>'s head row token X's row with every block scale doubled (its logit is
    then exactly twice X's), and store the region's new digest (CRC-32 of its bytes)."""
    b, hdr, tens, regs = _tables(path)
    ti = next(i for i, t in enumerate(tens) if t["name"] == "lm_head")
    rb = D // 32 * 34                                  # Q8_0: f16 scale + 32 int8 per block
    base = hdr["off_d"] + tens[ti]["off"]
    row = bytearray(b[base + X * rb: base + (X + 1) * rb])
    for g in range(D // 32):
        sc = np.frombuffer(bytes(row[g * 34:g * 34 + 2]), np.float16)[0]
        row[g * 34:g * 34 + 2] = np.float16(sc * 2).tobytes()
    os.pwrite(fd, bytes(row), base + IM_END * rb)
    ri = next(i for i, g in enumerate(regs) if g["lo"] <= ti < g["hi"])
    g = regs[ri]
    crc = zlib.crc32(os.pread(fd, g["len"], hdr["off_d"] + g["off"]))
    os.pwrite(fd, int(crc).to_bytes(8, "little"), hdr["off_r"] + 4 + 43 * ri + 35)


def test_chat_stops_at_im_end(cpg, tok_dir):
    """A turn ends at <|im_end|>, which is neither handed to the callback nor fed back, and the
    next turn continues after it. The synthetic weights never produce it, so its head row is
    made to win: a copy of the row of the token greedy decoding emits 10 steps in, its scales
    doubled."""
    from oracle.refrun import spawn_chat
    v = TF.Vocab()
    inv = {t: i for i, t in enumerate(v.tokens)}
    turns = [TURNS[0], ["Then?", 8, 0]]
    fd, path = model_fd("chat_eos")
    try:
        first = ours(path, tok_dir, turns[:1])[0]
        X = inv[bytes.fromhex(first["tokens"][10])]
        patch_im_end_row(fd, path, X, CHAT["d_model"])
        got = ours(path, tok_dir, turns)
        want = spawn_chat(fd, tok_dir, turns, MAX_CTX)
    finally:
        os.close(fd)
    compare(got, want)
    assert [w["stop"] for w in want] == [0, 0]         # both turns end at <|im_end|>
    assert want[0]["generated_tokens"] < 10


def test_tokenizer_next_to_the_model(cpg, tmp_path, tok_dir):
    """cp_open finds the tokenizer files in <model dir>/tokenizer (engine/api/cachepotato.c:
    187-203); a tokenizer_dir without them is refused with a reason."""
    import shutil
    path = tmp_path / "m.v4"
    Q.write_synthetic(Q.bind(C.lib()), path, **CHAT)
    shutil.copytree(tok_dir, tmp_path / "tokenizer")
    m = Q.Model(C.lib(), path, max_ctx=MAX_CTX)
    try:
        rc, got, t = m.chat("hi", 3)
        assert rc == 0 and t.generated_tokens == 3 and len(got) == 3
    finally:
        m.close()
    with pytest.raises(RuntimeError, match="not found in"):
        Q.Model(C.lib(), path, tokenizer_dir=str(tmp_path / "nowhere"))
