"""The whole model through the public API (include/cachepotato.h) on the GPU against the
reference engine's own block functions run in its eval driver's --decode flow
(tools/qwen3_eval.c:338-400, compiled from source in oracle/_ref): both open the same CPW1 v4
file, prefill the same prompt ids and decode greedily.

Bar: the greedy token ids are identical at every step compared (the north-star gate is 64
steps), and the experts each layer chooses for each decoded token agree in at least 98% of
(layer, step) pairs: router inputs differ in the low bits between the engines (the attention
and expert GEMVs sum in another order), so an expert pair whose router logits are within
rounding of each other may swap; everything downstream of such a swap is what the token gate
checks."""
import ctypes
import os

import numpy as np
import pytest

import cachepotato_amd as C
from cachepotato_amd import qwen3 as Q
from cachepotato_amd import synth

pytestmark = pytest.mark.gpu

SEED = synth.SEED

# two layers of the Qwen3-30B-A3B shapes: hidden 2048, 32 Q / 4 KV heads of 128, 128 experts
# top-8 of 768, the full vocabulary; Q4_0 experts and attention, Q8_0 embedding and head
QWEN3_2L = dict(n_layers=2, d_model=2048, n_heads=32, n_kv=4, head_dim=128, n_experts=128,
                topk=8, d_exp=768, vocab=151936, rope_theta=1e6, enc_attn=Q.ENC_Q4,
                enc_exp=Q.ENC_Q4, enc_embed=Q.ENC_Q8, enc_head=Q.ENC_Q8, norm_sigma=0.1,
                seed=SEED)


def say(*a):
    print(*a, flush=True)


def prompt(n, vocab, seed=7):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)


def memfd_model(cfg, name):
    """A synthetic model file held in memory (memfd), path /proc/self/fd/N."""
    return Q.memfd_model(Q.bind(C.lib()), cfg, name)


@pytest.fixture(scope="module")
def reference():
    from oracle.bindings import Reference
    return Reference(threads=1)      # scalar Q4 numerics (kernels.c:524-539)


def run_both(cfg, path, reference, T, gen):
    ids = prompt(T, cfg["vocab"])
    m = Q.Model(C.lib(), path, max_ctx=T + gen)
    try:
        got = m.eval_decode(ids, gen, route=True)
        st = m.stats
        assert (st.n_layers, st.d_model, st.n_experts, st.topk, st.vocab, st.budget_mb) == \
            (cfg["n_layers"], cfg["d_model"], cfg["n_experts"], cfg["topk"], cfg["vocab"], -1)
    finally:
        m.close()
    want = reference.eval_decode(path, ids, gen, K=cfg["topk"], L=cfg["n_layers"],
                                 vocab=cfg["vocab"], route=True)
    return got, want


def compare(got, want, n):
    gt, wt = got["tokens"][:n], want["tokens"][:n]
    same = int(np.argmax(gt != wt)) if np.any(gt != wt) else n
    agree = np.mean([set(a) == set(b) for a, b in
                     zip(got["route"][:, :n].reshape(-1, got["route"].shape[2]),
                         want["route"][:, :n].reshape(-1, want["route"].shape[2]))])
    say(f"tokens identical for {same}/{n} steps; route sets agree in {agree:.4f} of "
        f"(layer, step) pairs")
    say("  ours:", gt.tolist())
    say("  ref: ", wt.tolist())
    return same, agree


def test_small_model_greedy_tokens(cpg, reference, tmp_path):
    from tests.test_v4 import SMALL
    path = tmp_path / "small.v4"
    Q.write_synthetic(Q.bind(C.lib()), path, **SMALL)
    got, want = run_both(SMALL, path, reference, T=16, gen=64)
    same, agree = compare(got, want, 64)
    assert same == 64 and agree >= 0.98
    assert got["step_ms"].min() > 0


@pytest.mark.parametrize("encs", ["q4exp_q4attn", "q4exp_q8attn", "q8exp_q8attn"])
def test_qwen3_shaped_two_layers_greedy_tokens(cpg, reference, encs):
    """Two Qwen3-30B-A3B-shaped layers with the full vocabulary against the reference's decode
    flow, in the encodings of the reference's files: Q4_0 experts and attention (the shipped
    file), Q4_0 experts with Q8_0 attention, and everything Q8_0 (the reference's exact
    default, README.md:111); Q8_0 embedding and head throughout."""
    exp, attn = (Q.ENC_Q4 if encs.startswith("q4") else Q.ENC_Q8,
                 Q.ENC_Q4 if encs.endswith("q4attn") else Q.ENC_Q8)
    cfg = dict(QWEN3_2L, enc_exp=exp, enc_attn=attn)
    fd, path = memfd_model(cfg, "qwen3_2l_" + encs)
    try:
        got, want = run_both(cfg, path, reference, T=32, gen=64)
    finally:
        os.close(fd)
    same, agree = compare(got, want, 64)
    say(f"  ours: prefill {got['prefill_s'] * 1e3:.1f} ms, decode "
        f"{np.median(got['step_ms']):.3f} ms/token (median); reference prefill "
        f"{want['prefill_ms']:.0f} ms, decode {np.median(want['step_ms']):.1f} ms/token")
    assert same == 64 and agree >= 0.98


def test_qwen3_30b_a3b_full_model_greedy_tokens(cpg):
    """The whole random-init Qwen3-30B-A3B-shaped model (48 layers, the full geometry, Q4_0
    experts and attention, Q8_0 embedding and head; 17.5 GB in HBM): a 128-token prompt of
    seeded ids, then 256 greedy steps through the public API with the graph-replayed step,
    against the reference engine's eval driver on the same file (a child process at N
    threads), every step compared. Gates: the logits after the prefill (cp_last_logits after
    one step) within 1e-3 of the reference's (max|a - b| / max|b|); at least 64 greedy tokens
    identical; >= 98 % of (layer, step) expert sets equal over the identical steps; a stream
    that is not one repeated token (>= 16 distinct ids in 64 steps). The first divergence, if
    any, and the expert-set agreement over all 256 steps are reported."""
    from oracle.refrun import spawn_decode, baseline_threads
    from tests.gpu_helpers import rel_err
    cfg = Q.QWEN3_30B_A3B
    T, gen, gate = 128, 256, 64
    say(f"full model: writing the {cfg['n_layers']}-layer file (memfd)")
    fd, path = Q.memfd_model(Q.bind(C.lib()), cfg, "qwen3_30b_a3b")
    try:
        ids = np.random.default_rng(20261017).integers(0, cfg["vocab"], T).astype(np.int32)
        m = Q.Model(C.lib(), path, max_ctx=T + gen)
        try:
            first = m.eval_decode(ids, 1)
            logits = m.last_logits()
            got = m.eval_decode(ids, gen, route=True)
        finally:
            m.close()
        say(f"  ours: prefill {got['prefill_s'] * 1e3:.1f} ms, decode "
            f"{np.median(got['step_ms']):.3f} ms/token (median)")
        threads, _ = baseline_threads()
        say(f"  reference: {threads} threads, prefill {T} + {gen} steps (child process)")
        want = spawn_decode(fd, ids, gen, threads, pin=False, route=True, layers=cfg["n_layers"],
                            vocab=cfg["vocab"], topk=cfg["topk"], logits0=True)
    finally:
        os.close(fd)
    assert len(want["tokens"]) == gen
    e = rel_err(logits, want["logits0"])
    say(f"  logits after the {T}-token prefill: max rel err {e:.2e}, argmax "
        f"{int(np.argmax(logits))} / {int(np.argmax(want['logits0']))}")
    assert first["tokens"][0] == got["tokens"][0] == want["tokens"][0]
    gt, wt = got["tokens"], want["tokens"]
    same = int(np.argmax(gt != wt)) if np.any(gt != wt) else gen
    sets = np.array([[set(a) == set(b) for a, b in zip(got["route"][l], want["route"][l])]
                     for l in range(cfg["n_layers"])])          # (layer, step)
    agree_same = float(sets[:, :max(same, 1)].mean())
    say(f"  tokens identical for {same}/{gen} steps"
        + (f" (first divergence at step {same}: ours {gt[same]}, reference {wt[same]})"
           if same < gen else ""))
    say(f"  expert sets agree in {agree_same:.4f} of (layer, step) pairs over the identical "
        f"steps, {float(sets.mean()):.4f} over all {gen}")
    say("  ours:", gt[:32].tolist(), "...")
    distinct = len(set(gt[:gate].tolist()))
    say(f"  {distinct} distinct ids in {gate} steps; reference prefill {want['prefill_ms']:.0f} "
        f"ms, decode {np.median(want['step_ms']):.1f} ms/token")
    assert e <= 1e-3
    assert distinct >= 16
    assert same >= gate and agree_same >= 0.98


def test_graph_replay_equals_enqueued_steps(cpg, tmp_path, monkeypatch):
    """The captured-and-replayed decode step computes the same tokens and experts as the
    same step enqueued kernel by kernel (CP_NO_GRAPH=1), bit for bit."""
    from tests.test_v4 import SMALL
    path = tmp_path / "small.v4"
    Q.write_synthetic(Q.bind(C.lib()), path, **SMALL)
    ids = prompt(12, SMALL["vocab"], seed=3)
    runs = []
    for env in ("1", None):
        if env:
            monkeypatch.setenv("CP_NO_GRAPH", env)
        else:
            monkeypatch.delenv("CP_NO_GRAPH", raising=False)
        m = Q.Model(C.lib(), path, max_ctx=64)
        try:
            runs.append(m.eval_decode(ids, 40, route=True))
            runs.append(m.eval_decode(ids, 40, route=True))     # replay after a restart
            lg = m.last_logits()
        finally:
            m.close()
        runs[-1]["logits"] = lg
    for r in runs[1:]:
        assert np.array_equal(r["tokens"], runs[0]["tokens"])
        assert np.array_equal(r["route"], runs[0]["route"])
    assert np.array_equal(runs[1]["logits"].view(np.uint32), runs[3]["logits"].view(np.uint32))


def test_api_contract(cpg, tmp_path):
    """cp_chat without tokenizer files next to the model returns -2; one model at a time; a
    missing file is refused with a reason; cp_reset and cp_get_stats behave as the
    reference's."""
    from tests.test_v4 import SMALL
    lib = Q.bind_cp(C.lib())
    path = tmp_path / "small.v4"
    Q.write_synthetic(Q.bind(C.lib()), path, **SMALL)
    err = ctypes.create_string_buffer(256)
    assert not lib.cp_open(str(tmp_path / "absent.v4").encode(), None, err, 256)
    assert b"cannot open" in err.value
    m = Q.Model(C.lib(), path)
    try:
        assert m.stats.max_ctx == 2048 and m.stats.file_bytes == os.path.getsize(path)
        with pytest.raises(RuntimeError, match="already open"):
            Q.Model(C.lib(), path)
        turn = Q.CpTurn()
        assert lib.cp_chat(m.h, b"hello", 4, Q.CpTokenFn(), None, ctypes.byref(turn)) == -2
        ids = prompt(8, SMALL["vocab"])
        a = m.eval_decode(ids, 8)
        lib.cp_reset(m.h)
        b = m.eval_decode(ids, 8)
        assert np.array_equal(a["tokens"], b["tokens"])      # deterministic, restartable
        assert a["turn"].generated_tokens == 8 and a["turn"].context_tokens == 16
        lg = m.last_logits()
        assert int(np.argmax(lg)) == int(a["tokens"][-1])
        assert lib.cp_eval_decode(m.h, ids.ctypes.data, 8, 2041, a["tokens"].ctypes.data,
                                  None, None, None) == -1       # beyond max_ctx
    finally:
        m.close()
    m2 = Q.Model(C.lib(), path)         # a new model after cp_close
    m2.close()
