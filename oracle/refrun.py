"""The reference engine in a process of its own — TEST INFRASTRUCTURE AND CPU BASELINE ONLY.

The reference's thread pool is process-global and its size (and core pinning) is fixed by the
first call (engine/kernels/parallel.c:126-132), so every thread count it is run at needs its
own process. This module is that process: tests/ and bench.py start it with
`python -m oracle.refrun ...` (a child, never an exec of the caller) and read its JSON /
npz output. It loads oracle/_ref/libref.so (the reference's C sources compiled in place) and
nothing of the product library.

  moe     the MoE half of one layer (qwen3_layer with zero attention) on a synthetic
          workload of cachepotato_amd/synth.py, one call of T tokens at a time, the inputs
          cycled, for about --seconds; prints per-call microseconds (median, p10, p90).
  decode  the reference eval driver's --decode flow (tools/qwen3_eval.c:338-400) on a CPW1
          v4 model file: prefill the prompt, then greedy steps; writes tokens, per-layer
          expert ids and per-step milliseconds to --out (npz).
  chat    the reference's public API (engine/api/cachepotato.h): cp_open the model with the
          tokenizer files of --tokenizer-dir and no pager, then one cp_chat per turn of the
          --turns JSON ([message, max_new, stop_after], the callback asking to stop after
          stop_after tokens when > 0); prints each turn's return code, cp_turn fields and the
          callback's bytes (hex, one entry per token).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def affinity():
    """The CPUs this process may run on (its cgroup / taskset share)."""
    try:
        return sorted(os.sched_getaffinity(0))
    except AttributeError:
        return list(range(os.cpu_count() or 1))


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def pct(v):
    v = np.asarray(v, np.float64)
    return {"median": round(float(np.median(v)), 4), "p10": round(float(np.percentile(v, 10)), 4),
            "p90": round(float(np.percentile(v, 90)), 4), "n": int(v.size)}


def run_moe(a):
    from cachepotato_amd import synth
    from oracle.bindings import Reference
    cpus = len(affinity())
    # the workload first: a pinned pool confines this thread (and any it starts) to one core
    spec = synth.CONFIGS[a.config]
    wg, ln2, ex = synth.wgate(spec), synth.ln2(spec), synth.experts_v4(spec)
    NB = a.vectors
    X = synth.inputs(spec, a.first, NB * a.tokens)
    T = a.tokens
    ref = Reference(threads=a.threads, pin=a.pin)
    for i in range(min(3, NB)):                           # pool, page cache, branch warm-up
        ref.moe(spec, wg, ln2, ex, X[i * T:(i + 1) * T])
    times, n, t0 = [], 0, time.perf_counter()
    while time.perf_counter() - t0 < a.seconds:
        i = n % NB
        c0 = time.perf_counter()
        ref.moe(spec, wg, ln2, ex, X[i * T:(i + 1) * T])
        times.append((time.perf_counter() - c0) * 1e6)
        n += 1
    out = {"what": "moe", "config": a.config, "threads": ref.threads, "pinned": bool(a.pin),
           "tokens_per_call": T, "calls": n, "seconds": round(time.perf_counter() - t0, 3),
           "us_per_call": pct(times), "cpus_allowed": cpus, "cpu": cpu_model()}
    print(json.dumps(out), flush=True)


def run_decode(a):
    from oracle.bindings import Reference
    cpus = len(affinity())
    ref = Reference(threads=a.threads, pin=a.pin)
    ids = np.load(a.prompt, allow_pickle=False).astype(np.int32)
    w = ref.eval_decode(a.model, ids, a.gen, K=a.topk, L=a.layers, vocab=a.vocab,
                        max_seconds=a.max_seconds, route=a.route, logits0=a.logits0)
    arrays = {"tokens": w["tokens"], "step_ms": w["step_ms"],
              "prefill_ms": np.float32(w["prefill_ms"]), "threads": np.int32(ref.threads)}
    if a.route:
        arrays["route"] = w["route"]
    if "logits0" in w:
        arrays["logits0"] = w["logits0"]
    np.savez(a.out, **arrays)
    print(json.dumps({"what": "decode", "threads": ref.threads, "pinned": bool(a.pin),
                      "prompt_tokens": int(ids.size), "steps": int(len(w["tokens"])),
                      "prefill_ms": round(float(w["prefill_ms"]), 1),
                      "step_ms": pct(w["step_ms"]) if len(w["tokens"]) else None,
                      "cpus_allowed": cpus, "cpu": cpu_model()}), flush=True)


def run_chat(a):
    import ctypes as c
    L = c.CDLL(os.path.join(HERE, "_ref", "libref.so"))

    class Opt(c.Structure):           # cp_options, engine/api/cachepotato.h:32-38
        _fields_ = [("budget_mb", c.c_long), ("threads", c.c_int), ("pin_cores", c.c_int),
                    ("max_ctx", c.c_int), ("tokenizer_dir", c.c_char_p)]

    class Turn(c.Structure):          # cp_turn, engine/api/cachepotato.h:54-62
        _fields_ = [("prompt_tokens", c.c_int), ("context_tokens", c.c_int),
                    ("generated_tokens", c.c_int), ("context_reset", c.c_int),
                    ("prefill_s", c.c_double), ("decode_s", c.c_double), ("stop", c.c_int)]

    Fn = c.CFUNCTYPE(c.c_int, c.c_void_p, c.c_size_t, c.c_void_p)
    L.cp_open.restype = c.c_void_p
    L.cp_open.argtypes = [c.c_char_p, c.POINTER(Opt), c.c_char_p, c.c_size_t]
    L.cp_chat.argtypes = [c.c_void_p, c.c_char_p, c.c_int, Fn, c.c_void_p, c.POINTER(Turn)]
    L.cp_close.argtypes = [c.c_void_p]
    opt = Opt(-1, a.threads, a.pin, a.max_ctx, a.tokenizer_dir.encode())   # -1: no pager
    err = c.create_string_buffer(512)
    h = L.cp_open(a.model.encode(), c.byref(opt), err, 512)
    if not h:
        raise SystemExit("reference cp_open: " + err.value.decode())
    # its special tokens' entries get the terminating NUL its encoder's strlen() reads
    # (ref_harness.c); the vocabulary size read back checks where the tokenizer was found
    L.ref_model_tokenizer.restype = c.c_void_p
    L.ref_model_tokenizer.argtypes = [c.c_void_p]
    L.ref_tok_terminate_specials.argtypes = [c.c_void_p]
    tk = L.ref_model_tokenizer(h)
    with open(os.path.join(a.tokenizer_dir, "qwen2.5-tokenizer.bin"), "rb") as f:
        n_vocab = int.from_bytes(f.read(12)[8:12], "little")
    if c.c_uint32.from_address(tk).value != n_vocab or \
            L.ref_tok_terminate_specials(tk) != max(0, n_vocab - 151643):
        raise SystemExit("reference cp_model: the tokenizer is not where it was expected")
    out = []
    for msg, max_new, stop_after in json.load(open(a.turns)):
        got = []

        def on_token(p, n, user, got=got, stop_after=stop_after):
            got.append(c.string_at(p, n).hex() if n else "")
            return 1 if 0 < stop_after <= len(got) else 0

        t = Turn()
        rc = L.cp_chat(h, msg.encode(), max_new, Fn(on_token), None, c.byref(t))
        out.append({"rc": rc, "tokens": got, "prompt_tokens": t.prompt_tokens,
                    "context_tokens": t.context_tokens, "generated_tokens": t.generated_tokens,
                    "context_reset": t.context_reset, "stop": t.stop,
                    "prefill_s": t.prefill_s, "decode_s": t.decode_s})
    L.cp_close(h)
    print(json.dumps({"what": "chat", "threads": a.threads, "turns": out}), flush=True)


# ---------------------------------------------------------------- the caller's side


def _child(args, timeout, pass_fds=()):
    """Run `python -m oracle.refrun args` as a child and return its last JSON line."""
    import subprocess
    r = subprocess.run([sys.executable, "-m", "oracle.refrun"] + [str(x) for x in args],
                       cwd=ROOT, capture_output=True, text=True, timeout=timeout,
                       pass_fds=pass_fds)
    if r.returncode != 0:
        raise RuntimeError(f"oracle.refrun {' '.join(map(str, args[:1]))} failed "
                           f"({r.returncode}): {r.stderr[-2000:]}")
    return json.loads(r.stdout.strip().splitlines()[-1])


def spawn_moe(config, threads, pin=True, seconds=10.0, tokens=1, vectors=1000, timeout=600):
    """The reference's MoE half on workload `config` in a child at `threads` threads."""
    return _child(["moe", "--config", config, "--threads", threads, "--pin", int(pin),
                   "--seconds", seconds, "--tokens", tokens, "--vectors", vectors], timeout)


def spawn_decode(model_fd, ids, gen, threads, pin=True, route=False, max_seconds=0.0,
                 layers=0, vocab=0, topk=8, timeout=1200, logits0=False):
    """The reference's greedy decode of the model file open as descriptor `model_fd` (it is
    handed to the child, which reads /proc/self/fd/N) after prefilling `ids`. Returns the
    child's summary (step_stats: median / p10 / p90 ms) plus the arrays tokens, step_ms,
    prefill_ms[, route (L, n, K)][, logits0: the first step's logits (vocab must be given)]."""
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        pr, out = os.path.join(d, "prompt.npy"), os.path.join(d, "out.npz")
        np.save(pr, np.ascontiguousarray(ids, np.int32))
        args = ["decode", "--model", f"/proc/self/fd/{model_fd}", "--prompt", pr, "--gen", gen,
                "--threads", threads, "--pin", int(pin), "--max-seconds", max_seconds,
                "--layers", layers, "--vocab", vocab, "--topk", topk, "--out", out]
        summary = _child(args + (["--route"] if route else []) + (["--logits0"] if logits0 else []),
                         timeout, pass_fds=(model_fd,))
        summary["step_stats"] = summary.pop("step_ms")
        with np.load(out, allow_pickle=False) as z:
            summary.update({k: z[k] for k in z.files})
    return summary


def spawn_chat(model_fd, tokenizer_dir, turns, max_ctx, threads=1, timeout=1200):
    """The reference's cp_chat over `turns` ([message, max_new, stop_after]) on the model file
    open as descriptor `model_fd`, in a child process; returns the list of turn results."""
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        tj = os.path.join(d, "turns.json")
        with open(tj, "w") as f:
            json.dump(turns, f)
        args = ["chat", "--model", f"/proc/self/fd/{model_fd}", "--tokenizer-dir", tokenizer_dir,
                "--turns", tj, "--max-ctx", max_ctx, "--threads", threads, "--pin", 0]
        return _child(args, timeout, pass_fds=(model_fd,))["turns"]


def baseline_threads():
    """N of the reference's multi-thread arm: its own physical-core count
    (cp_physical_cores, engine/api/cachepotato.c:59-80) capped at its pool's 64
    (engine/kernels/parallel.c:13), and at the CPUs this process may use and the machine's
    declared share for one job (OMP_NUM_THREADS), whichever are smaller."""
    import ctypes
    from oracle.bindings import REF_SO
    phys = ctypes.CDLL(REF_SO).cp_physical_cores()
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    n = min(phys, 64, len(affinity()))
    if share > 0:
        n = min(n, share)
    return max(1, n), {"physical_cores": phys, "pool_cap": 64, "cpus_allowed": len(affinity()),
                       "OMP_NUM_THREADS": share or None}


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m oracle.refrun")
    sub = ap.add_subparsers(dest="cmd", required=True)
    m = sub.add_parser("moe")
    m.add_argument("--config", default="q4_b1")
    m.add_argument("--tokens", type=int, default=1)
    m.add_argument("--vectors", type=int, default=1000, help="calls' inputs cycled")
    m.add_argument("--first", type=int, default=0)
    m.add_argument("--seconds", type=float, default=10.0)
    d = sub.add_parser("decode")
    d.add_argument("--model", required=True)
    d.add_argument("--prompt", required=True, help=".npy of int32 token ids")
    d.add_argument("--gen", type=int, default=64)
    d.add_argument("--max-seconds", type=float, default=0.0)
    d.add_argument("--layers", type=int, default=0)
    d.add_argument("--vocab", type=int, default=0)
    d.add_argument("--topk", type=int, default=8)
    d.add_argument("--route", action="store_true")
    d.add_argument("--logits0", action="store_true")
    d.add_argument("--out", required=True)
    ch = sub.add_parser("chat")
    ch.add_argument("--model", required=True)
    ch.add_argument("--tokenizer-dir", required=True)
    ch.add_argument("--turns", required=True, help="JSON: [[message, max_new, stop_after], ...]")
    ch.add_argument("--max-ctx", type=int, default=0)
    for p in (m, d, ch):
        p.add_argument("--threads", type=int, default=1)
        p.add_argument("--pin", type=int, default=0, help="1: the reference's core pinning")
    a = ap.parse_args(argv)
    {"moe": run_moe, "decode": run_decode, "chat": run_chat}[a.cmd](a)


if __name__ == "__main__":
    main()
