#!/usr/bin/env python3
"""Benchmark of Qwen3-30B-A3B Q4 decode on one MI355X.

Default workload: the whole random-init Qwen3-30B-A3B-shaped model (48 layers, hidden 2048,
32 query / 4 key-value heads of 128, QK-RMSNorm, RoPE theta 1e6, 128 experts top-8 of
intermediate 768, vocabulary 151936; Q4_0 experts and attention, Q8_0 embedding and head),
written as a CPW1 v4 file by the C writer into memory and opened through the public API
(cp_open, cp_eval_decode): a 128-token prompt of seeded random ids, then greedy decoding. A
step is one decode token: the head's argmax, the embedding row, 48 x (attention half, MoE
half, residual), one replay of the captured HIP graph. `value` is decode tokens/s over
exactly --steps steps after --warmup untimed ones, timed by events on the stream the steps
run on, with everything resident in HBM.

Extra keys from the same invocation:
  moe_layer   the MoE half alone at decode batch 1 on the Q4_0 workload of 1000 seeded input
              vectors, 48 distinct layers cycled (16 GB of experts, beyond the 256 MB
              Infinity Cache): microseconds per layer, fraction of the HBM roofline, and the
              per-kernel times.
  roofline    the dominant kernel, k_gateup1 (gate/up projections of the 8 selected experts
              with SwiGLU, 2/3 of a layer's bytes): algorithmic bytes / its average duration,
              from an event pair bound to each of its dispatches over 1000 tokens (exact-
              routing fallbacks included and counted).
  parity      the reference engine's greedy tokens and expert choices on the same file.
  cpu_baseline the reference engine (oracle/_ref, its C sources compiled in place) on this
              host's cores: decode tok/s of the same model and MoE-layer microseconds, at one
              thread and at N threads pinned, the arms interleaved over two rounds, median /
              p10 / p90 per arm.

  python bench.py [--steps K] [--warmup W] [--config full_q4] [--no-cpu]

Other configurations: the whole model with other encodings of the reference's files,
--config full_q4exp (Q4_0 experts, Q8_0 attention) and full_q8 (everything Q8_0); the MoE half
alone, one JSON line each: --config q4_b1, q8_b1, q4_b16_zipf, q4_prefill512; --config copy
(counter calibration), readfloor (read floor).
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Qwen3-30B-A3B Q4 decode tok/s; MoE-layer µs and % of HBM roofline"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0     # dense f16 MFMA, MI355X
PROMPT_T = 128
PARITY_STEPS = 64             # greedy steps compared with the reference
KERNEL_TOKENS = 1000          # tokens over which the roofline kernel's launches are timed


def log(*a):
    print(*a, file=sys.stderr, flush=True)


TOKENS = {"q8_b1": 1, "q4_b1": 1, "q4_b16_zipf": 16, "q4_prefill512": 512}
MFMA_MIN_T = 8      # batches from this size run the expert products as MFMA GEMMs

# HBM bytes per launch of the roofline kernel, measured by rocprofv3 --pmc FETCH_SIZE and then
# WRITE_SIZE on this script (KiB per dispatch), FETCH scaled by 1.99926 and WRITE by 1.0: the
# factors that make the counters read 64 MiB for a 64 MiB device copy (--config copy). Where
# only FETCH_SIZE was measured the entry is None.
TRAFFIC = {"q4_b1": 14448421, "q4_b16_zipf": 96668058, "q4_prefill512": 306432418}
TRAFFIC_SOURCE = ("rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, of bench.py --config {config} "
                  "--no-cpu --steps 50, calibrated on a 64 MiB device copy")


def algorithmic_bytes(spec, T=1, U=None):
    """Bytes a step of T tokens must move: each distinct weight byte once (U distinct experts,
    exactly K for one token), activations once; and the experts' algorithmic flops."""
    bb = {4: 18, 8: 34}[spec.enc]
    D, F, K, E = spec.D, spec.F, spec.K, spec.E
    U = K if U is None or T == 1 else U
    TK = T * K
    wgu, wd = U * 2 * F * (D // 32) * bb, U * D * (F // 32) * bb
    if T == 1:        # k_gateup1 writes h; k_down1 reads h and adds into mlp
        gate_up = wgu + D * 4 + TK * F * 4
        down = wd + TK * F * 4 + TK * 4 + D * 4 * 2
    else:             # the gate/up GEMVs or GEMMs write h per pair; the down ones y per pair
        gate_up = wgu + T * D * 4 + TK * F * 4
        down = wd + TK * F * 4 + TK * D * 4
    router = E * D * 4 + T * D * 4 * 3 + TK * 8
    return dict(gate_up=int(gate_up), down=int(down), router=router,
                layer=int(U * (3 * F * (D // 32) * bb) + router + T * D * 4 * 2),
                flops_gate_up=TK * 2 * 2 * D * F, flops_down=TK * 2 * D * F,
                gate_up_kernel=(("k_gateup1" if T == 1 else "k_gateup_mm") +
                                ("<Q4_0>" if spec.enc == 4 else "<Q8_0>") if T < MFMA_MIN_T else
                                "k_pf_gemm<%s, gate/up>" % ("Q4_0" if spec.enc == 4 else "Q8_0")),
                down_kernel=("k_down1" if T == 1 else "k_down_mm" if T < MFMA_MIN_T else
                             "k_pf_gemm<%s, down>" % ("Q4_0" if spec.enc == 4 else "Q8_0")))


def full_model_bytes(c):
    """Algorithmic bytes of one decode token: every weight byte the token reads once (the K
    selected experts of each layer, attention, router, norms, the head), without the KV reads
    (4 KiB per layer per cached position, reported apart)."""
    blk = {4: 18, 8: 34}
    mat = lambda enc, r, k: r * k // 32 * blk[enc]
    D, H, KV, HD, E, K, F, V = (c[k] for k in ("d_model", "n_heads", "n_kv", "head_dim",
                                                "n_experts", "topk", "d_exp", "vocab"))
    ea, ee, eh, em = c["enc_attn"], c["enc_exp"], c["enc_head"], c["enc_embed"]
    attn = mat(ea, (H + 2 * KV) * HD, D) + mat(ea, D, H * HD) + 4 * (2 * D + 2 * HD)
    moe = E * D * 4 + K * (2 * mat(ee, F, D) + mat(ee, D, F))
    return c["n_layers"] * (attn + moe) + mat(eh, V, D) + D // 32 * blk[em] + 4 * D


# the whole-model workloads: the encodings of the reference's model files (the shipped Q4_0
# experts and attention; Q4_0 experts only; everything Q8_0, the reference's exact default),
# Q8_0 embedding and head in each, and the MoE-half configuration measured beside each
FULL = {"full_q4": ("Q4_0 experts and attention, Q8_0 embedding/head", 4, 4, "q4_b1"),
        "full_q4exp": ("Q4_0 experts, Q8_0 attention/embedding/head", 8, 4, "q4_b1"),
        "full_q8": ("Q8_0 experts, attention, embedding and head", 8, 8, "q8_b1")}


# ---------------------------------------------------------------- the MoE half alone

def moe_measure(config, steps, warmup, n_layers=48, experts="auto", kernel_tokens=KERNEL_TOKENS):
    """The MoE half on workload `config`: `steps` cpg_moe_forward calls timed by two events,
    cycling `n_layers` distinct layers; then every kernel's launches timed one by one (an event
    pair bound to each dispatch) over `kernel_tokens` tokens. Returns a dict of the figures."""
    import cachepotato_amd as C
    from cachepotato_amd import synth
    spec0 = synth.CONFIGS[config]
    T = TOKENS[config]
    L = C.lib()
    C.check(L.cpg_moe_expert_mode({"auto": C.EXPERTS_AUTO, "gemv": C.EXPERTS_GEMV,
                                   "mfma": C.EXPERTS_MFMA}[experts]), "expert mode")
    t0 = time.time()
    eb = L.cpg_expert_bytes(spec0.enc, spec0.D, spec0.F)
    layers, keep = [], []
    for l in range(n_layers):
        spec = spec0.with_layer(l)
        ex = C.DeviceBuffer(eb * spec.E)
        C.check(L.cpg_gen_experts(spec.enc, spec.seed, l, spec.D, spec.E, spec.F, ex.ptr), "gen")
        wg = C.to_device(synth.wgate(spec))
        ln = C.to_device(synth.ln2(spec))
        keep += [ex, wg, ln]
        layers.append(C.MoELayer(spec.D, spec.E, spec.K, spec.F, spec.enc, spec.eps, ln.ptr,
                                 wg.ptr, ex.ptr))
    C.sync()
    log(f"moe layer ({config}): generated {n_layers} layers "
        f"({n_layers * eb * spec0.E / 1e9:.1f} GB of experts) in {time.time() - t0:.1f}s")
    NB = 1000 if T == 1 else 4          # input vectors: 1000 single tokens, or 4 batches of T
    X = C.to_device(synth.inputs(spec0, 0, NB * T))
    mlp = C.DeviceBuffer(T * spec0.D * 4).zero()
    ws = L.cpg_moe_ws_create(spec0.D, spec0.E, spec0.K, spec0.F, T)
    D4 = spec0.D * 4

    def step(s):
        lay = layers[s % n_layers]
        return L.cpg_moe_forward(ctypes.byref(lay), X.ptr + (s % NB) * T * D4, None, T, None,
                                 None, None, None, mlp.ptr, ws)

    U = []                               # distinct experts per call, over every (layer, batch)
    for s in range(math.lcm(n_layers, NB) if T > 1 else 0):  # pair the timed steps cycle through
        C.check(step(s), "forward")
        U.append(L.cpg_moe_ws_distinct(ws))
    U = float(np.mean(U)) if T > 1 else float(spec0.K)
    for s in range(warmup):
        C.check(step(s), "forward")
    C.sync()
    C.check(L.cpg_event_record(0), "event")
    for s in range(steps):
        rc = step(warmup + s)
        if rc:
            C.check(rc, "forward")
    C.check(L.cpg_event_record(1), "event")
    C.sync()
    ms_per_step = L.cpg_event_elapsed_ms(0, 1) / steps

    nk = max(8 if T > 16 else 1, kernel_tokens // T)   # calls whose kernels are timed one by one

    def kernel_times():
        fb0 = L.cpg_moe_ws_fallbacks(ws)
        C.check(L.cpg_moe_timing(1), "timing")
        for s in range(nk):
            C.check(step(s), "forward")
        kms = (ctypes.c_double * C.KT_COUNT)()
        kn = (ctypes.c_int * C.KT_COUNT)()
        C.check(L.cpg_moe_timing_read(kms, kn, C.KT_COUNT), "timing")
        C.check(L.cpg_moe_timing(0), "timing")
        kus = {C.KT_NAMES[k]: (kms[k] / kn[k] * 1e3 if kn[k] else 0.0) for k in range(C.KT_COUNT)}
        klaunch = {C.KT_NAMES[k]: kn[k] / nk for k in range(C.KT_COUNT)}
        return kus, klaunch, L.cpg_moe_ws_fallbacks(ws) - fb0

    kus, klaunch, fallbacks = kernel_times()
    L.cpg_moe_ws_destroy(ws)
    B = algorithmic_bytes(spec0, T, U)
    gu_us, dn_us = kus["gateup"], kus["down"]
    gu_gbs = B["gate_up"] / (gu_us * 1e-6) / 1e9
    dn_gbs = B["down"] / (dn_us * 1e-6) / 1e9
    layer_us = ms_per_step * 1e3
    enc = "Q4_0" if spec0.enc == 4 else "Q8_0"
    kind = "decode, batch 1" if T == 1 else (f"decode, batch {T}" if T <= 16 else
                                              f"prefill chunk of {T} tokens")
    out = {
        "workload": f"Qwen3-30B-A3B MoE layer {kind}, {enc} experts (D={spec0.D}, E={spec0.E}, "
                    f"top-{spec0.K}, F={spec0.F}), f32 router/norm, {n_layers} distinct layers "
                    f"cycled, {NB * T} input vectors",
        "tokens_per_call": T, "steps": steps, "warmup": warmup,
        "us_per_moe_layer": round(layer_us, 3),
        "tok_s": round(T * 1e6 / layer_us, 1),
        "distinct_experts_per_step": U,
        "moe_layer_frac_hbm": round(B["layer"] / (layer_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm", "kernel": B["gate_up_kernel"],
            "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
            "traffic": TRAFFIC.get(config),
            "traffic_source": TRAFFIC_SOURCE.format(config=config) if TRAFFIC.get(config) else None,
            "bytes_per_launch": B["gate_up"], "us_per_launch": round(gu_us, 3),
            "launches_timed": int(round(klaunch["gateup"] * nk)),
            "exact_routing_fallbacks": f"{fallbacks} of {nk * T} tokens",
        },
        "kernels": {
            "route": {"us_per_step": round(kus["route"] * klaunch["route"], 3)},
            "select": {"us_per_step": round(kus["select"] * klaunch["select"], 3)},
            "gateup": {"kernel": B["gate_up_kernel"], "us_per_launch": round(gu_us, 3),
                       "bytes_per_launch": B["gate_up"], "GB/s": round(gu_gbs, 1),
                       "frac": round(gu_gbs / HBM_PEAK_GBS, 4)},
            "down": {"kernel": B["down_kernel"], "us_per_launch": round(dn_us, 3),
                     "bytes_per_launch": B["down"], "GB/s": round(dn_gbs, 1),
                     "frac": round(dn_gbs / HBM_PEAK_GBS, 4)},
            "combine": {"us_per_step": round(kus["combine"] * klaunch["combine"], 3)},
            "expert_gemvs": {"us": round(gu_us + dn_us, 3),
                             "frac": round((B["gate_up"] + B["down"]) / ((gu_us + dn_us) * 1e-6)
                                           / 1e9 / HBM_PEAK_GBS, 4)},
        },
    }
    if T >= MFMA_MIN_T:
        fl_gu, fl_dn = B["flops_gate_up"], B["flops_down"]
        out["mfma"] = {"flops_gate_up": fl_gu, "flops_down": fl_dn,
                       "tflops_gate_up": round(fl_gu / (gu_us * 1e-6) / 1e12, 2),
                       "tflops_down": round(fl_dn / (dn_us * 1e-6) / 1e12, 2),
                       "peak_tflops_f16": MFMA_PEAK_TFLOPS,
                       "frac_gate_up": round(fl_gu / (gu_us * 1e-6) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                       "note": "algorithmic flops (each token's 8 experts); the MFMA runs hi and "
                               "lo halves of the activations, twice these flops"}
    del keep, layers, X, mlp
    return out


# ---------------------------------------------------------------- the CPU baseline

def cpu_arms(model_fd, ids, cfg, seconds, moe_config="q4_b1"):
    """The reference engine's arms, each in a child process (its pool is process-global):
    decode of the model at N threads (the 128-token prompt, then greedy steps) and at one
    thread (a 1-token prompt, then steps for about `seconds`), and the MoE half of config
    q4_b1 at N and at one thread, all pinned (CP_PIN_CORES). Two rounds, the second in the
    reverse order, so that no arm always runs on a cold or a warm machine."""
    from oracle.refrun import spawn_moe, spawn_decode, baseline_threads
    N, why = baseline_threads()
    arms = {"decode_Nt": [], "decode_1t": [], "moe_Nt": [], "moe_1t": []}
    parity = None
    order = ["moe_1t", "moe_Nt", "decode_Nt", "decode_1t"]
    for rnd in range(2):
        for arm in (order if rnd == 0 else order[::-1]):
            th = N if arm.endswith("Nt") else 1
            t0 = time.time()
            if arm.startswith("moe"):
                r = spawn_moe(moe_config, th, pin=True, seconds=seconds / 2)
                arms[arm].append(r)
                log(f"cpu {arm} round {rnd}: {r['calls']} calls, median "
                    f"{r['us_per_call']['median']:.0f} us ({time.time() - t0:.1f}s)")
            elif th == N:
                gen = PARITY_STEPS if rnd == 0 else 24
                r = spawn_decode(model_fd, ids, gen, th, pin=True, route=rnd == 0,
                                 layers=cfg["n_layers"], vocab=cfg["vocab"], topk=cfg["topk"])
                if rnd == 0:
                    parity = r
                arms[arm].append(r)
                log(f"cpu {arm} round {rnd}: prefill {float(r['prefill_ms']):.0f} ms, {r['steps']} "
                    f"steps median {r['step_stats']['median']:.1f} ms ({time.time() - t0:.1f}s)")
            else:
                r = spawn_decode(model_fd, ids[:1], 64, 1, pin=True, max_seconds=seconds,
                                 layers=cfg["n_layers"], vocab=cfg["vocab"], topk=cfg["topk"])
                arms[arm].append(r)
                log(f"cpu {arm} round {rnd}: {r['steps']} steps median "
                    f"{r['step_stats']['median']:.0f} ms ({time.time() - t0:.1f}s)")

    def pooled(key, field):
        v = np.concatenate([np.atleast_1d(r[field]) for r in arms[key]]).astype(np.float64)
        return {"median": round(float(np.median(v)), 3), "p10": round(float(np.percentile(v, 10)), 3),
                "p90": round(float(np.percentile(v, 90)), 3), "n": int(v.size),
                "round_medians": [round(float(np.median(np.atleast_1d(r[field]))), 3)
                                  for r in arms[key]]}

    def moe_pooled(key):
        return {"us_per_call_median": [r["us_per_call"]["median"] for r in arms[key]],
                "us_per_call_p10": [r["us_per_call"]["p10"] for r in arms[key]],
                "us_per_call_p90": [r["us_per_call"]["p90"] for r in arms[key]],
                "calls": [r["calls"] for r in arms[key]]}

    dN, d1 = pooled("decode_Nt", "step_ms"), pooled("decode_1t", "step_ms")
    summary = {
        "value": round(1e3 / dN["median"], 3), "unit": "tok/s", "cores": N, "kind": "reference",
        "sample": (f"the same model file and prompt: {PROMPT_T}-token prefill then greedy steps "
                   f"({dN['n']} steps over 2 rounds) through the reference's own block "
                   f"functions at CP_THREADS={N}, pinned; value = 1000 / median step ms"),
        "threads_rule": why,
        "cpu": arms["decode_Nt"][0].get("cpu"),
        "arms": {
            "decode_step_ms_N_threads": dN,
            "decode_step_ms_1_thread": dict(d1, note="1-token prompt, steps for ~%ds per round"
                                            % seconds),
            "decode_tok_s_1_thread": round(1e3 / d1["median"], 3),
            "prefill_ms_N_threads": [round(float(r["prefill_ms"]), 1) for r in arms["decode_Nt"]],
            "moe_layer_us_N_threads": moe_pooled("moe_Nt"),
            "moe_layer_us_1_thread": moe_pooled("moe_1t"),
        },
    }
    return summary, parity


# ---------------------------------------------------------------- the whole model

def full_main(a):
    import cachepotato_amd as C
    from cachepotato_amd import qwen3 as Q
    C.init(0)
    dev = C.device_name()
    log("device:", dev)
    what, enc_attn, enc_exp, moe_config = FULL[a.config]
    cfg = dict(Q.QWEN3_30B_A3B, enc_attn=enc_attn, enc_exp=enc_exp)
    K, W = a.steps, a.warmup
    gen = max(W + K, PARITY_STEPS)
    t0 = time.time()
    fd, path = Q.memfd_model(Q.bind(C.lib()), cfg, "qwen3_30b_a3b_" + a.config)
    fbytes = os.fstat(fd).st_size
    log(f"wrote the {fbytes / 1e9:.2f} GB CPW1 v4 file in {time.time() - t0:.1f}s")
    ids = np.random.default_rng(20261017).integers(0, cfg["vocab"], PROMPT_T).astype(np.int32)
    t0 = time.time()
    m = Q.Model(C.lib(), path, max_ctx=PROMPT_T + gen)
    log(f"cp_open (upload + device form of {cfg['n_layers']} layers) {time.time() - t0:.1f}s")
    m.eval_decode(ids[:16], 8)                   # warm-up: first launches, graph capture
    r = m.eval_decode(ids, gen, route=True)
    m.close()
    step = r["step_ms"].astype(np.float64)
    timed_ms = float(step[W:W + K].sum())        # events between steps W and W + K
    tok_s = K / (timed_ms * 1e-3)
    B = full_model_bytes(cfg)
    med = float(np.median(step[W:W + K]))
    log(f"decode: {tok_s:.1f} tok/s over steps {W}..{W + K - 1} (median step {med:.3f} ms); "
        f"prefill {PROMPT_T} tokens {r['prefill_s'] * 1e3:.1f} ms")
    moe = moe_measure(moe_config, a.moe_steps, 200)
    log(f"moe layer: {moe['us_per_moe_layer']:.2f} us, k_gateup1 {moe['roofline']['us_per_launch']:.2f}"
        f" us ({moe['roofline']['frac']:.3f} of HBM), fallbacks "
        f"{moe['roofline']['exact_routing_fallbacks']}")
    roof = dict(moe["roofline"])
    roof["workload"] = ("the MoE half alone, decode batch 1, %s, 1000 input vectors, 48 "
                        "layers cycled (the kernel is the same in every decode layer)"
                        % ("Q4_0" if enc_exp == 4 else "Q8_0"))
    out = {
        "metric": METRIC if a.config == "full_q4" else METRIC.replace(" Q4 ", " %s " % a.config),
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(timed_ms / K, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "random-init Qwen3-30B-A3B-shaped model, 48 layers, hidden 2048, "
                               "32/4 heads of 128, 128 experts top-8 of 768, vocab 151936; "
                               + what + "; 128-token prompt of seeded random ids, then greedy "
                               "decode (graph-replayed steps)",
                   "global_batch": 1, "seq_len": PROMPT_T + gen, "parallelism": "none (1 GPU)"},
        "roofline": roof,
        "decode": {"step_ms": {"median": round(med, 4),
                               "p10": round(float(np.percentile(step[W:W + K], 10)), 4),
                               "p90": round(float(np.percentile(step[W:W + K], 90)), 4)},
                   "steps_decoded": gen, "prefill_ms": round(float(r["prefill_s"]) * 1e3, 2),
                   "wall_ms_all_steps": round(float(r["decode_s"]) * 1e3, 2),
                   "bytes_per_token": B,
                   "step_frac_hbm": round(B / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "moe_layer": {k: moe[k] for k in ("workload", "us_per_moe_layer", "moe_layer_frac_hbm",
                                          "kernels", "steps")},
        "us_per_moe_layer": moe["us_per_moe_layer"],
        "moe_layer_frac_hbm": moe["moe_layer_frac_hbm"],
        "file_bytes": fbytes, "device": dev,
    }
    if not a.no_cpu:
        from oracle.bindings import REF_SO
        if os.path.exists(REF_SO):
            cpu, w = cpu_arms(fd, ids, cfg, a.cpu_seconds, moe_config)
            n = len(w["tokens"])
            gt, wt = r["tokens"][:n], w["tokens"]
            same = int(np.argmax(gt != wt)) if np.any(gt != wt) else n
            rr, wr = r["route"][:, :n], w["route"]
            agree = float(np.mean([set(x) == set(y) for x, y in
                                   zip(rr.reshape(-1, cfg["topk"]), wr.reshape(-1, cfg["topk"]))]))
            out["parity"] = {"steps_compared": n, "tokens_identical_steps": same,
                             "route_set_agreement": round(agree, 5),
                             "distinct_tokens": len(set(gt.tolist())),
                             "first_tokens": [int(t) for t in gt[:12]]}
            out["cpu_baseline"] = cpu
            log(f"parity: tokens identical for {same}/{n} steps, route agreement {agree:.4f}")
        else:
            out["cpu_baseline"] = None
    else:
        out["cpu_baseline"] = None
    os.close(fd)
    print(json.dumps(out), flush=True)


def moe_main(a):
    """One MoE-half configuration as its own line (profiling and the other workloads)."""
    import cachepotato_amd as C
    C.init(0)
    dev = C.device_name()
    log("device:", dev)
    r = moe_measure(a.config, a.steps, a.warmup, a.layers, a.experts)
    out = {"metric": f"MoE-layer tok/s ({a.config})", "value": r["tok_s"], "unit": "tok/s",
           "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
           "ms_per_step": round(r["us_per_moe_layer"] / 1e3, 6), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
           "config": {"workload": r["workload"], "global_batch": r["tokens_per_call"],
                      "parallelism": "none (1 GPU)"}}
    out.update({k: v for k, v in r.items() if k not in ("workload", "tok_s")})
    out["device"] = dev
    out["cpu_baseline"] = None
    if not a.no_cpu:
        from oracle.bindings import REF_SO
        if os.path.exists(REF_SO):
            from oracle.refrun import spawn_moe, baseline_threads
            N, why = baseline_threads()
            T = TOKENS[a.config]
            res = spawn_moe(a.config, N, pin=True, seconds=a.cpu_seconds, tokens=T,
                            vectors=1000 if T == 1 else 4)
            out["cpu_baseline"] = {"value": round(T * 1e6 / res["us_per_call"]["median"], 2),
                                   "unit": "tok/s", "cores": N, "kind": "reference",
                                   "sample": f"{res['calls']} calls of {T} token(s), the inputs "
                                             f"cycled, reference qwen3_layer at CP_THREADS={N} "
                                             f"pinned; value from the median call",
                                   "us_per_call": res["us_per_call"], "threads_rule": why}
    print(json.dumps(out), flush=True)


COPY_BYTES = 64 << 20


def copy_main():
    """The counter calibration: five device-to-device copies of 64 MiB (the runtime's copy
    kernel), each reading and writing COPY_BYTES once. rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    of this run give what those counters report for known bytes."""
    import cachepotato_amd as C
    C.init(0)
    src = C.DeviceBuffer(COPY_BYTES).zero()
    dst = C.DeviceBuffer(COPY_BYTES)
    for _ in range(5):
        C.check(C.lib().cpg_d2d(dst.ptr, src.ptr, COPY_BYTES), "cpg_d2d")
    C.sync()
    print(json.dumps({"copy_calibration": {"bytes_read_per_copy": COPY_BYTES,
                                           "bytes_written_per_copy": COPY_BYTES, "copies": 5}}))


def readfloor_main():
    """The read floor: a plain streaming-read kernel (cpg_read_stream) of 1 MB to 256 MB,
    each launch timed on its own by an event pair (with a sync between launches, as one
    dependent kernel of a decode step runs) and back to back, over a 2 GiB pool read at
    rotating offsets so that no launch finds its bytes in the 256 MB Infinity Cache."""
    import cachepotato_amd as C
    C.init(0)
    L = C.lib()
    pool_bytes = 2 << 30
    pool = C.DeviceBuffer(pool_bytes).zero()
    out = C.DeviceBuffer(4).zero()
    unit = 64 << 10
    rows = []
    for mb, div in [(m, d) for m in (1, 2, 4, 7, 14, 21, 28, 64, 128, 256) for d in (1, 2, 4)]:
        size = mb << 20
        grid = max(1, min(2048, size // unit // div))
        size = size // (unit * grid) * (unit * grid)
        nrot = pool_bytes // size
        for r in range(4):
            C.check(L.cpg_read_stream(pool.ptr + (r % nrot) * size, size, grid, out.ptr), "read")
        C.sync()
        n = 40
        iso = []
        for r in range(n):
            C.check(L.cpg_event_record(0), "event")
            C.check(L.cpg_read_stream(pool.ptr + ((r + 4) % nrot) * size, size, grid, out.ptr), "read")
            C.check(L.cpg_event_record(1), "event")
            C.sync()
            iso.append(L.cpg_event_elapsed_ms(0, 1) * 1e3)
        C.check(L.cpg_event_record(0), "event")
        for r in range(n):
            C.check(L.cpg_read_stream(pool.ptr + ((r + 4 + n) % nrot) * size, size, grid, out.ptr), "read")
        C.check(L.cpg_event_record(1), "event")
        C.sync()
        b2b = L.cpg_event_elapsed_ms(0, 1) * 1e3 / n
        med = float(np.median(iso))
        rows.append({"bytes": size, "grid": grid, "isolated_us": round(med, 2),
                     "isolated_GBps": round(size / med / 1e3, 1),
                     "back_to_back_us": round(b2b, 2), "back_to_back_GBps": round(size / b2b / 1e3, 1)})
        log(json.dumps(rows[-1]))
    print(json.dumps({"read_floor": rows, "hbm_peak_GBps": HBM_PEAK_GBS}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed steps (decode tokens)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="full_q4")
    ap.add_argument("--layers", type=int, default=48, help="MoE configs: distinct layers cycled")
    ap.add_argument("--moe-steps", type=int, default=2000,
                    help="full_q4: MoE-layer calls timed for the moe_layer keys")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="CPU work per reference arm and round (about)")
    ap.add_argument("--experts", choices=("auto", "gemv", "mfma"), default="auto",
                    help="expert path for T > 1 (cpg_moe_expert_mode)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {a.gpus}); sharding the experts over GPUs is a design only",
              file=sys.stderr)
        sys.exit(2)
    if a.steps <= 0 or a.warmup < 0:
        sys.exit("--steps must be positive and --warmup non-negative")
    if a.config in FULL:
        return full_main(a)
    if a.config == "copy":
        return copy_main()
    if a.config == "readfloor":
        return readfloor_main()
    if a.config not in TOKENS:
        sys.exit(f"unknown --config {a.config}")
    return moe_main(a)


if __name__ == "__main__":
    main()
