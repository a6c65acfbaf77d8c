#!/usr/bin/env python3
"""Benchmark of the Qwen3-30B-A3B MoE half on one MI355X.

Workload: decode batch 1 through one Qwen3-30B-A3B-shaped MoE layer (hidden 2048, 128
experts, top-8 with softmax renormalisation, expert intermediate 768, SwiGLU) with Q4_0
expert weights quantised from seeded N(0, 0.02) f32 weights, f32 router and norm, over 1000
seeded N(0,1) input vectors. A step is one cpg_moe_forward call on one token: RMSNorm,
router GEMV, softmax/top-8/renormalise, the 8 selected experts' gate/up/down GEMVs and the
weighted combine. Steps cycle through 48 distinct layers (16 GB of expert weights) so that
the 256 MB Infinity Cache cannot hold the working set, as in real decode.

Output: one JSON line (see the keys below). `value` is MoE-layer tokens/s at batch 1 with
all inputs resident in HBM; `roofline` is for the dominant kernel (the gate/up kernel: the
selected experts' gate and up projections, 2/3 of the bytes) from HIP events bound to each of its
dispatches (hipExtLaunchKernel) on the stream it runs on; `cpu_baseline` is the reference engine
(oracle/_ref/libref.so, compiled from the reference's C sources) on this host's cores.

  python bench.py [--steps K] [--warmup W] [--layers 48] [--config q4_b1] [--no-cpu]

--config full_q4 instead runs the whole random-init Qwen3-30B-A3B-shaped model (48 layers,
hidden 2048, 32 Q / 4 KV heads of 128, QK-RMSNorm, RoPE theta 1e6, 128 experts top-8,
vocab 151936; Q4_0 experts and attention, Q8_0 embedding and head) through the public API
(cp_open, cp_eval_decode): a 128-token prompt of seeded random ids, then 256 greedy decode
steps. `value` is decode tok/s. The same file is decoded by the reference engine on the host
cores for the greedy-token comparison and the CPU baseline.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Qwen3-30B-A3B Q4 decode tok/s; MoE-layer µs and % of HBM roofline"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


TOKENS = {"q8_b1": 1, "q4_b1": 1, "q4_b16_zipf": 16, "q4_prefill512": 512}

# HBM bytes per launch of the roofline kernel, measured by rocprofv3 --pmc FETCH_SIZE and then
# WRITE_SIZE on this script (KiB per dispatch), FETCH scaled by 1.99926 and WRITE by 1.0: the
# factors that make the counters read 64 MiB for a 64 MiB device copy (--config copy). Where
# only FETCH_SIZE was measured the entry is None.
TRAFFIC = {"q4_b1": 14513366, "q4_b16_zipf": 80998138}
TRAFFIC_SOURCE = ("rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, of bench.py --steps 50 --layers 8, "
                  "calibrated on a 64 MiB device copy")
MFMA_PEAK_TFLOPS = 2500.0     # dense f16 MFMA, MI355X


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
    elif T <= 16:     # k_gateup_mm writes h per pair; k_down_mm reads it and writes y per pair
        gate_up = wgu + T * D * 4 + TK * F * 4
        down = wd + TK * F * 4 + TK * D * 4
    else:             # k_mfma_gateup writes h; k_mfma_down writes y per pair
        gate_up = wgu + T * D * 4 + TK * F * 4
        down = wd + TK * F * 4 + TK * D * 4
    router = E * D * 4 + T * D * 4 * 3 + TK * 8
    return dict(gate_up=int(gate_up), down=int(down), router=router,
                layer=int(U * (3 * F * (D // 32) * bb) + router + T * D * 4 * 2),
                flops_gate_up=TK * 2 * 2 * D * F, flops_down=TK * 2 * D * F,
                gate_up_kernel=("k_gateup1" if T == 1 else "k_gateup_mm" if T <= 16
                                else "k_mfma_gateup") + ("<Q4_0>" if spec.enc == 4 else "<Q8_0>"),
                down_kernel=("k_down1" if T == 1 else "k_down_mm" if T <= 16 else "k_mfma_down"))


def cpu_baseline(spec, seconds, threads, T=1):
    """The reference engine's qwen3_layer (MoE half, zero attention) on the same workload,
    timed on this host for about `seconds` of CPU work: calls of T tokens."""
    from cachepotato_amd import synth
    from oracle.bindings import Reference, REF_SO
    if not os.path.exists(REF_SO):
        return None
    ref = Reference(threads=threads)
    wg, ln2, ex = synth.wgate(spec), synth.ln2(spec), synth.experts_v4(spec)
    NB = 1000 if T == 1 else 4
    X = synth.inputs(spec, 0, NB * T)
    ref.moe(spec, wg, ln2, ex, X[:T])                # warm the pool and the page cache
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:        # the inputs cycle
        i = n % NB
        ref.moe(spec, wg, ln2, ex, X[i * T:(i + 1) * T])
        n += 1
    dt = time.perf_counter() - t0
    what = "decode tokens" if T == 1 else f"calls of {T} tokens"
    return {"value": round(n * T / dt, 2), "unit": "tok/s", "cores": ref.threads,
            "kind": "reference",
            "sample": f"{n} {what} (the {NB * T} input vectors cycled) through layer 0 of "
                      f"the same workload, reference qwen3_layer at CP_THREADS={ref.threads}, "
                      f"{dt:.1f} s"}


FULL_Q4 = dict(n_layers=48, d_model=2048, n_heads=32, n_kv=4, head_dim=128, n_experts=128,
               topk=8, d_exp=768, vocab=151936, rope_theta=1e6, enc_attn=4, enc_exp=4,
               enc_embed=8, enc_head=8, norm_sigma=0.1)


def full_model_bytes(c):
    """Algorithmic bytes of one decode token: every weight byte the token reads once (the K
    selected experts of each layer, attention, router, norms, the head row set) plus its KV
    reads at the final context length are excluded (reported apart)."""
    q4 = lambda r, k: r * k // 32 * 18
    q8 = lambda r, k: r * k // 32 * 34
    D, H, KV, HD, E, K, F, V = (c[k] for k in ("d_model", "n_heads", "n_kv", "head_dim",
                                                "n_experts", "topk", "d_exp", "vocab"))
    attn = q4((H + 2 * KV) * HD, D) + q4(D, H * HD) + 4 * (2 * D + 2 * HD)
    moe = E * D * 4 + K * (2 * q4(F, D) + q4(D, F))
    return c["n_layers"] * (attn + moe) + q8(V, D) + D // 32 * 34 + 4 * D


def full_main(a):
    """Config 5: the whole model, decode tok/s, greedy tokens against the reference."""
    import cachepotato_amd as C
    from cachepotato_amd import qwen3 as Q
    from cachepotato_amd import synth
    C.init(0)
    dev = C.device_name()
    log("device:", dev)
    T, gen = 128, a.gen
    cfg = dict(FULL_Q4, seed=synth.SEED)
    fd = os.memfd_create("qwen3_30b_a3b_q4")
    path = f"/proc/self/fd/{fd}"
    t0 = time.time()
    Q.write_synthetic(Q.bind(C.lib()), path, **cfg)
    fbytes = os.fstat(fd).st_size
    log(f"wrote the {fbytes / 1e9:.2f} GB CPW1 v4 file in {time.time() - t0:.1f}s")
    ids = np.random.default_rng(20261017).integers(0, cfg["vocab"], T).astype(np.int32)
    t0 = time.time()
    m = Q.Model(C.lib(), path, max_ctx=T + gen)
    log(f"cp_open (upload + device form of 48 layers) {time.time() - t0:.1f}s")
    m.eval_decode(ids[:16], 8)                     # warm-up: first launches, page-in
    r = m.eval_decode(ids, gen, route=True)
    m.close()
    tok_s = gen / r["decode_s"]
    step = r["step_ms"]
    B = full_model_bytes(cfg)
    med = float(np.median(step))
    log(f"decode: {tok_s:.1f} tok/s ({r['decode_s'] * 1e3 / gen:.3f} ms/token wall, "
        f"median step {np.median(step):.3f} ms); prefill {T} tokens {r['prefill_s'] * 1e3:.1f} ms")
    out = {
        "metric": "Qwen3-30B-A3B Q4 decode tok/s (whole model, batch 1)",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": gen, "warmup": 8,
        "ms_per_step": round(r["decode_s"] * 1e3 / gen, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "random-init Qwen3-30B-A3B-shaped model, 48 layers, Q4_0 experts "
                               "and attention, Q8_0 embedding/head, 128-token prompt of seeded "
                               "random ids then greedy decode", "global_batch": 1,
                   "seq_len": T + gen, "parallelism": "none (1 GPU)"},
        "prefill_ms": round(float(r["prefill_s"]) * 1e3, 2),
        "step_ms": {"median": round(float(np.median(step)), 4),
                    "p10": round(float(np.percentile(step, 10)), 4),
                    "p90": round(float(np.percentile(step, 90)), 4)},
        "roofline": {"bound": "hbm", "achieved": round(B / (med * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(B / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": None, "bytes_per_token": B,
                     "note": "whole decode step (all kernels) at the median step time"},
        "file_bytes": fbytes, "device": dev,
    }
    if not a.no_cpu:
        from oracle.bindings import Reference, REF_SO
        if os.path.exists(REF_SO):
            threads = min(16, os.cpu_count() or 1)
            ref = Reference(threads=threads)
            log(f"reference engine: {threads} threads, prefill + up to {a.ref_steps} steps")
            w = ref.eval_decode(path, ids, a.ref_steps, K=cfg["topk"], L=cfg["n_layers"],
                                vocab=cfg["vocab"], max_seconds=a.cpu_seconds, route=True)
            n = len(w["tokens"])
            gt, wt = r["tokens"][:n], w["tokens"]
            same = int(np.argmax(gt != wt)) if np.any(gt != wt) else n
            rr, wr = r["route"][:, :n], w["route"]
            agree = float(np.mean([set(x) == set(y) for x, y in
                                   zip(rr.reshape(-1, cfg["topk"]), wr.reshape(-1, cfg["topk"]))]))
            ref_tok_s = n / (float(np.sum(w["step_ms"])) * 1e-3)
            out["parity"] = {"steps_compared": n, "tokens_identical_steps": same,
                             "route_set_agreement": round(agree, 5),
                             "first_tokens": [int(t) for t in gt[:16]]}
            out["cpu_baseline"] = {"value": round(float(ref_tok_s), 3), "unit": "tok/s", "cores": threads,
                                   "kind": "reference",
                                   "sample": f"the same file and prompt: {T}-token prefill "
                                             f"({w['prefill_ms'] / 1e3:.1f} s) then {n} greedy "
                                             f"decode steps, reference qwen3_layer_kv at "
                                             f"CP_THREADS={threads}"}
            log(f"parity: tokens identical for {same}/{n} steps, route agreement {agree:.4f}; "
                f"reference {ref_tok_s:.2f} tok/s")
    os.close(fd)
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
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--config", default="q4_b1")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--gen", type=int, default=256, help="full_q4: greedy decode steps")
    ap.add_argument("--ref-steps", type=int, default=64, help="full_q4: reference steps")
    ap.add_argument("--experts", choices=("auto", "gemv", "mfma"), default="auto",
                    help="expert path for T > 1 (cpg_moe_expert_mode)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {a.gpus}); the expert-parallel design is described in DESIGN.md",
              file=sys.stderr)
        sys.exit(2)

    if a.config == "full_q4":
        return full_main(a)
    if a.config == "copy":
        return copy_main()
    if a.config == "readfloor":
        return readfloor_main()
    import cachepotato_amd as C
    from cachepotato_amd import synth
    spec0 = synth.CONFIGS[a.config]
    T = TOKENS[a.config]
    C.init(0)
    L = C.lib()
    dev = C.device_name()
    log("device:", dev)
    C.check(L.cpg_moe_expert_mode({"auto": C.EXPERTS_AUTO, "gemv": C.EXPERTS_GEMV,
                                   "mfma": C.EXPERTS_MFMA}[a.experts]), "expert mode")

    # ---- weights: a.layers distinct layers generated on the GPU
    t0 = time.time()
    eb = L.cpg_expert_bytes(spec0.enc, spec0.D, spec0.F)
    layers, keep = [], []
    for l in range(a.layers):
        spec = spec0.with_layer(l)
        ex = C.DeviceBuffer(eb * spec.E)
        C.check(L.cpg_gen_experts(spec.enc, spec.seed, l, spec.D, spec.E, spec.F, ex.ptr), "gen")
        wg = C.to_device(synth.wgate(spec))
        ln = C.to_device(synth.ln2(spec))
        keep += [ex, wg, ln]
        layers.append(C.MoELayer(spec.D, spec.E, spec.K, spec.F, spec.enc, spec.eps, ln.ptr,
                                 wg.ptr, ex.ptr))
    C.sync()
    log(f"generated {a.layers} layers ({a.layers * eb * spec0.E / 1e9:.1f} GB of experts) "
        f"in {time.time() - t0:.1f}s")
    # inputs: 1000 vectors for one token per step, else 4 batches of T tokens cycled
    NB = 1000 if T == 1 else 4
    X = C.to_device(synth.inputs(spec0, 0, NB * T))
    mlp = C.DeviceBuffer(T * spec0.D * 4).zero()
    ws = L.cpg_moe_ws_create(spec0.D, spec0.E, spec0.K, spec0.F, T)
    D4 = spec0.D * 4

    def step(s):
        lay = layers[s % a.layers]
        return L.cpg_moe_forward(ctypes.byref(lay), X.ptr + (s % NB) * T * D4, None, T, None,
                                 None, None, None, mlp.ptr, ws)

    # distinct experts per batch (each batch on layer 0), for the algorithmic bytes
    U = []
    for b in range(min(NB, 8)):
        C.check(step(b * a.layers), "forward")
        U.append(L.cpg_moe_ws_distinct(ws))
    U = float(np.mean(U)) if T > 1 else float(spec0.K)   # one token: its K experts, no grouping
    for s in range(a.warmup):
        C.check(step(s), "forward")
    C.sync()
    # ---- timed region: K steps between two events on the stream the kernels run on
    C.check(L.cpg_event_record(0), "event")
    for s in range(a.steps):
        rc = step(a.warmup + s)
        if rc:
            C.check(rc, "forward")
    C.check(L.cpg_event_record(1), "event")
    C.sync()
    ms = L.cpg_event_elapsed_ms(0, 1)
    ms_per_step = ms / a.steps

    # ---- per-kernel durations: each launch carries an event pair bound to its dispatch
    nk = min(a.steps, 4000)

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
    fused_us, timeouts = 0.0, 0
    if T == 1:                # the opt-in one-kernel layer, timed in a side pass for the record
        C.check(L.cpg_moe_fused(1), "fused")
        fused_us = kernel_times()[0]["fused"]
        C.check(L.cpg_moe_fused(0), "fused")
        timeouts = L.cpg_moe_ws_status(ws)
    gu_us, dn_us = kus["gateup"], kus["down"]

    B = algorithmic_bytes(spec0, T, U)
    gu_gbs = B["gate_up"] / (gu_us * 1e-6) / 1e9
    dn_gbs = B["down"] / (dn_us * 1e-6) / 1e9
    layer_us = ms_per_step * 1e3
    enc = "Q4_0" if spec0.enc == 4 else "Q8_0"
    kind = "decode, batch 1" if T == 1 else (f"decode, batch {T}" if T <= 16 else
                                              f"prefill chunk of {T} tokens")
    out = {
        "metric": METRIC,
        "value": round(T * 1e3 / ms_per_step, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"Qwen3-30B-A3B MoE layer {kind}, {enc} experts (D={spec0.D}, "
                        f"E={spec0.E}, top-{spec0.K}, F={spec0.F}), f32 router/norm, "
                        f"{a.layers} distinct layers cycled, {NB * T} input vectors",
            "global_batch": T,
            "parallelism": "none (1 GPU)",
        },
        "us_per_moe_layer": round(layer_us, 3),
        "distinct_experts_per_step": U,
        "moe_layer_frac_hbm": round(B["layer"] / (layer_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": B["gate_up_kernel"],
            "achieved": round(gu_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
            "traffic": TRAFFIC.get(a.config),
            "traffic_source": TRAFFIC_SOURCE if TRAFFIC.get(a.config) else None,
            "bytes_per_launch": B["gate_up"],
            "us_per_launch": round(gu_us, 3),
        },
        "kernels": {
            "fused_opt_in": {"kernel": "k_moe1", "us_per_launch": round(fused_us, 3),
                             "grid_barrier_timeouts": timeouts} if fused_us > 0 else None,
            "route": {"us_per_step": round(kus["route"] * klaunch["route"], 3),
                      "exact_fallbacks": f"{fallbacks} of {nk * T} tokens"},
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
        "device": dev,
    }
    if T > 16:
        fl_gu, fl_dn = B["flops_gate_up"], B["flops_down"]
        out["mfma"] = {"flops_gate_up": fl_gu, "flops_down": fl_dn,
                       "tflops_gate_up": round(fl_gu / (gu_us * 1e-6) / 1e12, 2),
                       "tflops_down": round(fl_dn / (dn_us * 1e-6) / 1e12, 2),
                       "peak_tflops_f16": MFMA_PEAK_TFLOPS,
                       "frac_gate_up": round(fl_gu / (gu_us * 1e-6) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                       "note": "algorithmic flops (each token's 8 experts); the MFMA runs hi and "
                               "lo halves of the activations, twice these flops"}
    L.cpg_moe_ws_destroy(ws)
    if not a.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        log(f"cpu baseline: reference engine, {threads} threads, ~{a.cpu_seconds:.0f}s")
        out["cpu_baseline"] = cpu_baseline(spec0, a.cpu_seconds, threads, T)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
