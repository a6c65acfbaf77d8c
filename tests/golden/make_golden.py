"""Write the golden fixtures of the MoE half from the REFERENCE ENGINE itself.

Runs only where the reference tree exists (the development container): it calls
oracle/_ref/libref.so — the reference's engine/blocks/qwen3_moe.c and
engine/kernels/kernels.c compiled from source by oracle/Makefile — through
oracle/ref_harness.c (qwen3_layer on a hand-filled layer with zero attention, the pattern of
the reference's tools/verify_qwen3_blocks.py:16-39).

Inputs are the synthetic workloads of cachepotato_amd/synth.py (counter-based generator,
reproducible on any host and on the GPU); their bytes are pinned by sha256 in the fixtures.

One fixture per (workload, reference thread count): CP_THREADS=1 takes the reference's
scalar Q4_0 loop and CP_THREADS=8 its AVX2 loop (engine/kernels/kernels.c:514-540), so the
two Q4 fixtures differ in the low bits of the MoE output and agree on routing.

Usage: python tests/golden/make_golden.py [--threads 1 8]
"""
import argparse
import hashlib
import os
import subprocess
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from cachepotato_amd import synth  # noqa: E402

# (workload, calls): each call is a list of input vector ids processed as one T-token call
PLAN = {
    "small_q4": dict(calls=[list(range(0, 8))], full=[0]),
    "small_q8": dict(calls=[list(range(0, 8))], full=[0]),
    "q4_b1": dict(calls=[[v] for v in range(1000)], full=list(range(8))),
    "q8_b1": dict(calls=[[v] for v in range(1000)], full=list(range(8))),
    "q4_b16_zipf": dict(calls=[list(range(16 * b, 16 * b + 16)) for b in range(8)], full=[0]),
    "q4_prefill512": dict(calls=[list(range(512))], full=[0]),
}
PREFILL_KEEP = list(range(0, 4)) + list(range(508, 512))   # tokens whose mlp is stored


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def spec_of(name):
    return synth.CONFIGS.get(name) or synth.SMALL[name]


def run_one(name, threads):
    from oracle.bindings import Reference
    ref = Reference(threads=threads)
    spec = spec_of(name)
    plan = PLAN[name]
    t0 = time.time()
    wg, ln2, ex = synth.wgate(spec), synth.ln2(spec), synth.experts_v4(spec)
    vids = sorted({v for c in plan["calls"] for v in c})
    X = synth.inputs(spec, 0, max(vids) + 1)
    out = dict(threads=np.int32(ref.threads), sha_wgate=sha(wg), sha_experts=sha(*ex),
               sha_inputs=sha(X))
    topk, router, mlp_norm, full_x, full_router, full_topk, full_mlp = [], [], [], [], [], [], []
    for ci, call in enumerate(plan["calls"]):
        x = X[call]
        r = ref.moe(spec, wg, ln2, ex, x)
        topk.append(r["topk"])
        router.append(r["router"])
        mlp_norm.append(np.sqrt((r["mlp"].astype(np.float64) ** 2).sum(axis=1)))
        if ci in plan["full"]:
            keep = PREFILL_KEEP if name == "q4_prefill512" else list(range(len(call)))
            full_x.append(np.array([call[k] for k in keep], np.int32))
            full_router.append(r["router"][keep])
            full_topk.append(r["topk"][keep])
            full_mlp.append(r["mlp"][keep])
    out["calls"] = np.array(plan["calls"], dtype=np.int32)
    out["topk"] = np.concatenate(topk)
    out["sha_router"] = sha(np.concatenate(router))
    out["mlp_norm"] = np.concatenate(mlp_norm)
    out["full_vec"] = np.concatenate(full_x)
    out["full_call"] = np.array(plan["full"], np.int32)
    out["full_router"] = np.concatenate(full_router)
    out["full_topk"] = np.concatenate(full_topk)
    out["full_mlp"] = np.concatenate(full_mlp)
    path = os.path.join(HERE, f"moe_{name}_t{threads}.npz")
    np.savez_compressed(path, **out)
    print(f"{path}: {len(plan['calls'])} calls in {time.time() - t0:.1f}s "
          f"({os.path.getsize(path) // 1024} KiB)", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, nargs="*", default=[1, 8])
    ap.add_argument("--only", nargs="*", default=list(PLAN))
    ap.add_argument("--child", action="store_true")
    a = ap.parse_args()
    if a.child:
        for name in a.only:
            run_one(name, a.threads[0])
        return
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    # the reference's thread pool is process-global: one child process per thread count
    procs = [subprocess.Popen([sys.executable, __file__, "--child", "--threads", str(t),
                               "--only", *a.only]) for t in a.threads]
    rc = [p.wait() for p in procs]
    if any(rc):
        sys.exit(1)


if __name__ == "__main__":
    main()
