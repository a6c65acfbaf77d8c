"""The block / port interface (include/qwen3_moe.h) on the GPU against the reference engine's
own implementation of the same functions (engine/blocks/qwen3_moe.c, compiled from source in
oracle/_ref), both loading the same CPW1 v4 file.

Bars: attention output within 1e-4 and MoE output within 1e-3 (normwise relative error);
router logits within 1e-4; top-k indices identical wherever the reference's own top-k gap
(the k-th vs (k+1)-th logit) exceeds 1e-4, i.e. wherever fp32 differences in the attention
projections upstream of the router cannot reorder it (they are never allowed to differ
elsewhere); qwen3_mm within 1e-5 of the reference on file tensors of every encoding."""
import ctypes
import os

import numpy as np
import pytest

import cachepotato_amd as C
from cachepotato_amd import qwen3 as Q
from tests.gpu_helpers import rel_err

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    from tests.test_v4 import SMALL
    p = tmp_path_factory.mktemp("blk") / "small.v4"
    Q.write_synthetic(Q.bind(C.lib()), p, **SMALL)
    return p, SMALL


@pytest.fixture(scope="module")
def ref_lib():
    from oracle.bindings import REF_SO, Reference
    Reference(threads=1)        # start the reference pool (scalar Q4 numerics)
    return Q.bind(ctypes.CDLL(REF_SO), extra=False)


def _run(lib, path, layer, X, steps, cap=32):
    m = Q.QW3Layer()
    assert lib.qwen3_load_v4(ctypes.byref(m), str(path).encode(), layer) == 0
    kv = Q.QW3KV()
    assert lib.qwen3_kv_alloc(ctypes.byref(kv), ctypes.byref(m), cap) == 0
    outs = []
    for pos0, T in steps:
        o = Q.QW3Out()
        assert lib.qwen3_layer_alloc(ctypes.byref(o), ctypes.byref(m), T) == 0
        x = np.ascontiguousarray(X[pos0:pos0 + T], np.float32)
        assert lib.qwen3_layer_kv(ctypes.byref(m), x.ctypes.data, T, pos0, ctypes.byref(kv),
                                  ctypes.byref(o)) == 0
        outs.append(Q.out_arrays(o, T, m.d_model, m.n_experts, m.topk))
        lib.qwen3_layer_free(ctypes.byref(o))
    lib.qwen3_kv_free(ctypes.byref(kv))
    lib.qwen3_layer_free_weights(ctypes.byref(m))
    return outs


def test_layer_kv_vs_reference(cpg, model_file, ref_lib):
    path, s = model_file
    ours = Q.bind(C.lib())
    X = C.gen_normal(s["seed"], C.stream_id(0, C.K_INPUT, 9), 16 * s["d_model"], 1.0).reshape(16, -1)
    steps = [(0, 6), (6, 1), (7, 3), (10, 1)]
    for layer in range(s["n_layers"]):
        got = _run(ours, path, layer, X, steps)
        want = _run(ref_lib, path, layer, X, steps)
        for (pos0, T), g, w in zip(steps, got, want):
            ea, em, er = rel_err(g["attn"], w["attn"]), rel_err(g["mlp"], w["mlp"]), rel_err(g["router"], w["router"])
            say(f"layer {layer} pos0={pos0} T={T}: attn {ea:.2e} mlp {em:.2e} router {er:.2e}")
            assert ea <= 1e-4 and em <= 1e-3 and er <= 1e-4
            srt = -np.sort(-w["router"], axis=1)
            K = s["topk"]
            clear = (srt[:, K - 1] - srt[:, K]) > 1e-4
            for t in range(T):
                if clear[t]:
                    assert set(g["topk"][t]) == set(w["topk"][t]), (layer, pos0, t)
            assert clear.mean() > 0.5


def test_layer_without_cache_and_range_errors(cpg, model_file, ref_lib):
    """qwen3_layer (positions 0..T-1, no cache kept) equals the first qwen3_layer_kv call; a
    range beyond the cache is refused with -1, as the reference does."""
    path, s = model_file
    ours = Q.bind(C.lib())
    X = C.gen_normal(s["seed"], C.stream_id(0, C.K_INPUT, 10), 5 * s["d_model"], 1.0).reshape(5, -1)
    m = Q.QW3Layer()
    assert ours.qwen3_load_v4(ctypes.byref(m), str(path).encode(), 0) == 0
    o = Q.QW3Out()
    assert ours.qwen3_layer_alloc(ctypes.byref(o), ctypes.byref(m), 5) == 0
    assert ours.qwen3_layer(ctypes.byref(m), X.ctypes.data, 5, ctypes.byref(o)) == 0
    a = Q.out_arrays(o, 5, m.d_model, m.n_experts, m.topk)
    kv = Q.QW3KV()
    assert ours.qwen3_kv_alloc(ctypes.byref(kv), ctypes.byref(m), 4) == 0
    assert ours.qwen3_layer_kv(ctypes.byref(m), X.ctypes.data, 5, 0, ctypes.byref(kv), ctypes.byref(o)) == -1
    ours.qwen3_kv_free(ctypes.byref(kv))
    ours.qwen3_layer_free(ctypes.byref(o))
    b = _run(ours, path, 0, X, [(0, 5)])[0]
    for k in ("attn", "router", "topk"):
        assert np.array_equal(a[k], b[k]), k
    ours.qwen3_layer_free_weights(ctypes.byref(m))


def test_mm_vs_reference(cpg, model_file, ref_lib):
    path, s = model_file
    ours = Q.bind(C.lib())
    mo, mr = Q.QW3Layer(), Q.QW3Layer()
    assert ours.qwen3_load_v4(ctypes.byref(mo), str(path).encode(), 1) == 0
    assert ref_lib.qwen3_load_v4(ctypes.byref(mr), str(path).encode(), 1) == 0
    rng = np.random.default_rng(3)
    D, H, HD = s["d_model"], s["n_heads"], s["head_dim"]
    for name, n_in, n_out in (("Wq", D, H * HD), ("Wo", H * HD, D), ("Wgate", D, s["n_experts"]),
                              ("embed", D, s["vocab"])):
        x = rng.standard_normal(n_in).astype(np.float32)
        a, b = np.empty(n_out, np.float32), np.empty(n_out, np.float32)
        ours.qwen3_mm(ctypes.byref(getattr(mo, name)), a.ctypes.data, x.ctypes.data, n_in, n_out)
        ref_lib.qwen3_mm(ctypes.byref(getattr(mr, name)), b.ctypes.data, x.ctypes.data, n_in, n_out)
        e = rel_err(a, b)
        say(f"qwen3_mm {name} enc={getattr(mo, name).enc}: {e:.2e}")
        assert e <= 1e-5
        if getattr(mo, name).enc == 0:
            assert np.array_equal(a, b)       # f32: the same serial chain
    # a tensor outside any mapped file
    w = rng.standard_normal((64, 96)).astype(np.float32)
    t = Q.QW3T(w.ctypes.data, 0)
    x = rng.standard_normal(96).astype(np.float32)
    a = np.empty(64, np.float32)
    ours.qwen3_mm(ctypes.byref(t), a.ctypes.data, x.ctypes.data, 96, 64)
    b = np.empty(64, np.float32)
    ref_lib.qwen3_mm(ctypes.byref(t), b.ctypes.data, x.ctypes.data, 96, 64)
    assert np.array_equal(a, b)
    ours.qwen3_layer_free_weights(ctypes.byref(mo))
    ref_lib.qwen3_layer_free_weights(ctypes.byref(mr))
