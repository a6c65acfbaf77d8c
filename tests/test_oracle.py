"""The oracle (oracle/oracle.c) pinned before it is trusted as the checker.

Every restated function is checked against something a plausible mistake would fail:
the reference engine compiled from source (oracle/_ref/libref.so, where present), the
golden fixtures it wrote (tests/golden/), the host glibc, and closed forms.
"""
import ctypes
import math
import os
from decimal import Decimal, getcontext

import numpy as np
import pytest

from tests.conftest import golden, ROOT
from oracle.bindings import REF_SO

HAVE_REF = os.path.exists(REF_SO)
needs_ref = pytest.mark.skipif(not HAVE_REF, reason="oracle/_ref/libref.so not built")


@pytest.fixture(scope="module")
def ref():
    from oracle.bindings import Reference
    return Reference(threads=8)


# ------------------------------------------------------------------ fp16 and dequant

def all_scale_blocks_q8():
    """65,536 scales x all 256 int8 values: 8 blocks per scale, byte i of block j = 32j+i."""
    scales = np.arange(65536, dtype=np.uint32)
    blk = np.zeros((65536, 8, 34), np.uint8)
    blk[:, :, 0] = (scales & 0xFF)[:, None]
    blk[:, :, 1] = (scales >> 8)[:, None]
    blk[:, :, 2:] = (np.arange(256, dtype=np.uint16).reshape(8, 32) & 0xFF).astype(np.uint8)
    return blk.reshape(-1)


def all_scale_blocks_q4():
    """65,536 scales x all 16 nibbles in both positions: byte k = k | (15-k) << 4."""
    scales = np.arange(65536, dtype=np.uint32)
    blk = np.zeros((65536, 18), np.uint8)
    blk[:, 0] = scales & 0xFF
    blk[:, 1] = scales >> 8
    blk[:, 2:] = np.array([k | ((15 - k) << 4) for k in range(16)], np.uint8)
    return blk.reshape(-1)


def closed_form_q8():
    d = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    q = np.arange(256, dtype=np.uint16).astype(np.uint8).view(np.int8).astype(np.float32)
    with np.errstate(invalid="ignore"):                 # 0 * inf in the NaN/inf scales
        return (q[None, :] * d[:, None]).reshape(-1)


def closed_form_q4():
    d = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    lo = np.array([k if k < 8 else k - 16 for k in range(16)], np.float32)
    hi = np.array([(15 - k) if (15 - k) < 8 else (15 - k) - 16 for k in range(16)], np.float32)
    q = np.concatenate([lo, hi])
    with np.errstate(invalid="ignore"):
        return (q[None, :] * d[:, None]).reshape(-1)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_f16_to_f32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint16)
    mine = np.array([oracle.L.or_f16_to_f32(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)     # numpy's exact widening
    nan = np.isnan(want)
    assert np.array_equal(bits(mine)[~nan], bits(want)[~nan])
    assert np.isnan(mine[nan]).all()


@pytest.mark.parametrize("enc", [4, 8])
def test_dequant_exhaustive_closed_form(oracle, enc):
    blk = all_scale_blocks_q4() if enc == 4 else all_scale_blocks_q8()
    n = 65536 * 32 if enc == 4 else 65536 * 256
    got = oracle.dequant_row(enc, blk, n)
    want = closed_form_q4() if enc == 4 else closed_form_q8()
    nan = np.isnan(want)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])
    assert np.isnan(got[nan]).all()


@needs_ref
@pytest.mark.parametrize("enc", [4, 8])
def test_dequant_exhaustive_vs_reference(oracle, ref, enc):
    blk = all_scale_blocks_q4() if enc == 4 else all_scale_blocks_q8()
    n = 65536 * 32 if enc == 4 else 65536 * 256
    a, b = oracle.dequant_row(enc, blk, n), ref.dequant_row(enc, blk, n)
    assert np.array_equal(bits(a), bits(b))


# ------------------------------------------------------------------ expf

def test_exp2_table_from_first_principles(oracle):
    """Table entry i = bits(binary64 nearest 2^(i/32)) - (i << 47), recomputed in 80 digits."""
    getcontext().prec = 80
    ln2 = Decimal(2).ln()
    for i in range(32):
        v = float(str((ln2 * i / 32).exp()))
        want = (int(np.float64(v).view(np.uint64)) - (i << 47)) & 0xFFFFFFFFFFFFFFFF
        assert oracle.L.or_exp2f_tab(i) == want, i


@pytest.mark.slow
def test_expf_exhaustive_vs_glibc(oracle):
    """All 2^32 float inputs against the host libm (glibc 2.35)."""
    fn = oracle.L.or_expf_check
    fn.restype = ctypes.c_long
    fn.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int,
                   ctypes.POINTER(ctypes.c_uint64)]
    fb = ctypes.c_uint64(0)
    bad = fn(0, 1 << 32, None, os.cpu_count() or 8, ctypes.byref(fb))
    assert bad == 0, f"{bad} mismatches, first at bits {fb.value:#010x}"


def test_expf_special_values(oracle):
    e = oracle.L.or_expf
    assert e(0.0) == 1.0 and e(-0.0) == 1.0
    assert e(float("-inf")) == 0.0 and math.isinf(e(float("inf")))
    assert math.isnan(e(float("nan")))
    assert math.isinf(e(89.0)) and e(-104.0) == 0.0
    assert e(1.0) == np.float32(math.e)


# ------------------------------------------------------------------ kernels vs reference

@needs_ref
@pytest.mark.parametrize("enc,n_in,n_out", [(4, 2048, 768), (4, 768, 2048), (4, 256, 128),
                                            (8, 2048, 768), (8, 768, 2048), (0, 2048, 128)])
def test_matmul_vs_reference(oracle, ref, enc, n_in, n_out):
    """The reference pool runs 8 threads here: n_in*n_out >= 60000 takes the AVX2 Q4 loop,
    256x128 the scalar one (kernels.c:514-540); the oracle selects the same."""
    rng = np.random.default_rng(n_in * 7 + n_out + enc)
    x = rng.normal(0, 1, n_in).astype(np.float32)
    w32 = rng.normal(0, 0.02, (n_out, n_in)).astype(np.float32)
    w = w32 if enc == 0 else oracle.encode(enc, w32.ravel())
    a = oracle.matmul(enc, w, x, n_in, n_out, threads=ref.threads)
    b = ref.matmul(enc, w, x, n_in, n_out)
    assert np.array_equal(bits(a), bits(b))


@pytest.mark.parametrize("enc", [4, 8])
@pytest.mark.parametrize("threads", [1, 8])
def test_matmul_vs_float64(oracle, enc, threads):
    """The reference's own kernel gate: quantised GEMV vs float64 dequant+matmul at 1e-5
    (tools/verify_q8_kernels.py:21,54-56)."""
    rng = np.random.default_rng(7)
    n_in, n_out = 2048, 768
    x = rng.normal(0, 1, n_in).astype(np.float32)
    w = oracle.encode(enc, rng.normal(0, 0.02, n_in * n_out).astype(np.float32))
    deq = oracle.dequant_row(enc, w, n_in * n_out).reshape(n_out, n_in).astype(np.float64)
    want = deq @ x.astype(np.float64)
    got = oracle.matmul(enc, w, x, n_in, n_out, threads=threads)
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5


@needs_ref
def test_norm_softmax_silu_vs_reference(oracle, ref):
    rng = np.random.default_rng(20261017)
    for n in (7, 128, 2048):
        x = (rng.normal(0, 3, n)).astype(np.float32)
        g = rng.normal(1, 0.1, n).astype(np.float32)
        assert np.array_equal(bits(oracle.rmsnorm(x, g, 1e-6)), bits(ref.rmsnorm(x, g, 1e-6)))
        assert np.array_equal(bits(oracle.softmax(x)), bits(ref.softmax(x)))
    for v in rng.normal(0, 8, 4096).astype(np.float32):
        assert np.float32(oracle.L.or_silu(float(v))) == np.float32(ref.L.silu(float(v)))


def test_softmax_and_rmsnorm_closed_forms(oracle):
    for n in (1, 3, 128, 1000):
        y = oracle.softmax(np.full(n, 0.37, np.float32))
        assert np.all(y == np.float32(1.0) / np.float32(n))
    x = np.full(2048, 2.0, np.float32)
    y = oracle.rmsnorm(x, np.ones(2048, np.float32), 0.0)
    assert np.all(y == np.float32(1.0))
    # a dropped eps, sign or gain would break this one
    y = oracle.rmsnorm(np.array([3.0, -4.0], np.float32), np.array([1.0, 2.0], np.float32), 0.0)
    inv = np.float32(1.0) / np.sqrt(np.float32(12.5))
    assert np.array_equal(y, np.array([np.float32(3.0) * inv, np.float32(-4.0) * inv * 2], np.float32))


def test_topk_tie_rule(oracle):
    """Equal logits: the lower expert id wins (qwen3_moe.c:184-194), i.e. a stable sort."""
    from cachepotato_amd.synth import MoESpec
    spec = MoESpec(D=64, E=16, K=4, F=64, enc=8)
    wg = np.zeros((16, 64), np.float32)
    wg[[3, 9, 12], :] = 0.05        # three tied winners
    wg[[1, 14], :] = 0.02           # two tied runners-up
    experts = [oracle.encode(8, np.zeros(64 * 64, np.float32))] * 48
    r = oracle.moe(spec, wg, np.ones(64, np.float32), experts, np.ones((1, 64), np.float32))
    assert r["topk"][0].tolist() == [3, 9, 12, 1]
    assert np.isclose(r["wt"][0].sum(), 1.0)


# ------------------------------------------------------------------ encoders

def test_encoders_vs_reference_vectors(oracle):
    z = golden("encoder_vectors.npz")
    x = z["x"].ravel()
    assert np.array_equal(oracle.encode(4, x), z["q4"])
    assert np.array_equal(oracle.encode(8, x), z["q8"])


def test_f64_to_f16_vs_numpy(oracle):
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.normal(0, 1, 20000) * 2.0 ** rng.integers(-30, 20, 20000),
                        [65504.0, 65520.0, 65519.99, 2 ** -24, 2 ** -25, 2 ** -25 * 1.0001,
                         2 ** -14, 2 ** -14 * (1 - 2 ** -11), 0.0, -0.0, 1e300, -1e-300]])
    with np.errstate(over="ignore"):
        want = v.astype(np.float16).view(np.uint16)
    got = np.array([oracle.L.or_f64_to_f16(float(a)) for a in v], np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ the MoE half

SMALL_FIXTURES = ["moe_small_q4_t1.npz", "moe_small_q4_t8.npz", "moe_small_q8_t1.npz",
                  "moe_small_q8_t8.npz"]


@pytest.mark.parametrize("fx", SMALL_FIXTURES)
def test_moe_small_vs_golden(oracle, fx):
    from cachepotato_amd import synth
    from tests.golden.make_golden import sha, spec_of
    z = golden(fx)
    name = fx[len("moe_"):-len("_t1.npz")]
    spec = spec_of(name)
    wg, ln2, ex = synth.wgate(spec), synth.ln2(spec), synth.experts_v4(spec)
    X = synth.inputs(spec, 0, 8)
    assert sha(wg) == str(z["sha_wgate"]) and sha(*ex) == str(z["sha_experts"])
    r = oracle.moe(spec, wg, ln2, ex, X[z["calls"][0]], threads=int(z["threads"]))
    assert np.array_equal(r["topk"], z["full_topk"])
    assert np.array_equal(bits(r["router"]), bits(z["full_router"]))
    assert np.array_equal(bits(r["mlp"]), bits(z["full_mlp"]))


@pytest.fixture(scope="module")
def q4_full():
    from cachepotato_amd import synth
    spec = synth.CONFIGS["q4_b1"]
    return spec, synth.wgate(spec), synth.ln2(spec), synth.experts_v4(spec)


@pytest.mark.parametrize("threads", [1, 8])
def test_moe_q4_b1_vs_golden(oracle, q4_full, threads):
    """Full-size decode batch 1, Q4_0: the first 8 vectors bit-exact against the fixture the
    reference engine wrote at CP_THREADS=1 / 8, and routing of the first 64 vectors."""
    from cachepotato_amd import synth
    from tests.golden.make_golden import sha
    spec, wg, ln2, ex = q4_full
    z = golden(f"moe_q4_b1_t{threads}.npz")
    assert sha(wg) == str(z["sha_wgate"]) and sha(*ex) == str(z["sha_experts"])
    X = synth.inputs(spec, 0, 64)
    for v in range(8):
        r = oracle.moe(spec, wg, ln2, ex, X[v:v + 1], threads=threads)
        assert np.array_equal(r["topk"][0], z["full_topk"][v])
        assert np.array_equal(bits(r["router"][0]), bits(z["full_router"][v]))
        assert np.array_equal(bits(r["mlp"][0]), bits(z["full_mlp"][v]))
    r = oracle.moe(spec, wg, ln2, ex, X[8:64], threads=threads)
    assert np.array_equal(r["topk"], z["topk"][8:64])


# ------------------------------------------------------------------ attention half

@pytest.mark.parametrize("enc", [0, 8, 4])
def test_attn_vs_reference(oracle, ref, enc):
    """or_attn restates qwen3_moe.c:110-167: bit-identical to the reference's qwen3_layer_kv
    (its o->attn and the cache rows it writes) for a prefill of 5 tokens, then 1 and 3 more
    tokens attending to the cache (pos0 = 5, 6)."""
    from tests.attn_helpers import attn_layer, inputs
    a = attn_layer(enc=enc)
    cap, kvw = 16, a["KV"] * a["HD"]
    kc_o, vc_o = np.zeros((cap, kvw), np.float32), np.zeros((cap, kvw), np.float32)
    kc_r, vc_r = np.zeros((cap, kvw), np.float32), np.zeros((cap, kvw), np.float32)
    X = inputs(a["D"], 0, 9)
    for pos0, T in ((0, 5), (5, 1), (6, 3)):
        got = oracle.attn(a, X[pos0:pos0 + T], pos0, kc_o, vc_o, threads=ref.threads)
        want = ref.attn(a, X[pos0:pos0 + T], pos0, kc_r, vc_r)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (enc, pos0)
        assert np.array_equal(kc_o.view(np.uint32), kc_r.view(np.uint32))
        assert np.array_equal(vc_o.view(np.uint32), vc_r.view(np.uint32))
        assert np.abs(got).max() > 0


def test_rope_closed_forms(oracle):
    """Position 0 rotates by angle 0 (identity, exactly); every rotation keeps the norm of
    each (i, i + hd/2) pair to float rounding; a pair's angle grows linearly in position."""
    rng = np.random.default_rng(5)
    hd = 64
    q = rng.standard_normal((3, 2 * hd)).astype(np.float32)
    k = rng.standard_normal((3, hd)).astype(np.float32)
    q0, k0 = q.copy(), k.copy()
    oracle.rope(q[:1], k[:1], 0, hd, 1e6)
    assert np.array_equal(q[0], q0[0]) and np.array_equal(k[0], k0[0])
    oracle.rope(q, k, 7, hd, 1e6)
    half = hd // 2
    for v, v0 in ((q.reshape(-1, hd), q0.reshape(-1, hd)), (k, k0)):
        n = np.hypot(v[:, :half], v[:, half:])
        n0 = np.hypot(v0[:, :half], v0[:, half:])
        assert np.allclose(n, n0, rtol=1e-5)
    # pair 0 rotates by exactly pos (inv_freq = theta^0 = 1): angle of token t is 7 + t
    ang = np.arctan2(k[:, half], k[:, 0]) - np.arctan2(k0[:, half], k0[:, 0])
    assert np.allclose(np.mod(ang - (7 + np.arange(3)) + np.pi, 2 * np.pi) - np.pi, 0, atol=1e-5)
