"""GPU parity of the attention half (cpg_attn_forward) and the row-tiled GEMV, through the C
ABI, against the oracle's restatement of qwen3_moe.c:110-167 (itself bit-identical to the
reference engine, tests/test_oracle.py::test_attn_vs_reference).

Bars: the RoPE table bit-identical to the reference's powf/cosf/sinf; attention output and
cache rows within ATTN_TOL normwise relative error (max|gpu - ref| / max|ref|) of the oracle
at both Q4 numerics of the reference (the projections accumulate in another order)."""
import numpy as np
import pytest

from tests.gpu_helpers import rel_err

pytestmark = pytest.mark.gpu

ATTN_TOL = 1e-4
# prefill (MFMA projections and attention core): measured at most 1.5e-6; an activation
# split whose lo half misses its hi half (an f16 unit lost) shows as ~3e-5
PREFILL_TOL = 1e-5


def say(*a):
    print(*a, flush=True)


def test_rope_table_matches_reference_formula(cpg, oracle):
    """cpg_rope_table equals the oracle's RoPE (which calls the same libm functions as the
    reference) applied to unit vectors: cos and sin of every (position, pair) bit for bit."""
    import cachepotato_amd as C
    HD, P = 128, 40
    tab = np.empty(P * HD, np.float32)
    C.check(C.lib().cpg_rope_table(np.float32(1e6), HD, P, tab.ctypes.data), "rope")
    tab = tab.reshape(P, HD // 2, 2)
    # rotate e_i (a=1, b=0): v[i] = 1*c - 0*s = c, v[i+half] = 0*c + 1*s = s
    q = np.zeros((P, HD), np.float32)
    q[:, :HD // 2] = 1.0
    k = q.copy()
    for p in range(P):
        oracle.rope(q[p:p + 1], k[p:p + 1], p, HD, 1e6)
    assert np.array_equal(q[:, :HD // 2].view(np.uint32), tab[:, :, 0].view(np.uint32))
    assert np.array_equal(q[:, HD // 2:].view(np.uint32), tab[:, :, 1].view(np.uint32))


@pytest.mark.parametrize("enc,geom", [(4, "small"), (8, "small"), (4, "qwen3")])
def test_attn_vs_oracle(cpg, oracle, enc, geom):
    from tests.attn_helpers import attn_layer, inputs, DeviceAttn
    kw = dict(D=2048, H=32, KV=4, HD=128) if geom == "qwen3" else {}
    a = attn_layer(enc=enc, **kw)
    dev = DeviceAttn(a, cap=64)
    cap, kvw = 64, a["KV"] * a["HD"]
    X = inputs(a["D"], 100, 12)
    caches = {th: (np.zeros((cap, kvw), np.float32), np.zeros((cap, kvw), np.float32))
              for th in (1, 8)}
    try:
        for pos0, T in ((0, 7), (7, 1), (8, 4)):
            got = dev.forward(X[pos0:pos0 + T], pos0)
            kc, vc = dev.cache()
            for th, (kc_o, vc_o) in caches.items():
                want = oracle.attn(a, X[pos0:pos0 + T], pos0, kc_o, vc_o, threads=th)
                e = rel_err(got, want)
                ek = rel_err(kc[:pos0 + T], kc_o[:pos0 + T])
                ev = rel_err(vc[:pos0 + T], vc_o[:pos0 + T])
                say(f"attn {geom} enc={enc} pos0={pos0} T={T} threads={th}: out {e:.2e} "
                    f"k {ek:.2e} v {ev:.2e}")
                assert e <= ATTN_TOL and ek <= ATTN_TOL and ev <= ATTN_TOL
    finally:
        dev.close()


@pytest.mark.parametrize("enc,geom", [(4, "small"), (8, "small"), (4, "qwen3"), (8, "qwen3")])
def test_attn_prefill_dense_vs_oracle(cpg, oracle, enc, geom):
    """Prefill calls of 32 tokens and more, whose q|k|v and output projections run as MFMA
    GEMMs with the k range split into parts: ragged token counts (70 = one full tile of 64 and
    6 more, 33, 40) between single-token calls, against the oracle with its cache."""
    from tests.attn_helpers import attn_layer, inputs, DeviceAttn
    kw = dict(D=2048, H=32, KV=4, HD=128) if geom == "qwen3" else {}
    a = attn_layer(enc=enc, **kw)
    cap, kvw = 160, a["KV"] * a["HD"]
    dev = DeviceAttn(a, cap=cap, max_T=80)
    X = inputs(a["D"], 100, 144)
    kc_o, vc_o = np.zeros((cap, kvw), np.float32), np.zeros((cap, kvw), np.float32)
    try:
        for pos0, T in ((0, 70), (70, 1), (71, 33), (104, 40)):
            got = dev.forward(X[pos0:pos0 + T], pos0)
            kc, vc = dev.cache()
            want = oracle.attn(a, X[pos0:pos0 + T], pos0, kc_o, vc_o, threads=8)
            e = rel_err(got, want)
            ek = rel_err(kc[:pos0 + T], kc_o[:pos0 + T])
            ev = rel_err(vc[:pos0 + T], vc_o[:pos0 + T])
            say(f"attn prefill {geom} enc={enc} pos0={pos0} T={T}: out {e:.2e} k {ek:.2e} "
                f"v {ev:.2e}")
            assert e <= PREFILL_TOL and ek <= PREFILL_TOL and ev <= PREFILL_TOL
    finally:
        dev.close()


@pytest.mark.parametrize("enc", [4, 8])
def test_attn_prefill_long_vs_oracle(cpg, oracle, enc):
    """Long prefill calls at the Qwen3 geometry (GQA 8 query heads per kv head, head dim 128,
    the MFMA attention core): 200 tokens from position 0, one token, then 150 tokens over a
    201-position history (ragged blocks of 8 tokens, key tiles of 64 cut by the causal mask),
    against the oracle with its cache."""
    from tests.attn_helpers import attn_layer, inputs, DeviceAttn
    a = attn_layer(enc=enc, D=2048, H=32, KV=4, HD=128)
    cap, kvw = 400, a["KV"] * a["HD"]
    dev = DeviceAttn(a, cap=cap, max_T=200)
    X = inputs(a["D"], 101, 351)
    kc_o, vc_o = np.zeros((cap, kvw), np.float32), np.zeros((cap, kvw), np.float32)
    try:
        for pos0, T in ((0, 200), (200, 1), (201, 150)):
            got = dev.forward(X[pos0:pos0 + T], pos0)
            kc, vc = dev.cache()
            want = oracle.attn(a, X[pos0:pos0 + T], pos0, kc_o, vc_o, threads=8)
            e = rel_err(got, want)
            ek = rel_err(kc[:pos0 + T], kc_o[:pos0 + T])
            ev = rel_err(vc[:pos0 + T], vc_o[:pos0 + T])
            erow = max(rel_err(got[t], want[t]) for t in range(T))
            say(f"attn long prefill enc={enc} pos0={pos0} T={T}: out {e:.2e} (worst token "
                f"{erow:.2e}) k {ek:.2e} v {ev:.2e}")
            assert max(e, erow, ek, ev) <= PREFILL_TOL
    finally:
        dev.close()


@pytest.mark.parametrize("H,KV", [(16, 4), (16, 1), (4, 4), (8, 4)])
def test_attn_prefill_gqa_groups_vs_oracle(cpg, oracle, H, KV):
    """The MFMA attention core at every query-head group it takes (G = H/KV = 4, 16, 1, 2;
    head dim 128): 90 tokens from position 0 (blocks of 64/G tokens, the last one ragged),
    then 40 tokens over a 90-position history, against the oracle with its cache."""
    from tests.attn_helpers import attn_layer, inputs, DeviceAttn
    a = attn_layer(enc=4, D=512, H=H, KV=KV, HD=128)
    cap, kvw = 160, a["KV"] * a["HD"]
    dev = DeviceAttn(a, cap=cap, max_T=90)
    X = inputs(a["D"], 102, 130)
    kc_o, vc_o = np.zeros((cap, kvw), np.float32), np.zeros((cap, kvw), np.float32)
    try:
        for pos0, T in ((0, 90), (90, 40)):
            got = dev.forward(X[pos0:pos0 + T], pos0)
            kc, vc = dev.cache()
            want = oracle.attn(a, X[pos0:pos0 + T], pos0, kc_o, vc_o, threads=8)
            e = rel_err(got, want)
            erow = max(rel_err(got[t], want[t]) for t in range(T))
            ek = rel_err(kc[:pos0 + T], kc_o[:pos0 + T])
            ev = rel_err(vc[:pos0 + T], vc_o[:pos0 + T])
            say(f"attn prefill G={H // KV} pos0={pos0} T={T}: out {e:.2e} (worst token "
                f"{erow:.2e}) k {ek:.2e} v {ev:.2e}")
            assert max(e, erow, ek, ev) <= PREFILL_TOL
    finally:
        dev.close()


def test_attn_device_position_equals_host_position(cpg):
    """cpg_attn_forward_at (position read on the device, as in a replayed graph) computes the
    same bits as cpg_attn_forward at the same positions, cache included; a position whose rows
    would fall outside the cache writes nothing to the cache, gives NaN instead of a stale
    output, and sets the workspace status (read and cleared by cpg_attn_ws_status), with
    either one-token kernel and for several tokens."""
    import cachepotato_amd as C
    from tests.attn_helpers import attn_layer, inputs, DeviceAttn
    a = attn_layer(enc=4, D=2048, H=32, KV=4, HD=128)
    cap = 48
    X = inputs(a["D"], 100, cap)
    host, dev = DeviceAttn(a, cap=cap), DeviceAttn(a, cap=cap)
    try:
        for pos0, T in ((0, 5), (5, 1), (6, 1), (7, 3), (10, 1)):
            g1 = host.forward(X[pos0:pos0 + T], pos0)
            g2 = dev.forward_at(X[pos0:pos0 + T], pos0)
            assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32)), (pos0, T)
        for c1, c2 in zip(host.cache(), dev.cache()):
            assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))
        assert C.lib().cpg_attn_ws_status(dev.ws) == 0
        before = dev.cache()
        for mode in (C.ATTN_SPLIT, C.ATTN_PER_HEAD):
            C.check(C.lib().cpg_attn_decode_mode(mode), "mode")
            # one past the last row: nothing written to the cache, NaN out, the status set
            out = dev.forward_at(X[:1], cap)
            for c1, c2 in zip(before, dev.cache()):
                assert np.array_equal(c1, c2)
            assert np.isnan(out).all(), mode
            assert C.lib().cpg_attn_ws_status(dev.ws) == 1, mode
            assert C.lib().cpg_attn_ws_status(dev.ws) == 0, mode      # read and cleared
        # several tokens from a device position whose last rows fall outside
        dev.forward_at(X[:3], cap - 2)
        assert C.lib().cpg_attn_ws_status(dev.ws) == 1
        g = dev.forward_at(X[10:11], 10)           # in range again: no status
        assert C.lib().cpg_attn_ws_status(dev.ws) == 0 and np.isfinite(g).all()
    finally:
        C.check(C.lib().cpg_attn_decode_mode(C.ATTN_SPLIT), "mode")
        host.close()
        dev.close()


@pytest.mark.parametrize("mode", ["split", "per_head"])
@pytest.mark.parametrize("pos", [1000, 1537, 2047])
def test_attn_decode_long_context_vs_oracle(cpg, oracle, pos, mode):
    """One decode step (the device-held position of the graph-replayed step) of the Qwen3
    geometry at positions 1000-2047 of a 2048-row cache, the cache's earlier rows seeded with
    N(0, 1) values, with either one-token kernel: the output and the new cache row against
    the oracle's attention half on the same cache (long score vectors, many value batches or
    splits, the per-head kernel's LDS score buffer at its largest)."""
    import cachepotato_amd as C
    from tests.attn_helpers import attn_layer, inputs, DeviceAttn
    C.check(C.lib().cpg_attn_decode_mode(C.ATTN_SPLIT if mode == "split" else C.ATTN_PER_HEAD),
            "mode")
    a = attn_layer(enc=4, D=2048, H=32, KV=4, HD=128)
    cap, kvw = 2048, a["KV"] * a["HD"]
    rng = np.random.default_rng(pos)
    kc0 = rng.standard_normal((cap, kvw), dtype=np.float32)
    vc0 = rng.standard_normal((cap, kvw), dtype=np.float32)
    kc0[pos:], vc0[pos:] = 0.0, 0.0
    x = inputs(a["D"], 500 + pos, 1)
    dev = DeviceAttn(a, cap=cap, max_T=1)
    try:
        dev.set_cache(kc0, vc0)
        got = dev.forward_at(x, pos)
        kc, vc = dev.cache()
    finally:
        dev.close()
        C.lib().cpg_attn_decode_mode(C.ATTN_SPLIT)       # the default
    kc_o, vc_o = kc0.copy(), vc0.copy()
    want = oracle.attn(a, x, pos, kc_o, vc_o, threads=1)
    e, ek, ev = rel_err(got, want), rel_err(kc[pos], kc_o[pos]), rel_err(vc[pos], vc_o[pos])
    say(f"decode attention at position {pos}: out {e:.2e}, new k row {ek:.2e}, v row {ev:.2e}")
    assert e <= ATTN_TOL and ek <= ATTN_TOL and ev <= ATTN_TOL
    assert np.array_equal(kc[:pos].view(np.uint32), kc0[:pos].view(np.uint32))


@pytest.mark.parametrize("P0,N,cap", [(20, 100, 128), (222, 262, 320)])
def test_attn_decode_splits_vs_oracle(cpg, oracle, P0, N, cap):
    """One token at a time from position P0 to N - 1 after a P0-token prefill: positions 20-99
    (one to four splits of 32 positions) and 222-261 (seven to nine splits), with the split
    kernel (CPG_ATTN_SPLIT; the position read from device memory on odd steps, as in the
    decode graph) and one workgroup per query head (CPG_ATTN_PER_HEAD): every step's output
    and the cache rows within ATTN_TOL of the oracle for both, and the two kernels within
    rounding of each other."""
    import cachepotato_amd as C
    from tests.attn_helpers import attn_layer, inputs, DeviceAttn
    a = attn_layer(enc=4, D=2048, H=32, KV=4, HD=128)
    kvw = a["KV"] * a["HD"]
    X = inputs(a["D"], 100 + P0, N)
    split, head = DeviceAttn(a, cap=cap, max_T=P0), DeviceAttn(a, cap=cap, max_T=P0)
    kc_o, vc_o = np.zeros((cap, kvw), np.float32), np.zeros((cap, kvw), np.float32)
    worst = 0.0
    L = C.lib()
    try:
        oracle.attn(a, X[:P0], 0, kc_o, vc_o, threads=1)
        for dev in (split, head):
            dev.forward(X[:P0], 0)
        for pos in range(P0, N):
            want = oracle.attn(a, X[pos:pos + 1], pos, kc_o, vc_o, threads=1)
            C.check(L.cpg_attn_decode_mode(C.ATTN_SPLIT), "mode")
            # the device-held position on odd steps (the decode graph's form)
            g1 = (split.forward_at if pos % 2 else split.forward)(X[pos:pos + 1], pos)
            C.check(L.cpg_attn_decode_mode(C.ATTN_PER_HEAD), "mode")
            g2 = head.forward(X[pos:pos + 1], pos)
            e1, e2, e12 = rel_err(g1, want), rel_err(g2, want), rel_err(g1, g2)
            worst = max(worst, e1, e2)
            assert e1 <= ATTN_TOL and e2 <= ATTN_TOL and e12 <= ATTN_TOL, (pos, e1, e2, e12)
        for dev in (split, head):
            kc, vc = dev.cache()
            assert rel_err(kc[:N], kc_o[:N]) <= ATTN_TOL and rel_err(vc[:N], vc_o[:N]) <= ATTN_TOL
        say(f"decode positions {P0}..{N - 1}: worst error against the oracle {worst:.2e}")
    finally:
        L.cpg_attn_decode_mode(C.ATTN_SPLIT)       # the default
        for dev in (split, head):
            dev.close()


@pytest.mark.parametrize("enc,n_in,n_out,T", [(4, 2048, 5120, 1), (4, 4096, 2048, 3),
                                              (8, 2048, 1024, 5), (4, 256, 192, 2),
                                              (4, 4096, 2048, 1), (8, 4096, 2048, 1),
                                              (4, 3072, 256, 1)])
def test_gemv_tiled(cpg, oracle, enc, n_in, n_out, T):
    """cpg_gemv on a row-tiled matrix against matmul_wx_q4 / matmul_wx_q8 on the v4 blocks
    (both numerics), within fp32 accumulation error."""
    import cachepotato_amd as C
    rng = np.random.default_rng(n_in + n_out + T)
    w = oracle.encode(enc, (rng.standard_normal(n_out * n_in) * 0.02).astype(np.float32))
    x = rng.standard_normal((T, n_in)).astype(np.float32)
    L = C.lib()
    wd = C.DeviceBuffer(L.cpg_matrix_bytes(enc, n_out, n_in))
    C.check(L.cpg_upload_matrix(enc, wd.ptr, w.ctypes.data, n_out, n_in), "upload")
    xd, od = C.to_device(x), C.DeviceBuffer(T * n_out * 4)
    C.check(L.cpg_gemv(enc, wd.ptr, n_in, n_out, xd.ptr, T, od.ptr), "cpg_gemv")
    C.sync()
    got = od.download(np.float32, T * n_out).reshape(T, n_out)
    for t in range(T):
        for th in (1, 8):
            want = oracle.matmul(enc, w, x[t], n_in, n_out, threads=th)
            assert rel_err(got[t], want) <= 1e-5
    for b in (wd, xd, od):
        b.close()


@pytest.mark.parametrize("enc,D,V", [(8, 2048, 151936), (4, 2048, 4096), (8, 1024, 640)])
def test_head_next(cpg, oracle, enc, D, V):
    """cpg_head_next (final RMSNorm, head GEMV, greedy argmax and the next token's embedding
    row in one launch): logits within fp32 accumulation error of the oracle's matmul of the v4
    blocks (both Q4 numerics) on the oracle's rmsnorm within a common scale factor; the token
    is the argmax of the logits it wrote, lowest index on ties (two identical top rows planted);
    x becomes that token's embedding row bit for bit (cpg_embed_rows); a second call (the
    counter left at zero by the first) gives the same."""
    import cachepotato_amd as C
    L = C.lib()
    rng = np.random.default_rng(D + V)
    wf = rng.standard_normal((V, D), dtype=np.float32) * np.float32(0.02)
    top = int(rng.integers(V // 2, V))           # plant a tie: rows lo and top identical and largest
    lo = int(rng.integers(0, V // 2))
    x = rng.standard_normal(D).astype(np.float32)
    g = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    xn = oracle.rmsnorm(x, g, 1e-6)
    wf[top] = 0.5 * np.sign(xn)                  # the largest dot product by far
    wf[lo] = wf[top]
    w = oracle.encode(enc, wf.ravel())
    emb = oracle.encode(8, rng.standard_normal(V * D, dtype=np.float32))
    wd = C.DeviceBuffer(L.cpg_matrix_bytes(enc, V, D))
    C.check(L.cpg_upload_matrix(enc, wd.ptr, w.ctypes.data, V, D), "upload")
    ed, gd = C.to_device(emb), C.to_device(g)
    xd, lg, tok = C.DeviceBuffer(D * 4), C.DeviceBuffer(V * 4), C.DeviceBuffer(4)
    sc = C.DeviceBuffer(L.cpg_head_scratch_bytes(V)).zero()
    row = C.DeviceBuffer(D * 4)
    try:
        for call in range(2):
            xd.upload(x)
            C.check(L.cpg_head_next(enc, wd.ptr, D, V, xd.ptr, gd.ptr, np.float32(1e-6), lg.ptr,
                                    tok.ptr, 8, ed.ptr, V, sc.ptr), "cpg_head_next")
            C.sync()
            logits = lg.download(np.float32, V)
            t = int(tok.download(np.int32, 1)[0])
            assert t == lo == int(np.argmax(logits)), (call, t, lo, top)
            for th in (1, 8):
                want = oracle.matmul(enc, w, xn, D, V, threads=th)
                e = rel_err(logits, want)
                assert e <= 1e-5, (th, e)
            C.check(L.cpg_embed_rows(8, ed.ptr, V, D, tok.ptr, 1, row.ptr), "embed")
            C.sync()
            assert np.array_equal(xd.download(np.float32, D).view(np.uint32),
                                  row.download(np.float32, D).view(np.uint32))
            say(f"head_next enc={enc} D={D} V={V} call {call}: token {t}, logits err {e:.2e}")
    finally:
        for b in (wd, ed, gd, xd, lg, tok, sc, row):
            b.close()
