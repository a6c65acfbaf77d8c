"""CPW1 v4 files (format/SPEC.md §3-§8): the synthetic writer's output is validated by our
parser and loaded by the reference engine's own loader (engine/blocks/qwen3_moe.c:296-459,
compiled from source in oracle/_ref) with the geometry it was written with; region digests
are CRC-32 over the covered bytes; payloads are the generator's values; malformed files are
refused with the reference's table-mismatch code (-3)."""
import ctypes
import os
import zlib

import numpy as np
import pytest

import cachepotato_amd as C
from cachepotato_amd import qwen3 as Q
from cachepotato_amd import synth

SMALL = dict(n_layers=2, d_model=256, n_heads=4, n_kv=2, head_dim=64, n_experts=16, topk=8,
             d_exp=128, vocab=512, rope_theta=1e6, enc_attn=Q.ENC_Q4, enc_exp=Q.ENC_Q4,
             enc_embed=Q.ENC_Q8, enc_head=Q.ENC_Q8, norm_sigma=0.1, seed=synth.SEED)


@pytest.fixture(scope="module")
def small_file(tmp_path_factory):
    p = tmp_path_factory.mktemp("v4") / "small.v4"
    Q.write_synthetic(Q.bind(C.lib()), p, **SMALL)
    return p


def _tables(path):
    """A plain-Python reading of the header and the tensor / region tables (SPEC §3, §5, §8)."""
    b = open(path, "rb").read()
    u = lambda o, n: int.from_bytes(b[o:o + n], "little")
    hdr = dict(n_t=u(16, 4), n_b=u(20, 4), n_r=u(24, 4), n_e=u(28, 4), off_t=u(40, 8),
               off_r=u(56, 8), off_d=u(64, 8))
    o = u(32, 8)
    kinds = []
    for _ in range(hdr["n_e"]):
        kinds.append(u(o + 4, 1))
        o += 4 + 1 + 1 + 2 + 2 + 3
        o += 2 + u(o, 2)
    hdr["enc_kind"] = kinds
    o = hdr["off_t"] + 4
    tens = []
    for _ in range(hdr["n_t"]):
        nl = u(o, 2); name = b[o + 2:o + 2 + nl].decode(); o += 2 + nl
        enc = u(o, 4); rank = u(o + 4, 1); o += 5
        dims = [u(o + 4 * d, 4) for d in range(rank)]; o += 4 * rank
        off, ln = u(o, 8), u(o + 8, 8); o += 8 + 8 + 4 + 2
        tens.append(dict(name=name, enc=enc, dims=dims, off=off, len=ln))
    o = hdr["off_r"] + 4
    regs = []
    for _ in range(hdr["n_r"]):
        regs.append(dict(off=u(o, 8), len=u(o + 8, 8), lo=u(o + 16, 4), hi=u(o + 20, 4),
                         kind=u(o + 24, 1), digest=u(o + 35, 8)))
        o += 43
    return b, hdr, tens, regs


def test_crc32_known_answer():
    """the standard vector the reference cites (engine/core/weights_v4.c:30-32)"""
    L = Q.bind(C.lib())
    s = b"123456789"
    assert L.cpw4_crc32(0, s, len(s)) == 0xCBF43926
    data = np.random.default_rng(1).integers(0, 256, 10000, dtype=np.uint8)
    assert L.cpw4_crc32(0, data.ctypes.data, data.size) == zlib.crc32(data.tobytes())


def test_synthetic_file_structure(small_file):
    L = Q.bind(C.lib())
    rc, msg = Q.check_file(L, small_file)
    assert rc == 0, msg
    b, hdr, tens, regs = _tables(small_file)
    n_e, Lr = SMALL["n_experts"], SMALL["n_layers"]
    assert hdr["n_t"] == 1 + Lr * (9 + 3 * n_e) + 2 and hdr["n_b"] == 1 + 2 * Lr
    assert hdr["n_r"] == Lr * n_e + (hdr["n_t"] - Lr * n_e * 3)
    # f32 tensors first, then the quantised ones, each 64-byte aligned, no overlap
    order = sorted(range(len(tens)), key=lambda i: tens[i]["off"])
    f32 = [i for i in order if hdr["enc_kind"][tens[i]["enc"]] == 0]
    assert order[:len(f32)] == f32 and len(f32) == 4 * Lr + Lr + 1
    assert all(t["off"] % 64 == 0 for t in tens)
    for a, c in zip(order, order[1:]):
        assert tens[a]["off"] + tens[a]["len"] <= tens[c]["off"]
    # every region digest is the CRC-32 of its tensors' bytes with their padding
    for r in regs:
        end = tens[r["hi"] - 1]["off"] + tens[r["hi"] - 1]["len"]
        end = (end + 63) // 64 * 64
        blob = b[hdr["off_d"] + r["off"]:hdr["off_d"] + end]
        assert zlib.crc32(blob) == r["digest"]
        assert r["len"] == tens[r["hi"] - 1]["off"] + tens[r["hi"] - 1]["len"] - r["off"]


def test_synthetic_payload_is_the_generator(small_file):
    b, hdr, tens, _ = _tables(small_file)
    byname = {t["name"]: t for t in tens}
    s = SMALL
    t = byname["expert.1.3.Wu"]
    want = C.gen_blocks(4, s["seed"], C.stream_id(1, C.K_WU, 3), s["d_exp"] * s["d_model"], 0.02)
    got = np.frombuffer(b, np.uint8, t["len"], hdr["off_d"] + t["off"])
    assert np.array_equal(got, want)
    t = byname["ln2.0"]
    g = C.gen_normal(s["seed"], C.stream_id(0, C.K_NORM, 2), s["d_model"], 0.1)
    got = np.frombuffer(b, np.float32, s["d_model"], hdr["off_d"] + t["off"])
    assert np.array_equal(got, (np.float32(1.0) + g).astype(np.float32))
    t = byname["Wgate.1"]
    g = C.gen_normal(s["seed"], C.stream_id(1, C.K_WGATE, 0), s["n_experts"] * s["d_model"], 0.02)
    assert np.array_equal(np.frombuffer(b, np.float32, g.size, hdr["off_d"] + t["off"]), g)


def test_reference_loader_binds_every_layer(small_file):
    """The reference's qwen3_load_v4 / qwen3_bind_layer accept the file and see the geometry
    and encodings it was written with."""
    from oracle.bindings import REF_SO
    if not os.path.exists(REF_SO):
        pytest.skip("reference engine not built here")
    R = Q.bind(ctypes.CDLL(REF_SO), extra=False)
    s = SMALL
    for layer in range(s["n_layers"]):
        m = Q.QW3Layer()
        assert R.qwen3_load_v4(ctypes.byref(m), str(small_file).encode(), layer) == 0
        assert (m.d_model, m.n_heads, m.n_kv, m.head_dim, m.d_exp, m.n_experts, m.topk,
                m.n_layers) == (s["d_model"], s["n_heads"], s["n_kv"], s["head_dim"],
                                s["d_exp"], s["n_experts"], s["topk"], s["n_layers"])
        assert m.Wq.enc == 4 and m.exp[0].enc == 4 and m.Wgate.enc == 0 and m.embed.enc == 8
        assert m.lm_head.p and m.final_norm and m.embed.p
        R.qwen3_layer_free_weights(ctypes.byref(m))


def _tensor_record(b, hdr, name):
    """Byte offsets of the dims, offset and length fields of tensor `name`'s record."""
    u = lambda o, n: int.from_bytes(b[o:o + n], "little")
    o = hdr["off_t"] + 4
    for _ in range(hdr["n_t"]):
        nl = u(o, 2)
        nm = bytes(b[o + 2:o + 2 + nl]).decode()
        o += 2 + nl + 4
        rank = b[o]
        dims = o + 1
        o += 1 + 4 * rank
        if nm == name:
            return dict(rank=rank, dims=dims, offset=o, length=o + 8)
        o += 8 + 8 + 4 + 2
    raise KeyError(name)


def _set_dims(b, rec, dims, length=None):
    for d, v in enumerate(dims):
        b[rec["dims"] + 4 * d:rec["dims"] + 4 * d + 4] = int(v).to_bytes(4, "little")
    if length is not None:
        b[rec["length"]:rec["length"] + 8] = int(length).to_bytes(8, "little")


def _moe_param(b, hdr, layer, index, value):
    """Set params[index] of layer `layer`'s MoE block (block table, SPEC §5)."""
    u = lambda o, n: int.from_bytes(b[o:o + n], "little")
    o = u(48, 8) + 4
    for _ in range(hdr["n_b"]):
        kind, lay, nr = b[o], u(o + 1, 4), b[o + 5]
        o += 6 + 4 * nr
        npar = b[o]
        if kind == 0x20 and lay == layer:
            q = o + 1 + 4 * index
            b[q:q + 4] = int(value).to_bytes(4, "little")
            return
        o += 1 + 4 * npar
    raise KeyError(layer)


# Shapes that pass the table checks (each record's length still matches its dims) but
# disagree with the model's geometry, and one whose size wraps 64 bits: each would size a copy
# from one tensor and apply it to another, or divide by zero, if the loader believed it.
GEOMETRY_CASES = {
    # Wgate.1 [16, 256] read as [32, 128]: 32 experts of the wrong width
    "router_rows": lambda b, h: _set_dims(b, _tensor_record(b, h, "Wgate.1"), [32, 128]),
    # head_dim 0: q_norm.0 empty
    "head_dim_zero": lambda b, h: _set_dims(b, _tensor_record(b, h, "q_norm.0"), [0], length=0),
    # Wq.0 [256, 256] read as [512, 128]
    "wq_width": lambda b, h: _set_dims(b, _tensor_record(b, h, "Wq.0"), [512, 128]),
    # an expert's down projection transposed: [128, 256] instead of [256, 128]
    "expert_transposed": lambda b, h: _set_dims(b, _tensor_record(b, h, "expert.1.2.Wd"),
                                                [128, 256]),
    # k_norm.1 half as long as head_dim (its length shortened to match)
    "k_norm_short": lambda b, h: _set_dims(b, _tensor_record(b, h, "k_norm.1"), [32], length=128),
    # top-k beyond the expert count
    "topk": lambda b, h: _moe_param(b, h, 1, 1, 17),
    # Wgate.0 f32 [2175126601, 2120192000]: 2^62 + 4096 elements, 2^64 + 16384 bytes, which
    # wraps to the record's 16384
    "size_wraps": lambda b, h: _set_dims(b, _tensor_record(b, h, "Wgate.0"),
                                         [268501 * 8101, 4096 * 125 * 41 * 101]),
}


@pytest.mark.parametrize("what", sorted(GEOMETRY_CASES))
def test_geometry_mismatch_is_refused(small_file, tmp_path, what):
    """The loader's geometry check (cpw4_qwen3_geometry) refuses a file whose tensors disagree
    with its own layer-0 geometry, before anything is allocated or copied."""
    L = Q.bind(C.lib())
    b, hdr, _, _ = _tables(small_file)
    b = bytearray(b)
    GEOMETRY_CASES[what](b, hdr)
    p = tmp_path / f"bad_{what}.v4"
    p.write_bytes(bytes(b))
    rc, msg = Q.check_file(L, p)
    assert rc == -3, (what, rc, msg)
    if what == "size_wraps":
        assert "overflows" in msg, msg


@pytest.mark.parametrize("what", ["magic", "truncated", "misaligned", "length", "reserved"])
def test_malformed_files_are_refused(small_file, tmp_path, what):
    L = Q.bind(C.lib())
    b, hdr, tens, _ = _tables(small_file)
    b = bytearray(b)
    if what == "magic":
        b[0] ^= 1
    elif what == "truncated":
        b = b[:len(b) - 100]
    elif what == "reserved":
        b[72] = 1
    else:
        # the first tensor record: string, enc, rank, dims, then offset and length
        o = hdr["off_t"] + 4
        nl = int.from_bytes(b[o:o + 2], "little")
        o += 2 + nl + 4
        rank = b[o]
        o += 1 + 4 * rank
        field = o if what == "misaligned" else o + 8
        v = int.from_bytes(b[field:field + 8], "little") + (4 if what == "misaligned" else 2)
        b[field:field + 8] = v.to_bytes(8, "little")
    p = tmp_path / "bad.v4"
    p.write_bytes(bytes(b))
    rc, msg = Q.check_file(L, p)
    assert rc == -3, (what, rc, msg)
