"""ctypes mirror of the block / port interface (include/qwen3_moe.h, field for field the
reference's engine/blocks/qwen3_moe.h), of the CPW1 v4 helpers (include/cpw4.h) and of the
public API (include/cachepotato.h, the reference's engine/api/cachepotato.h).

The structures have the reference's layout, so `bind(lib)` works on libcachepotato_amd.so
and on the reference engine compiled from its own sources alike: a test can drive both
through the same calls."""
import ctypes

import numpy as np

_c = ctypes
_vp, _i, _f, _sz, _u32, _u64 = _c.c_void_p, _c.c_int, _c.c_float, _c.c_size_t, _c.c_uint32, _c.c_uint64

ENC_F32, ENC_Q8, ENC_Q4 = 0, 8, 4


class QW3T(_c.Structure):
    _fields_ = [("p", _vp), ("enc", _i)]


class QW3Layer(_c.Structure):
    _fields_ = [("d_model", _i), ("n_heads", _i), ("n_kv", _i), ("head_dim", _i), ("d_exp", _i),
                ("n_experts", _i), ("topk", _i), ("vocab", _i), ("n_layers", _i),
                ("rope_theta", _f), ("rms_eps", _f),
                ("ln1", _vp), ("ln2", _vp), ("q_norm", _vp), ("k_norm", _vp),
                ("Wq", QW3T), ("Wk", QW3T), ("Wv", QW3T), ("Wo", QW3T), ("Wgate", QW3T),
                ("exp", _c.POINTER(QW3T)), ("exp_owned", _i), ("map", _vp), ("map_len", _sz),
                ("embed", QW3T), ("lm_head", QW3T), ("final_norm", _vp),
                ("off_tens", _u64), ("off_data", _u64), ("n_tens", _u32), ("n_enc", _u32),
                ("enc_code", _i * 64), ("cur_layer", _i), ("pager", _i), ("n_regions", _i),
                ("tensor_reg", _c.POINTER(_i)), ("reg_exp", _c.POINTER(_i)),
                ("reg_ln1", _i), ("reg_ln2", _i), ("reg_qnorm", _i), ("reg_knorm", _i),
                ("reg_Wq", _i), ("reg_Wk", _i), ("reg_Wv", _i), ("reg_Wo", _i), ("reg_Wgate", _i),
                ("reg_embed", _i), ("reg_lm_head", _i), ("reg_final_norm", _i),
                ("embed_chunks", _i), ("embed_rows", _i), ("reg_embed_chunk", _c.POINTER(_i)),
                ("embed_chunk_ptr", _c.POINTER(_vp))]


class QW3Out(_c.Structure):
    _fields_ = [("attn", _c.POINTER(_f)), ("mlp", _c.POINTER(_f)), ("router", _c.POINTER(_f)),
                ("topk_idx", _c.POINTER(_i))]


class QW3KV(_c.Structure):
    _fields_ = [("k", _vp), ("v", _vp), ("cap", _i)]


class SynthCfg(_c.Structure):
    """qw3_synth_cfg of include/cpw4.h"""
    _fields_ = [("n_layers", _i), ("d_model", _i), ("n_heads", _i), ("n_kv", _i),
                ("head_dim", _i), ("n_experts", _i), ("topk", _i), ("d_exp", _i), ("vocab", _i),
                ("rope_theta", _f), ("enc_attn", _i), ("enc_exp", _i), ("enc_embed", _i),
                ("enc_head", _i), ("norm_sigma", _c.c_double), ("seed", _u64),
                ("embed_sigma", _c.c_double), ("out_sigma", _c.c_double)]


BLOCK_API = [
    ("qwen3_layer_alloc", _i, [_c.POINTER(QW3Out), _c.POINTER(QW3Layer), _i]),
    ("qwen3_layer_free", None, [_c.POINTER(QW3Out)]),
    ("qwen3_layer_free_weights", None, [_c.POINTER(QW3Layer)]),
    ("qwen3_layer", _i, [_c.POINTER(QW3Layer), _vp, _i, _c.POINTER(QW3Out)]),
    ("qwen3_layer_kv", _i, [_c.POINTER(QW3Layer), _vp, _i, _i, _c.POINTER(QW3KV),
                            _c.POINTER(QW3Out)]),
    ("qwen3_kv_alloc", _i, [_c.POINTER(QW3KV), _c.POINTER(QW3Layer), _i]),
    ("qwen3_kv_free", None, [_c.POINTER(QW3KV)]),
    ("qwen3_mm", None, [_c.POINTER(QW3T), _vp, _vp, _i, _i]),
    ("qwen3_load_blob", _i, [_c.POINTER(QW3Layer), _c.c_char_p, _c.POINTER(_vp)]),
    ("qwen3_map", _i, [_c.POINTER(QW3Layer), _c.c_char_p]),
    ("qwen3_map_ex", _i, [_c.POINTER(QW3Layer), _c.c_char_p, _c.c_long]),
    ("qwen3_bind_layer", _i, [_c.POINTER(QW3Layer), _i]),
    ("qwen3_load_v4", _i, [_c.POINTER(QW3Layer), _c.c_char_p, _i]),
]

V4_API = [
    ("qwen3_write_synthetic", _i, [_c.c_char_p, _c.POINTER(SynthCfg), _c.c_char_p, _sz]),
    ("cpw4_check_file", _i, [_c.c_char_p, _c.c_char_p, _sz]),
    ("cpw4_crc32", _u32, [_u32, _vp, _sz]),
]


def bind(lib, extra=True):
    """Set restype/argtypes of the block API on a loaded library (ours or the reference's)."""
    for name, res, args in BLOCK_API + (V4_API if extra else []):
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


# The random-init Qwen3-30B-A3B-shaped model: 48 layers, hidden 2048, 32 query / 4 key-value
# heads of 128, QK-RMSNorm, RoPE theta 1e6, 128 experts top-8 of intermediate 768, vocabulary
# 151936; Q4_0 experts and attention, Q8_0 embedding and head; norm gains 1 + N(0, 0.1^2).
# The embedding rows are N(0, 1) and the two projections that write into the residual stream
# (Wo and the experts' Wd) N(0, (0.02 / sqrt(2 * 48))^2), every other matrix N(0, 0.02^2):
# with all matrices at 0.02 the hidden states of every position drift to one shared direction
# over the 48 layers and greedy decoding repeats a single token (cpw4.h, qw3_synth_cfg).
QWEN3_30B_A3B = dict(n_layers=48, d_model=2048, n_heads=32, n_kv=4, head_dim=128,
                     n_experts=128, topk=8, d_exp=768, vocab=151936, rope_theta=1e6,
                     enc_attn=ENC_Q4, enc_exp=ENC_Q4, enc_embed=ENC_Q8, enc_head=ENC_Q8,
                     norm_sigma=0.1, embed_sigma=1.0, out_sigma=0.02 / 96 ** 0.5,
                     seed=20261017)       # synth.SEED, the seed of every synthetic workload


def memfd_model(lib, cfg, name="qwen3_synthetic"):
    """A synthetic model file written into memory (memfd): returns (fd, "/proc/self/fd/N").
    The caller closes fd; a child process given fd reads the same path."""
    import os
    fd = os.memfd_create(name)
    path = f"/proc/self/fd/{fd}"
    try:
        write_synthetic(lib, path, **cfg)
    except BaseException:
        os.close(fd)
        raise
    return fd, path


def write_synthetic(lib, path, **kw):
    cfg = SynthCfg(**kw)
    err = _c.create_string_buffer(256)
    rc = lib.qwen3_write_synthetic(str(path).encode(), _c.byref(cfg), err, 256)
    if rc:
        raise RuntimeError(f"qwen3_write_synthetic: {rc}: {err.value.decode()}")
    return cfg


def check_file(lib, path):
    err = _c.create_string_buffer(256)
    rc = lib.cpw4_check_file(str(path).encode(), err, 256)
    return rc, err.value.decode()


def out_arrays(o, T, D, E, K):
    """numpy copies of a QW3Out's buffers"""
    g = lambda p, n: np.ctypeslib.as_array(p, shape=(n,)).copy()
    return dict(attn=g(o.attn, T * D).reshape(T, D), mlp=g(o.mlp, T * D).reshape(T, D),
                router=g(o.router, T * E).reshape(T, E), topk=g(o.topk_idx, T * K).reshape(T, K))


# ---------------------------------------------------------------- the public API (cachepotato.h)

class CpOptions(_c.Structure):
    _fields_ = [("budget_mb", _c.c_long), ("threads", _i), ("pin_cores", _i), ("max_ctx", _i),
                ("tokenizer_dir", _c.c_char_p)]


class CpTurn(_c.Structure):
    _fields_ = [("prompt_tokens", _i), ("context_tokens", _i), ("generated_tokens", _i),
                ("context_reset", _i), ("prefill_s", _c.c_double), ("decode_s", _c.c_double),
                ("stop", _i)]


CpTokenFn = _c.CFUNCTYPE(_i, _c.c_void_p, _sz, _c.c_void_p)


class CpStats(_c.Structure):
    _fields_ = [("n_layers", _i), ("d_model", _i), ("n_experts", _i), ("topk", _i),
                ("vocab", _i), ("max_ctx", _i), ("threads", _i), ("budget_mb", _c.c_long),
                ("file_bytes", _c.c_longlong), ("hits", _c.c_long), ("misses", _c.c_long),
                ("evictions", _c.c_long), ("bytes_fetched", _c.c_longlong),
                ("resident_bytes", _c.c_longlong)]


CP_API = [
    ("cp_options_default", None, [_c.POINTER(CpOptions)]),
    ("cp_open", _vp, [_c.c_char_p, _c.POINTER(CpOptions), _c.c_char_p, _sz]),
    ("cp_close", None, [_vp]),
    ("cp_chat", _i, [_vp, _c.c_char_p, _i, CpTokenFn, _vp, _c.POINTER(CpTurn)]),
    ("cp_reset", None, [_vp]),
    ("cp_get_stats", None, [_vp, _c.POINTER(CpStats)]),
    ("cp_physical_cores", _i, []),
    ("cp_mem_available_mb", _c.c_long, []),
    ("cp_auto_budget_mb", _c.c_long, [_c.c_longlong]),
    ("cp_eval_decode", _i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _c.POINTER(CpTurn)]),
    ("cp_last_logits", _i, [_vp, _vp]),
]


def bind_cp(lib):
    for name, res, args in CP_API:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def chat_turn(lib, h, msg, max_new, stop_after=0):
    """One cp_chat call through `lib` (this library or another with the same API): returns
    (rc, the bytes handed to the callback, one entry per token, CpTurn)."""
    got = []

    def on_token(p, n, user):
        got.append(_c.string_at(p, n) if n else b"")
        return 1 if 0 < stop_after <= len(got) else 0

    fn = CpTokenFn(on_token)
    turn = CpTurn()
    rc = lib.cp_chat(h, msg.encode() if isinstance(msg, str) else msg, max_new, fn, None,
                     _c.byref(turn))
    return rc, got, turn


class Model:
    """A model opened through cp_open (one at a time per process)."""

    def __init__(self, lib, path, max_ctx=0, tokenizer_dir=None):
        self.lib = bind_cp(lib)
        opt = CpOptions()
        lib.cp_options_default(_c.byref(opt))
        opt.max_ctx = max_ctx
        opt.tokenizer_dir = None if tokenizer_dir is None else str(tokenizer_dir).encode()
        err = _c.create_string_buffer(512)
        self.h = lib.cp_open(str(path).encode(), _c.byref(opt), err, 512)
        if not self.h:
            raise RuntimeError("cp_open: " + err.value.decode())
        self.stats = CpStats()
        lib.cp_get_stats(self.h, _c.byref(self.stats))

    def eval_decode(self, ids, gen, route=False):
        """cp_eval_decode: dict(tokens, step_ms, prefill_s, decode_s[, route (L, gen, K)])."""
        st = self.stats
        ids = np.ascontiguousarray(ids, np.int32)
        toks = np.zeros(gen, np.int32)
        steps = np.zeros(gen, np.float32)
        rt = np.zeros((st.n_layers, gen, st.topk), np.int32) if route else None
        turn = CpTurn()
        rc = self.lib.cp_eval_decode(self.h, ids.ctypes.data, ids.size, gen, toks.ctypes.data,
                                     None if rt is None else rt.ctypes.data, steps.ctypes.data,
                                     _c.byref(turn))
        if rc:
            raise RuntimeError(f"cp_eval_decode returned {rc}")
        out = dict(tokens=toks, step_ms=steps, prefill_s=turn.prefill_s, decode_s=turn.decode_s,
                   turn=turn)
        if route:
            out["route"] = rt
        return out

    def chat(self, msg, max_new, stop_after=0):
        """cp_chat: (rc, [token bytes], CpTurn); the callback asks to stop after `stop_after`
        tokens when that is > 0."""
        return chat_turn(self.lib, self.h, msg, max_new, stop_after)

    def last_logits(self):
        out = np.zeros(self.stats.vocab, np.float32)
        if self.lib.cp_last_logits(self.h, out.ctypes.data):
            raise RuntimeError("cp_last_logits failed")
        return out

    def close(self):
        if self.h:
            self.lib.cp_close(self.h)
            self.h = None
