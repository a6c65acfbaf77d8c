"""ctypes access to the checker libraries — TEST INFRASTRUCTURE ONLY.

  liboracle.so      the CPU restatement of the reference arithmetic (oracle.c)
  _ref/libref.so    the reference engine compiled from its own sources + ref_harness.c

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module; the
product library never does. `make -C oracle` builds both (libref only where the reference
tree exists; the built file travels with the repository snapshot to the GPU box).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")

_c = ctypes
_vp, _i, _f, _sz = _c.c_void_p, _c.c_int, _c.c_float, _c.c_size_t


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _p(a):
    return None if a is None else a.ctypes.data


def _ptr_array(arrs):
    return (_vp * len(arrs))(*[a.ctypes.data for a in arrs])


class Oracle:
    """The C restatement (oracle.c)."""

    def __init__(self):
        if not os.path.exists(ORACLE_SO):
            build()
        L = ctypes.CDLL(ORACLE_SO)
        L.or_f16_to_f32.restype = _f
        L.or_f16_to_f32.argtypes = [_c.c_uint16]
        for n in ("or_q8_dequant_row", "or_q4_dequant_row"):
            getattr(L, n).argtypes = [_vp, _vp, _i]
        L.or_matmul_wx.argtypes = [_vp, _vp, _vp, _i, _i]
        L.or_matmul_wx_q8.argtypes = [_vp, _vp, _vp, _i, _i]
        L.or_matmul_wx_q4.argtypes = [_vp, _vp, _vp, _i, _i, _i]
        L.or_rmsnorm.argtypes = [_vp, _vp, _vp, _i, _f]
        L.or_expf.restype = _f
        L.or_expf.argtypes = [_f]
        L.or_softmax.argtypes = [_vp, _i]
        L.or_silu.restype = _f
        L.or_silu.argtypes = [_f]
        L.or_moe.argtypes = [_i, _i, _i, _i, _f, _vp, _vp, _vp, _i, _i, _vp, _vp, _i,
                             _vp, _vp, _vp, _vp, _vp]
        L.or_attn.argtypes = [_i, _i, _i, _i, _f, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i,
                              _vp, _i, _i, _vp, _vp, _vp]
        L.or_rope.argtypes = [_vp, _vp, _i, _i, _i, _i, _i, _f]
        L.or_encode_q4_0.argtypes = [_vp, _sz, _vp]
        L.or_encode_q8_0.argtypes = [_vp, _sz, _vp]
        L.or_exp2f_tab.restype = _c.c_uint64
        L.or_exp2f_tab.argtypes = [_i]
        L.or_f64_to_f16.restype = _c.c_uint16
        L.or_f64_to_f16.argtypes = [_c.c_double]
        self.L = L

    def dequant_row(self, enc, blocks, n):
        out = np.empty(n, dtype=np.float32)
        fn = self.L.or_q4_dequant_row if enc == 4 else self.L.or_q8_dequant_row
        fn(np.ascontiguousarray(blocks).ctypes.data, out.ctypes.data, n)
        return out

    def matmul(self, enc, w, x, n_in, n_out, threads=1):
        out = np.empty(n_out, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w)
        if enc == 4:
            self.L.or_matmul_wx_q4(out.ctypes.data, x.ctypes.data, w.ctypes.data, n_in, n_out, threads)
        elif enc == 8:
            self.L.or_matmul_wx_q8(out.ctypes.data, x.ctypes.data, w.ctypes.data, n_in, n_out)
        else:
            self.L.or_matmul_wx(out.ctypes.data, x.ctypes.data, w.ctypes.data, n_in, n_out)
        return out

    def rmsnorm(self, x, g, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        self.L.or_rmsnorm(out.ctypes.data, x.ctypes.data, np.ascontiguousarray(g, dtype=np.float32).ctypes.data, x.size, eps)
        return out

    def softmax(self, x):
        y = np.array(x, dtype=np.float32, copy=True)
        self.L.or_softmax(y.ctypes.data, y.size)
        return y

    def moe(self, spec, wgate, ln2, experts, x, threads=1, attn=None):
        """or_moe: returns dict(xn, router, topk, wt, mlp) for x (T, D)."""
        T = x.shape[0]
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = dict(xn=np.empty((T, spec.D), np.float32), router=np.empty((T, spec.E), np.float32),
                   topk=np.empty((T, spec.K), np.int32), wt=np.empty((T, spec.K), np.float32),
                   mlp=np.zeros((T, spec.D), np.float32))
        ptrs = _ptr_array(experts)
        self.L.or_moe(spec.D, spec.E, spec.K, spec.F, spec.eps, ln2.ctypes.data,
                      np.ascontiguousarray(wgate).ctypes.data, ptrs, spec.enc, threads,
                      x.ctypes.data, _p(attn), T, out["xn"].ctypes.data,
                      out["router"].ctypes.data, out["topk"].ctypes.data,
                      out["wt"].ctypes.data, out["mlp"].ctypes.data)
        return out

    def attn(self, a, x, pos0, kc, vc, threads=1):
        """or_attn for the layer dict `a` (see tests/attn_helpers.py); kc/vc are updated."""
        T = x.shape[0]
        out = np.empty((T, a["D"]), np.float32)
        x = np.ascontiguousarray(x, np.float32)
        self.L.or_attn(a["D"], a["H"], a["KV"], a["HD"], a["theta"], a["eps"],
                       a["ln1"].ctypes.data, a["qn"].ctypes.data, a["kn"].ctypes.data,
                       a["wq"].ctypes.data, a["wk"].ctypes.data, a["wv"].ctypes.data,
                       a["wo"].ctypes.data, a["enc"], threads, x.ctypes.data, T, pos0,
                       kc.ctypes.data, vc.ctypes.data, out.ctypes.data)
        return out

    def rope(self, q, k, pos0, hd, theta):
        T = q.shape[0]
        self.L.or_rope(q.ctypes.data, k.ctypes.data, T, pos0, q.shape[1] // hd,
                       k.shape[1] // hd, hd, theta)

    def encode(self, enc, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.size // 32 * (18 if enc == 4 else 34), dtype=np.uint8)
        (self.L.or_encode_q4_0 if enc == 4 else self.L.or_encode_q8_0)(x.ctypes.data, x.size, out.ctypes.data)
        return out


class Reference:
    """The reference engine compiled from its own sources (oracle/_ref/libref.so)."""

    def __init__(self, threads=None, pin=False):
        if not os.path.exists(REF_SO):
            raise FileNotFoundError(f"{REF_SO} absent (built by `make -C oracle` where the "
                                    "reference tree exists)")
        L = ctypes.CDLL(REF_SO)
        L.ref_threads_init.restype = _i
        L.ref_threads_init.argtypes = [_i]
        L.ref_moe_layer.restype = _i
        L.ref_moe_layer.argtypes = [_i, _i, _i, _i, _f, _vp, _vp, _vp, _i, _vp, _i, _vp, _vp, _vp]
        L.q8_dequant_row.argtypes = [_vp, _vp, _i]
        L.q4_dequant_row.argtypes = [_vp, _vp, _i]
        L.matmul_wx_q4.argtypes = [_vp, _vp, _vp, _i, _i]
        L.matmul_wx_q8.argtypes = [_vp, _vp, _vp, _i, _i]
        L.matmul_wx.argtypes = [_vp, _vp, _vp, _i, _i]
        L.rmsnorm.argtypes = [_vp, _vp, _vp, _i, _f]
        L.softmax.argtypes = [_vp, _i]
        L.silu.restype = _f
        L.silu.argtypes = [_f]
        L.ref_attn_layer.restype = _i
        L.ref_attn_layer.argtypes = [_i, _i, _i, _i, _f, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _i, _vp, _i, _i, _vp, _vp, _i, _vp]
        L.ref_eval_decode.restype = _i
        L.ref_eval_decode.argtypes = [_c.c_char_p, _i, _i, _vp, _i, _i, _c.c_double, _vp, _vp,
                                      _vp, _vp]
        L.ref_set_gap_out.restype = None
        L.ref_set_gap_out.argtypes = [_vp]
        L.ref_set_logits0_out.restype = None
        L.ref_set_logits0_out.argtypes = [_vp]
        L.ref_threads_init_pinned.restype = _i
        L.ref_threads_init_pinned.argtypes = [_i, _i]
        self.L = L
        # the pool is process-global: the first call fixes the thread count (and pinning)
        self.threads = L.ref_threads_init_pinned(threads if threads else 1, 1 if pin else 0)

    def eval_decode(self, path, ids, gen, K=None, L=0, vocab=0, max_seconds=0.0, route=False,
                    gap=False, logits0=False):
        """The reference eval driver's --decode flow (ref_eval_decode): greedy tokens after
        prefilling `ids`. Returns dict(tokens, step_ms, prefill_ms[, route (L, n, K)]) with
        as many tokens as were produced before max_seconds of decode."""
        ids = np.ascontiguousarray(ids, np.int32)
        toks = np.zeros(gen, np.int32)
        steps = np.zeros(gen, np.float32)
        pre = np.zeros(1, np.float32)
        rt = np.zeros((L, gen, K), np.int32) if route else None
        gp = np.zeros(gen, np.float32)
        lg0 = np.zeros(max(vocab, 1), np.float32) if logits0 else None
        if logits0 and vocab <= 0:
            raise ValueError("logits0 needs the vocabulary size")
        self.L.ref_set_gap_out(gp.ctypes.data if gap else None)
        self.L.ref_set_logits0_out(_p(lg0))
        n = self.L.ref_eval_decode(str(path).encode(), L, vocab, ids.ctypes.data, ids.size, gen,
                                   max_seconds, toks.ctypes.data, _p(rt), steps.ctypes.data,
                                   pre.ctypes.data)
        if n < 0:
            raise RuntimeError(f"ref_eval_decode returned {n}")
        out = dict(tokens=toks[:n], step_ms=steps[:n], prefill_ms=float(pre[0]))
        if route:
            out["route"] = rt[:, :n]
        if gap:
            out["gap"] = gp[:n]
        if logits0 and n > 0:
            out["logits0"] = lg0
        self.L.ref_set_logits0_out(None)
        return out

    def moe(self, spec, wgate, ln2, experts, x):
        T = x.shape[0]
        x = np.ascontiguousarray(x, dtype=np.float32)
        mlp = np.empty((T, spec.D), np.float32)
        router = np.empty((T, spec.E), np.float32)
        topk = np.empty((T, spec.K), np.int32)
        rc = self.L.ref_moe_layer(spec.D, spec.E, spec.K, spec.F, spec.eps, ln2.ctypes.data,
                                  np.ascontiguousarray(wgate).ctypes.data, _ptr_array(experts),
                                  spec.enc, x.ctypes.data, T, mlp.ctypes.data,
                                  router.ctypes.data, topk.ctypes.data)
        if rc:
            raise RuntimeError(f"ref_moe_layer returned {rc}")
        return dict(router=router, topk=topk, mlp=mlp)

    def attn(self, a, x, pos0, kc, vc):
        """The reference's qwen3_layer_kv attention half (o->attn) for layer dict `a`; the
        cache arrays kc/vc (cap, KV*HD) are read and written in place."""
        T = x.shape[0]
        out = np.empty((T, a["D"]), np.float32)
        x = np.ascontiguousarray(x, np.float32)
        rc = self.L.ref_attn_layer(a["D"], a["H"], a["KV"], a["HD"], a["theta"], a["eps"],
                                   a["ln1"].ctypes.data, a["qn"].ctypes.data,
                                   a["kn"].ctypes.data, a["wq"].ctypes.data,
                                   a["wk"].ctypes.data, a["wv"].ctypes.data,
                                   a["wo"].ctypes.data, a["enc"], x.ctypes.data, T, pos0,
                                   kc.ctypes.data, vc.ctypes.data, kc.shape[0],
                                   out.ctypes.data)
        if rc:
            raise RuntimeError(f"ref_attn_layer returned {rc}")
        return out

    def dequant_row(self, enc, blocks, n):
        out = np.empty(n, dtype=np.float32)
        fn = self.L.q4_dequant_row if enc == 4 else self.L.q8_dequant_row
        fn(np.ascontiguousarray(blocks).ctypes.data, out.ctypes.data, n)
        return out

    def matmul(self, enc, w, x, n_in, n_out):
        out = np.empty(n_out, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w)
        fn = {4: self.L.matmul_wx_q4, 8: self.L.matmul_wx_q8, 0: self.L.matmul_wx}[enc]
        fn(out.ctypes.data, x.ctypes.data, w.ctypes.data, n_in, n_out)
        return out

    def softmax(self, x):
        y = np.array(x, dtype=np.float32, copy=True)
        self.L.softmax(y.ctypes.data, y.size)
        return y

    def rmsnorm(self, x, g, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        self.L.rmsnorm(out.ctypes.data, x.ctypes.data, np.ascontiguousarray(g, dtype=np.float32).ctypes.data, x.size, eps)
        return out
