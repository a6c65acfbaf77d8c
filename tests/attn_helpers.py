"""Synthetic attention layers (the attention half of a Qwen3 decoder layer) for the tests:
seeded weights from the counter-based generator, encoded like the reference's files."""
import ctypes

import numpy as np

import cachepotato_amd as C
from cachepotato_amd import synth


def attn_layer(D=256, H=4, KV=2, HD=64, enc=4, seed=synth.SEED, layer=0, theta=1e6, eps=1e-6):
    """dict with the layer's geometry and host weights: ln1/qn/kn f32 gains near 1, Wq (H*HD, D),
    Wk/Wv (KV*HD, D), Wo (D, H*HD) as v4 blocks of `enc` (f32 arrays for enc 0)."""
    def mat(idx, rows, cols, sigma):
        sid = C.stream_id(layer, C.K_ATTN, idx)
        if enc == 0:
            return C.gen_normal(seed, sid, rows * cols, sigma).reshape(rows, cols)
        return C.gen_blocks(enc, seed, sid, rows * cols, sigma)
    def gain(idx, n):
        return (1.0 + C.gen_normal(seed, C.stream_id(layer, C.K_NORM, idx), n, 0.1)).astype(np.float32)
    s = 1.0 / np.sqrt(D)
    return dict(D=D, H=H, KV=KV, HD=HD, enc=enc, theta=np.float32(theta), eps=np.float32(eps),
                ln1=gain(1, D), qn=gain(2, HD), kn=gain(3, HD),
                wq=mat(0, H * HD, D, s), wk=mat(1, KV * HD, D, s),
                wv=mat(2, KV * HD, D, s), wo=mat(3, D, H * HD, 1.0 / np.sqrt(H * HD)))


def inputs(D, first, n, seed=synth.SEED):
    return C.gen_normal(seed, C.stream_id(0, C.K_INPUT, 0), n * D, 1.0, first=first * D).reshape(n, D)


class DeviceAttn:
    """One attention layer resident on the device (cpg_attn_layer) with a cache of `cap`
    positions and a workspace for max_T tokens."""

    def __init__(self, a, cap=64, max_T=16):
        L = C.lib()
        D, H, KV, HD, enc = a["D"], a["H"], a["KV"], a["HD"], a["enc"]
        self.a, self.cap = a, cap
        nqkv = (H + 2 * KV) * HD
        self.wqkv = C.DeviceBuffer(L.cpg_matrix_bytes(enc, nqkv, D))
        self.wo = C.DeviceBuffer(L.cpg_matrix_bytes(enc, D, H * HD))
        qkv_v4 = np.concatenate([a["wq"], a["wk"], a["wv"]])
        C.check(L.cpg_upload_matrix(enc, self.wqkv.ptr, qkv_v4.ctypes.data, nqkv, D), "upload")
        C.check(L.cpg_upload_matrix(enc, self.wo.ptr, a["wo"].ctypes.data, D, H * HD), "upload")
        self.ln1, self.qn, self.kn = (C.to_device(a[k]) for k in ("ln1", "qn", "kn"))
        rope = np.empty(cap * HD, np.float32)
        C.check(L.cpg_rope_table(a["theta"], HD, cap, rope.ctypes.data), "rope")
        self.rope_host = rope
        self.rope = C.to_device(rope)
        self.layer = C.AttnLayer(D, H, KV, HD, a["theta"], a["eps"], enc, self.ln1.ptr,
                                 self.qn.ptr, self.kn.ptr, self.wqkv.ptr, self.wo.ptr,
                                 self.rope.ptr, cap)
        self.ws = L.cpg_attn_ws_create(D, H, KV, HD, max_T)
        if not self.ws:
            raise C.CPGError(C.last_error())
        self.kc = C.DeviceBuffer(cap * KV * HD * 4).zero()
        self.vc = C.DeviceBuffer(cap * KV * HD * 4).zero()
        self.x = C.DeviceBuffer(max_T * D * 4)
        self.out = C.DeviceBuffer(max_T * D * 4)

    def forward(self, x, pos0):
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        self.x.upload(x)
        C.check(C.lib().cpg_attn_forward(ctypes.byref(self.layer), self.x.ptr, T, pos0,
                                         self.kc.ptr, self.vc.ptr, self.cap, self.out.ptr,
                                         self.ws), "cpg_attn_forward")
        C.sync()
        return self.out.download(np.float32, T * self.a["D"]).reshape(T, self.a["D"])

    def forward_at(self, x, pos0):
        """cpg_attn_forward_at with the position read from device memory."""
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        self.x.upload(x)
        pos = C.to_device(np.array([pos0], np.int32))
        C.check(C.lib().cpg_attn_forward_at(ctypes.byref(self.layer), self.x.ptr, T, pos.ptr,
                                            self.kc.ptr, self.vc.ptr, self.cap, self.out.ptr,
                                            self.ws), "cpg_attn_forward_at")
        C.sync()
        pos.close()
        return self.out.download(np.float32, T * self.a["D"]).reshape(T, self.a["D"])

    def set_cache(self, kc, vc):
        """Replace the whole cache (cap rows of KV * HD floats each)."""
        self.kc.upload(np.ascontiguousarray(kc, np.float32))
        self.vc.upload(np.ascontiguousarray(vc, np.float32))

    def cache(self):
        n = self.cap * self.a["KV"] * self.a["HD"]
        return (self.kc.download(np.float32, n).reshape(self.cap, -1),
                self.vc.download(np.float32, n).reshape(self.cap, -1))

    def close(self):
        C.lib().cpg_attn_ws_destroy(self.ws)
        for b in (self.wqkv, self.wo, self.ln1, self.qn, self.kn, self.rope, self.kc, self.vc,
                  self.x, self.out):
            b.close()
