"""Staging synthetic MoE layers on the GPU through the C ABI (used by the gpu tests and
bench.py). Everything goes through libcachepotato_amd (cpg_* entry points)."""
import ctypes
import hashlib

import numpy as np

import cachepotato_amd as C
from cachepotato_amd import synth


class DeviceMoE:
    """One synthetic MoE layer resident on the device, plus a workspace for max_T tokens."""

    def __init__(self, spec, max_T=16, device_gen=False, check_sha=None):
        L = C.lib()
        self.spec = spec
        D, E, K, F, enc = spec.D, spec.E, spec.K, spec.F, spec.enc
        self.exp_bytes = L.cpg_expert_bytes(enc, D, F)
        self.experts = C.DeviceBuffer(self.exp_bytes * E)
        self.mat_g = L.cpg_matrix_bytes(enc, F, D)
        self.sha_experts = None
        if device_gen:
            self._device_gen(check_sha)
        else:
            mats = synth.experts_v4(spec)
            h = hashlib.sha256()
            for e in range(E):
                for kind in range(3):
                    rows, cols = synth.expert_matrix_shape(spec, kind)
                    b = mats[e * 3 + kind]
                    h.update(b.tobytes())
                    dst = self.experts.ptr + e * self.exp_bytes + kind * self.mat_g
                    C.check(L.cpg_upload_matrix(enc, dst, b.ctypes.data, rows, cols), "upload")
            self.sha_experts = h.hexdigest()
            self.host_mats = mats
        self.wgate_host = synth.wgate(spec)
        self.wgate = C.to_device(self.wgate_host)
        self.ln2 = C.to_device(synth.ln2(spec))
        self.layer = C.MoELayer(D, E, K, F, enc, spec.eps, self.ln2.ptr, self.wgate.ptr,
                                self.experts.ptr)
        self.max_T = max_T
        self.ws = L.cpg_moe_ws_create(D, E, K, F, max_T)
        if not self.ws:
            raise C.CPGError(C.last_error())
        self.x = C.DeviceBuffer(max_T * D * 4)
        self.xn = C.DeviceBuffer(max_T * D * 4)
        self.router = C.DeviceBuffer(max_T * E * 4)
        self.topk = C.DeviceBuffer(max_T * K * 4)
        self.wt = C.DeviceBuffer(max_T * K * 4)
        self.mlp = C.DeviceBuffer(max_T * D * 4)

    def _device_gen(self, check_sha):
        """Generate v4 blocks on the GPU matrix by matrix, hash them on the host (the bytes
        the reference engine consumed when the fixtures were written), repack to tiles."""
        L, s = C.lib(), self.spec
        h = hashlib.sha256()
        maxb = max(s.F * s.D, s.D * s.F) // 32 * C.BLOCK_BYTES[s.enc]
        stage = C.DeviceBuffer(maxb)
        kinds = (C.K_WG, C.K_WU, C.K_WD)
        for e in range(s.E):
            for kind in range(3):
                rows, cols = synth.expert_matrix_shape(s, kind)
                nbytes = rows * cols // 32 * C.BLOCK_BYTES[s.enc]
                C.check(L.cpg_gen_blocks(s.enc, s.seed, C.stream_id(s.layer, kinds[kind], e),
                                         rows, cols, 0.02, stage.ptr), "cpg_gen_blocks")
                if check_sha is not None:
                    h.update(stage.download(np.uint8, nbytes).tobytes())
                dst = self.experts.ptr + e * self.exp_bytes + kind * self.mat_g
                C.check(L.cpg_repack(s.enc, dst, stage.ptr, rows, cols), "cpg_repack")
        C.sync()
        stage.close()
        if check_sha is not None:
            self.sha_experts = h.hexdigest()

    def forward(self, x, mlp_in=None, attn=None, outputs=True, noalloc=False):
        """Run cpg_moe_forward on x (T, D); returns dict of numpy outputs. outputs=False asks
        for neither xn nor the router logits (the certified routing path for T <= 16).
        noalloc=True runs cpg_moe_forward_noalloc instead (the static scratch, no ws)."""
        s, L = self.spec, C.lib()
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        assert T <= self.max_T
        self.x.upload(x)
        if mlp_in is None:
            C.check(L.cpg_memset(self.mlp.ptr, 0, T * s.D * 4), "memset")
        else:
            self.mlp.upload(np.ascontiguousarray(mlp_in, np.float32))
        attn_ptr = None
        if attn is not None:
            self.attn = C.to_device(np.ascontiguousarray(attn, np.float32))
            attn_ptr = self.attn.ptr
        xn_p, rt_p = (self.xn.ptr, self.router.ptr) if outputs else (None, None)
        if noalloc:
            C.check(L.cpg_moe_forward_noalloc(ctypes.byref(self.layer), self.x.ptr, attn_ptr, T,
                                              xn_p, rt_p, self.topk.ptr, self.wt.ptr,
                                              self.mlp.ptr), "cpg_moe_forward_noalloc")
        else:
            C.check(L.cpg_moe_forward(ctypes.byref(self.layer), self.x.ptr, attn_ptr, T,
                                      xn_p, rt_p, self.topk.ptr, self.wt.ptr,
                                      self.mlp.ptr, self.ws), "cpg_moe_forward")
        C.sync()
        out = dict(topk=self.topk.download(np.int32, T * s.K).reshape(T, s.K),
                   wt=self.wt.download(np.float32, T * s.K).reshape(T, s.K),
                   mlp=self.mlp.download(np.float32, T * s.D).reshape(T, s.D))
        if outputs:
            out["xn"] = self.xn.download(np.float32, T * s.D).reshape(T, s.D)
            out["router"] = self.router.download(np.float32, T * s.E).reshape(T, s.E)
        return out

    def forward_res(self, x, attn):
        """cpg_moe_forward_res: returns (x + attn + MoE(x + attn), topk, mlp scratch after)."""
        s, L = self.spec, C.lib()
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        self.x.upload(x)
        self.attn = C.to_device(np.ascontiguousarray(attn, np.float32))
        C.check(L.cpg_memset(self.mlp.ptr, 0, T * s.D * 4), "memset")
        C.check(L.cpg_moe_forward_res(ctypes.byref(self.layer), self.x.ptr, self.attn.ptr, T,
                                      self.topk.ptr, self.mlp.ptr, self.ws), "cpg_moe_forward_res")
        C.sync()
        return (self.x.download(np.float32, T * s.D).reshape(T, s.D),
                self.topk.download(np.int32, T * s.K).reshape(T, s.K),
                self.mlp.download(np.float32, T * s.D).reshape(T, s.D))

    def status(self):
        """waits of the fused kernel that gave up so far (0 when it ran as designed)"""
        n = C.lib().cpg_moe_ws_status(self.ws)
        C.check(min(n, 0), "cpg_moe_ws_status")
        return n

    def fallbacks(self):
        """tokens whose certificate failed so far (routed by the refined or exact fallback)"""
        n = C.lib().cpg_moe_ws_fallbacks(self.ws)
        C.check(min(n, 0), "cpg_moe_ws_fallbacks")
        return n

    def exact_routings(self):
        """of those, the tokens that needed the exact chains of every router row"""
        n = C.lib().cpg_moe_ws_exact_routings(self.ws)
        C.check(min(n, 0), "cpg_moe_ws_exact_routings")
        return n

    def distinct(self):
        return C.lib().cpg_moe_ws_distinct(self.ws)

    def close(self):
        C.lib().cpg_moe_ws_destroy(self.ws)
        for b in (self.experts, self.wgate, self.ln2, self.x, self.xn, self.router, self.topk,
                  self.wt, self.mlp):
            b.close()


class route_mode:
    """with route_mode(C.ROUTE_...): cpg_moe_forward calls inside use that routing mode"""

    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        C.check(C.lib().cpg_moe_route_mode(self.mode), "cpg_moe_route_mode")

    def __exit__(self, *exc):
        C.lib().cpg_moe_route_mode(C.ROUTE_AUTO)


class fused_mode:
    """with fused_mode(False): one-token cpg_moe_forward calls run the separate kernels"""

    def __init__(self, on):
        self.on = on

    def __enter__(self):
        C.check(C.lib().cpg_moe_fused(1 if self.on else 0), "cpg_moe_fused")

    def __exit__(self, *exc):
        C.lib().cpg_moe_fused(0)


class expert_mode:
    """with expert_mode(C.EXPERTS_...): cpg_moe_forward calls inside use that expert path"""

    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        C.check(C.lib().cpg_moe_expert_mode(self.mode), "cpg_moe_expert_mode")

    def __exit__(self, *exc):
        C.lib().cpg_moe_expert_mode(C.EXPERTS_AUTO)


def rel_err(got, want):
    """max |got - want| / max |want| over the whole output (normwise relative error)."""
    want = np.asarray(want, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)
