"""cachepotato_amd — Python access to libcachepotato_amd.so (the C ABI of include/cpg.h).

The GPU work is done by the HIP kernels in the shared library; this module only binds its
C entry points with ctypes and moves numpy arrays in and out. There is no fallback: if the
library is not built, or no GPU is present, the calls raise.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcachepotato_amd.so")

ENC_F32, ENC_Q4, ENC_Q8 = 0, 4, 8
MATH_EXPF, MATH_SQRT, MATH_DIV, MATH_SILU, MATH_F16 = 0, 1, 2, 3, 4
ROUTE_AUTO, ROUTE_EXACT, ROUTE_FORCE_FALLBACK, ROUTE_FORCE_REFINE = 0, 1, 2, 3
EXPERTS_AUTO, EXPERTS_GEMV, EXPERTS_MFMA = 0, 1, 2
ATTN_PER_HEAD, ATTN_SPLIT = 0, 1
KT_ROUTE, KT_SELECT, KT_GATEUP, KT_DOWN, KT_COMBINE, KT_FUSED, KT_COUNT = 0, 1, 2, 3, 4, 5, 6
KT_NAMES = ("route", "select", "gateup", "down", "combine", "fused")
BLOCK_BYTES = {ENC_Q4: 18, ENC_Q8: 34}

# stream kinds of the synthetic generator (cpg_math.h)
K_WGATE, K_WG, K_WU, K_WD, K_INPUT, K_ATTN, K_EMBED, K_HEAD, K_NORM = range(1, 10)


def stream_id(layer, kind, index):
    """CPG_STREAM(layer, kind, index) of cpg_math.h."""
    return (layer << 40) | (kind << 32) | index


class CPGError(RuntimeError):
    pass


_c = ctypes
_vp, _i, _sz, _u64, _f, _d = _c.c_void_p, _c.c_int, _c.c_size_t, _c.c_uint64, _c.c_float, _c.c_double

# (name, restype, argtypes) for every entry point of include/cpg.h
SIGNATURES = [
    ("cpg_init", _i, [_i]),
    ("cpg_shutdown", None, []),
    ("cpg_last_error", _c.c_char_p, []),
    ("cpg_device_count", _i, []),
    ("cpg_device_name", _i, [_c.c_char_p, _sz]),
    ("cpg_malloc", _vp, [_sz]),
    ("cpg_free", _i, [_vp]),
    ("cpg_h2d", _i, [_vp, _vp, _sz]),
    ("cpg_d2h", _i, [_vp, _vp, _sz]),
    ("cpg_memset", _i, [_vp, _i, _sz]),
    ("cpg_sync", _i, []),
    ("cpg_event_record", _i, [_i]),
    ("cpg_event_elapsed_ms", _f, [_i, _i]),
    ("cpg_matrix_bytes", _sz, [_i, _i, _i]),
    ("cpg_expert_bytes", _sz, [_i, _i, _i]),
    ("cpg_repack", _i, [_i, _vp, _vp, _i, _i]),
    ("cpg_upload_matrix", _i, [_i, _vp, _vp, _i, _i]),
    ("cpg_gen_host", None, [_u64, _u64, _u64, _sz, _d, _vp]),
    ("cpg_gen_blocks_host", None, [_i, _u64, _u64, _sz, _d, _vp]),
    ("cpg_gen_experts", _i, [_i, _u64, _i, _i, _i, _i, _vp]),
    ("cpg_gen_blocks", _i, [_i, _u64, _u64, _i, _i, _d, _vp]),
    ("cpg_moe_ws_create", _vp, [_i, _i, _i, _i, _i]),
    ("cpg_moe_ws_destroy", None, [_vp]),
    ("cpg_moe_forward", _i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    ("cpg_moe_forward_noalloc", _i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    ("cpg_head_scratch_bytes", _sz, [_i]),
    ("cpg_head_next", _i, [_i, _vp, _i, _i, _vp, _vp, _f, _vp, _vp, _i, _vp, _i, _vp]),
    ("cpg_moe_ws_distinct", _i, [_vp]),
    ("cpg_moe_timing", _i, [_i]),
    ("cpg_moe_timing_read", _i, [_vp, _vp, _i]),
    ("cpg_moe_ws_fallbacks", _i, [_vp]),
    ("cpg_moe_ws_exact_routings", _i, [_vp]),
    ("cpg_moe_route_mode", _i, [_i]),
    ("cpg_dequant_rows", _i, [_i, _vp, _i, _i, _vp]),
    ("cpg_dequant_tiled", _i, [_i, _vp, _i, _i, _i, _i, _vp]),
    ("cpg_math_dev", _i, [_i, _vp, _vp, _vp, _sz]),
    ("cpg_mm", _i, [_i, _vp, _vp, _i, _i, _vp]),
    ("cpg_current_device", _i, []),
    ("cpg_d2d", _i, [_vp, _vp, _sz]),
    ("cpg_read_stream", _i, [_vp, _sz, _i, _vp]),
    ("cpg_rope_table", _i, [_f, _i, _i, _vp]),
    ("cpg_attn_ws_create", _vp, [_i, _i, _i, _i, _i]),
    ("cpg_attn_ws_destroy", None, [_vp]),
    ("cpg_attn_ws_status", _i, [_vp]),
    ("cpg_attn_forward", _i, [_vp, _vp, _i, _i, _vp, _vp, _i, _vp, _vp]),
    ("cpg_gemv", _i, [_i, _vp, _i, _i, _vp, _i, _vp]),
    ("cpg_rmsnorm", _i, [_vp, _vp, _i, _i, _f, _vp]),
    ("cpg_embed_rows", _i, [_i, _vp, _i, _i, _vp, _i, _vp]),
    ("cpg_residual", _i, [_vp, _vp, _vp, _sz]),
    ("cpg_argmax", _i, [_vp, _i, _vp]),
    ("cpg_attn_forward_at", _i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _vp]),
    ("cpg_gemv_norm", _i, [_i, _vp, _i, _i, _vp, _i, _vp, _f, _vp]),
    ("cpg_moe_forward_res", _i, [_vp, _vp, _vp, _i, _vp, _vp, _vp]),
    ("cpg_moe_expert_mode", _i, [_i]),
    ("cpg_attn_decode_mode", _i, [_i]),
    ("cpg_moe_fused", _i, [_i]),
    ("cpg_moe_ws_status", _i, [_vp]),
    ("cpg_decode_step_end", _i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    ("cpg_capture_begin", _i, []),
    ("cpg_capture_end", _vp, []),
    ("cpg_graph_launch", _i, [_vp]),
    ("cpg_graph_destroy", None, [_vp]),
]


class AttnLayer(ctypes.Structure):
    """cpg_attn_layer of include/cpg.h"""
    _fields_ = [("D", _i), ("H", _i), ("KV", _i), ("HD", _i), ("theta", _f), ("eps", _f),
                ("enc", _i), ("ln1", _vp), ("q_norm", _vp), ("k_norm", _vp), ("wqkv", _vp),
                ("wo", _vp), ("rope", _vp), ("max_pos", _i)]


class MoELayer(ctypes.Structure):
    """cpg_moe_layer of include/cpg.h"""
    _fields_ = [("D", _i), ("E", _i), ("K", _i), ("F", _i), ("enc", _i), ("eps", _f),
                ("ln2", _vp), ("wgate", _vp), ("experts", _vp)]


_lib = None


def lib():
    """Load the shared library once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise CPGError(f"{LIB_PATH} is not built: run `python -m cachepotato_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    return lib().cpg_last_error().decode(errors="replace")


def check(rc, what="cpg call"):
    if rc != 0:
        raise CPGError(f"{what} returned {rc}: {last_error()}")


def init(device=0):
    check(lib().cpg_init(device), "cpg_init")


def device_name():
    buf = ctypes.create_string_buffer(256)
    check(lib().cpg_device_name(buf, 256), "cpg_device_name")
    return buf.value.decode()


class DeviceBuffer:
    """A device allocation owned by Python (freed on close / garbage collection)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().cpg_malloc(self.nbytes)
        if not self.ptr:
            raise CPGError(f"cpg_malloc({self.nbytes}): {last_error()}")

    def upload(self, arr, offset=0):
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes, "upload past the end of the buffer"
        check(lib().cpg_h2d(self.ptr + offset, a.ctypes.data, a.nbytes), "cpg_h2d")
        return self

    def download(self, dtype, count, offset=0):
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes, "download past the end of the buffer"
        check(lib().cpg_d2h(out.ctypes.data, self.ptr + offset, out.nbytes), "cpg_d2h")
        return out

    def zero(self):
        check(lib().cpg_memset(self.ptr, 0, self.nbytes), "cpg_memset")
        return self

    def close(self):
        if self.ptr and _lib is not None:
            _lib.cpg_free(self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def to_device(arr):
    a = np.ascontiguousarray(arr)
    return DeviceBuffer(max(a.nbytes, 1)).upload(a)


def sync():
    check(lib().cpg_sync(), "cpg_sync")


# ---------------------------------------------------------------- host-side generator

def gen_normal(seed, stream, n, sigma, first=0):
    out = np.empty(n, dtype=np.float32)
    lib().cpg_gen_host(seed, stream, first, n, sigma, out.ctypes.data)
    return out


def gen_blocks(enc, seed, stream, n, sigma):
    out = np.empty(n // 32 * BLOCK_BYTES[enc], dtype=np.uint8)
    lib().cpg_gen_blocks_host(enc, seed, stream, n, sigma, out.ctypes.data)
    return out
