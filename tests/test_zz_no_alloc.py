"""cpg_moe_forward_noalloc (the entry point that allocates nothing: its workspace is a static
device array) computes what cpg_moe_forward computes with its own workspace, bit for bit, on
two calls in a row (the second smaller), for both routing paths (the certified one when
neither xn nor the router logits are asked for, the exact chains when they are), and after a
call of another geometry has used the same array. It refuses T beyond its maximum."""
import ctypes

import numpy as np
import pytest

import cachepotato_amd as C
from cachepotato_amd import synth
from tests.gpu_helpers import DeviceMoE, bits

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def same(a, b, what):
    for k in a:
        assert np.array_equal(bits(a[k]) if a[k].dtype == np.float32 else a[k],
                              bits(b[k]) if b[k].dtype == np.float32 else b[k]), (what, k)


@pytest.mark.parametrize("name", ["q4_b16_zipf", "q8_b1"])
def test_noalloc_equals_forward(cpg, name):
    spec = synth.CONFIGS[name]
    say(f"noalloc: {name}, T = 16 then 1, both routing paths")
    m = DeviceMoE(spec, max_T=16, device_gen=True)
    small = DeviceMoE(synth.SMALL["small_q4"], max_T=16)
    try:
        x = synth.inputs(spec, 0, 16)
        for outputs in (False, True):
            for T in (16, 1):                    # two calls in a row, the second smaller
                want = m.forward(x[:T], outputs=outputs)
                got = m.forward(x[:T], outputs=outputs, noalloc=True)
                same(got, want, (name, T, outputs))
                say(f"  T={T} outputs={outputs}: identical")
            # another geometry through the same array, then this one again
            xs = synth.inputs(small.spec, 0, 5)
            same(small.forward(xs, noalloc=True), small.forward(xs), "small")
            same(m.forward(x[:3], outputs=outputs, noalloc=True),
                 m.forward(x[:3], outputs=outputs), (name, 3, outputs))
        L = C.lib()
        rc = L.cpg_moe_forward_noalloc(ctypes.byref(m.layer), m.x.ptr, None, 17, None, None,
                                       m.topk.ptr, m.wt.ptr, m.mlp.ptr)
        assert rc == -1 and "T=17" in C.last_error()
    finally:
        small.close()
        m.close()
