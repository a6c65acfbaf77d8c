"""Host-side checks of the product library that need no GPU: it loads, exports every
entry point its headers declare, fails loudly without a device, and its host generator
reproduces the bytes the golden fixtures were made from."""
import glob
import os
import re

import numpy as np
import pytest

import cachepotato_amd as C
from cachepotato_amd import synth
from tests.conftest import golden, ROOT


def declared(header):
    src = open(header).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b(cpg_\w+|qwen3_\w+|cp_\w+)\s*\(", src)
    return sorted(set(n for n in names if not n.endswith("_t")))


def test_library_exports_every_declared_symbol():
    L = C.lib()
    headers = glob.glob(os.path.join(ROOT, "include", "*.h"))
    assert headers
    missing = [n for h in headers for n in declared(h) if not hasattr(L, n)]
    assert not missing, missing


def test_bindings_cover_cpg_header():
    names = declared(os.path.join(ROOT, "include", "cpg.h"))
    bound = {s[0] for s in C.SIGNATURES}
    assert set(names) <= bound, set(names) - bound


def test_no_gpu_fails_loudly():
    L = C.lib()
    if L.cpg_device_count() > 0:
        pytest.skip("a GPU is present")
    assert L.cpg_init(0) == -7
    assert "GPU" in C.last_error() or "device" in C.last_error()
    assert L.cpg_malloc(16) is None


def test_layout_sizes():
    L = C.lib()
    # Q4_0 expert: 3 matrices of 768x2048 elements at 18 B / 32 elements, planes 256-aligned
    assert L.cpg_expert_bytes(4, 2048, 768) == 3 * 1572864 // 32 * 18
    assert L.cpg_expert_bytes(8, 2048, 768) == 3 * 1572864 // 32 * 34
    assert L.cpg_matrix_bytes(4, 64, 32) == 1024 + 256


def test_generator_statistics():
    v = C.gen_normal(1, 2, 1 << 20, 0.02).astype(np.float64)
    assert abs(v.mean()) < 1e-4 and abs(v.std() - 0.02) < 2e-4
    # Irwin-Hall(12): bounded by 6 sigma, symmetric
    assert np.abs(v).max() <= 6 * 0.02 and abs((v > 0).mean() - 0.5) < 2e-3
    # counter-based: any window equals the same elements of a longer draw
    assert np.array_equal(C.gen_normal(1, 2, 100, 0.02, first=5000), C.gen_normal(1, 2, 5100, 0.02)[5000:])


def test_host_blocks_equal_oracle_encoder(oracle):
    f = C.gen_normal(5, 6, 32 * 1000, 0.02)
    for enc in (4, 8):
        assert np.array_equal(C.gen_blocks(enc, 5, 6, f.size, 0.02), oracle.encode(enc, f))


@pytest.mark.parametrize("name", ["small_q4", "small_q8", "q4_b1"])
def test_host_generator_matches_fixture(name):
    from tests.golden.make_golden import sha, spec_of
    z = golden(f"moe_{name}_t1.npz")
    spec = spec_of(name)
    assert sha(synth.wgate(spec)) == str(z["sha_wgate"])
    assert sha(*synth.experts_v4(spec)) == str(z["sha_experts"])


def test_zipf_workload_is_skewed():
    """The batch-16 workload's router bias makes popular experts: few distinct per batch."""
    z = golden("moe_q4_b16_zipf_t1.npz")
    distinct = [len(set(z["topk"][16 * b:16 * b + 16].ravel())) for b in range(8)]
    assert max(distinct) < 64 < 16 * 8
    z = golden("moe_q4_prefill512_t1.npz")
    counts = np.bincount(z["topk"].ravel(), minlength=128)
    assert counts.mean() == 32 and counts.max() > 100
