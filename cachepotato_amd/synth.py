"""Synthetic Qwen3-30B-A3B-shaped MoE workloads, built from the counter-based generator of
cpg_math.h (host side: libcachepotato_amd's cpg_gen_host / cpg_gen_blocks_host).

A layer of a workload is fully determined by (seed, layer, geometry, encoding, bias):
  Wgate (E, D) f32   = N(0, 0.02) [- (row . c) c + alpha * ln(p_zipf(e)) * c]
                                                                  stream (layer, WGATE, 0)
  expert e, Wg/Wu (F, D) and Wd (D, F) = N(0, 0.02), Q4_0/Q8_0     streams (layer, WG/WU/WD, e)
  ln2 = ones (the model's norms are ones in the random-init configs)
  input vector v (D) = N(0, 1) [+ gamma * sqrt(D) * c]              stream (0, INPUT, v)
c is the unit vector along stream (0, WGATE, 1), the same for every layer, and
p_zipf(e) = r(e)^-s / H with r(e) the rank of expert e under the ordering of stream
(layer, WGATE, 2), so each layer has its own popular experts.

The biased (Zipf) router: the inputs' shift gamma*sqrt(D)*c adds alpha*ln p_zipf(e) times a
fixed factor to every token's logit of expert e, and the random rows add independent noise
per token, so each token's top-K is a noisy draw favouring popular experts. The random rows'
own components along c are removed first: left in, the shift would add a second fixed
per-expert offset (row . c, as large as the noise), which concentrates every token on the
same few experts (37 distinct of 128 per 16 tokens instead of the ~54 of independent Zipf
draws). With them removed, alpha = 0.011 at gamma = 1 gives ~54. The direction is shared
by the layers because the inputs are: with a direction per layer, a layer other than 0
would see the inputs' shift only through its random rows (the fixed offsets above) and
none of its Zipf bias.

Everything that is not an IEEE basic operation is done where it is reproducible: the norm
of c with math.fsum, ln with math.log (glibc); the rest is elementwise float64 arithmetic
rounded once to float32.
"""
import math
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass

import numpy as np

from . import ENC_Q4, ENC_Q8, BLOCK_BYTES, K_WGATE, K_WG, K_WU, K_WD, K_INPUT
from . import gen_normal, gen_blocks, stream_id

SEED = 20261017


@dataclass(frozen=True)
class MoESpec:
    D: int = 2048
    E: int = 128
    K: int = 8
    F: int = 768
    enc: int = ENC_Q4
    alpha: float = 0.0       # Zipf bias strength in Wgate (0 = none)
    zipf_s: float = 1.1
    gamma: float = 0.0       # shift of the inputs along c
    seed: int = SEED
    layer: int = 0
    eps: float = 1e-6

    def with_layer(self, layer):
        return MoESpec(self.D, self.E, self.K, self.F, self.enc, self.alpha, self.zipf_s,
                       self.gamma, self.seed, layer, self.eps)


# The workloads of the benchmark configurations (hidden 2048, 128 experts, top-8, F=768)
CONFIGS = {
    "q8_b1": MoESpec(enc=ENC_Q8),
    "q4_b1": MoESpec(enc=ENC_Q4),
    "q4_b16_zipf": MoESpec(enc=ENC_Q4, alpha=0.011, gamma=1.0),
    "q4_prefill512": MoESpec(enc=ENC_Q4, gamma=0.6),
}
# Reduced geometry for fast checks
SMALL = {
    "small_q4": MoESpec(D=256, E=16, K=4, F=128, enc=ENC_Q4),
    "small_q8": MoESpec(D=256, E=16, K=4, F=128, enc=ENC_Q8),
}


def _unit_c(spec):
    # one direction for every layer: the inputs (shared by the layers) are shifted along it
    c = gen_normal(spec.seed, stream_id(0, K_WGATE, 1), spec.D, 1.0).astype(np.float64)
    return c / math.sqrt(math.fsum(float(v) * float(v) for v in c))


def wgate(spec):
    w = gen_normal(spec.seed, stream_id(spec.layer, K_WGATE, 0), spec.E * spec.D, 0.02)
    w = w.reshape(spec.E, spec.D)
    if spec.alpha == 0.0:
        return w
    order = gen_normal(spec.seed, stream_id(spec.layer, K_WGATE, 2), spec.E, 1.0)
    rank = np.empty(spec.E, dtype=np.int64)
    rank[np.argsort(order, kind="stable")] = np.arange(1, spec.E + 1)
    h = math.fsum(r ** -spec.zipf_s for r in range(1, spec.E + 1))
    bias = np.array([spec.alpha * math.log(int(rank[e]) ** -spec.zipf_s / h)
                     for e in range(spec.E)], dtype=np.float64)
    c = _unit_c(spec)
    w = w.astype(np.float64)
    # each row's component along c, summed exactly (fsum of the float64 products)
    along = np.array([math.fsum(w[e] * c) for e in range(spec.E)], dtype=np.float64)
    return (w + (bias - along)[:, None] * c[None, :]).astype(np.float32)


def ln2(spec):
    return np.ones(spec.D, dtype=np.float32)


def inputs(spec, first, n):
    """n input vectors (n, D) starting at vector id `first`."""
    x = np.stack([gen_normal(spec.seed, stream_id(0, K_INPUT, v), spec.D, 1.0)
                  for v in range(first, first + n)])
    if spec.gamma == 0.0:
        return x
    c = _unit_c(spec)
    return (x.astype(np.float64) + spec.gamma * math.sqrt(spec.D) * c[None, :]).astype(np.float32)


def expert_matrix_shape(spec, kind):
    return (spec.F, spec.D) if kind in (0, 1) else (spec.D, spec.F)


def expert_matrix_v4(spec, e, kind):
    """v4-layout bytes of expert e's matrix (kind 0 Wg, 1 Wu, 2 Wd)."""
    rows, cols = expert_matrix_shape(spec, kind)
    k = (K_WG, K_WU, K_WD)[kind]
    return gen_blocks(spec.enc, spec.seed, stream_id(spec.layer, k, e), rows * cols, 0.02)


def experts_v4(spec, threads=8):
    """All experts' matrices as a list indexed e*3 + kind (the reference's QW3Layer.exp)."""
    jobs = [(e, kind) for e in range(spec.E) for kind in range(3)]
    with ThreadPoolExecutor(max_workers=threads) as ex:
        return list(ex.map(lambda j: expert_matrix_v4(spec, *j), jobs))
