"""Input/output vectors of the reference's Q4_0 / Q8_0 encoders (format/q4.py:30-57,
format/q8.py:35-58), written by importing those two numpy-only modules from the reference
tree in the development container. Their rounding edge cases (fp16 rounding of the scale,
float32 division, rint half-to-even, clipping) are not pinned by any fixture the reference
holds, so the vectors are made here from the reference code itself and committed as data
(tests/golden/encoder_vectors.npz). The decoders need no such vectors: q*d is exact.

Usage: python tests/golden/make_encoder_vectors.py [/root/reference]
"""
import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def load(ref, name):
    spec = importlib.util.spec_from_file_location(name, os.path.join(ref, "format", name + ".py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def blocks():
    """Crafted 32-element blocks that land on each rounding boundary, plus random ones."""
    rng = np.random.default_rng(20261017)
    out = [np.zeros(32), np.full(32, 1.0), np.full(32, -1.0), np.full(32, -0.0)]
    # x/d exactly k + 0.5 for every k (ties to even), for both encoders' scales
    for amax, qmax in ((8.0, 8), (127.0, 127), (6.0, 8), (1.5, 8)):
        d = amax / qmax
        b = np.array([(k % 15 - 7 + 0.5) * d for k in range(31)] + [amax])
        out += [b, -b]
    # scales whose fp16 rounding is a tie or near-tie
    for m in (1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -11 + 2 ** -30, 1 - 2 ** -12):
        for e in (-3, 0, 5):
            b = rng.normal(0, 1, 32)
            b *= (m * 2.0 ** e * 8) / np.abs(b).max()
            out.append(b)
            b2 = b.copy()
            b2 *= 127 / 8
            out.append(b2)
    # tiny blocks: the scale is an fp16 subnormal or rounds to zero
    for s in (1e-5, 6e-8 * 8, 3e-8 * 8, 1e-9, 2 ** -24 * 8 * 1.5, 2 ** -24 * 127 * 0.6):
        out.append(rng.normal(0, 1, 32) / 3 * s)
        b = np.zeros(32)
        b[7] = s
        out.append(b)
    # large blocks near the fp16 maximum of the scale
    for s in (65504 * 8 * 0.999, 65504 * 127 * 0.999, 1e4):
        out.append(rng.normal(0, 1, 32) / 3 * s)
    # the -8 end of Q4: a block whose most negative value is its amax
    out.append(np.array([-8.0] + [float(k % 16 - 8) for k in range(31)]))
    out.append(np.array([-1.0] + [0.1 * k for k in range(31)]) * 0.37)
    # random blocks over many magnitudes
    for e in range(-12, 8):
        for _ in range(8):
            out.append(rng.normal(0, 2.0 ** e, 32))
    return np.stack(out).astype(np.float32)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    q4, q8 = load(ref, "q4"), load(ref, "q8")
    x = blocks()
    b4, _ = q4.encode_q4_0(x)
    b8, _ = q8.encode_q8_0(x)
    path = os.path.join(HERE, "encoder_vectors.npz")
    np.savez_compressed(path, x=x, q4=np.frombuffer(b4, np.uint8), q8=np.frombuffer(b8, np.uint8),
                        numpy_version=np.array(np.__version__))
    print(f"{path}: {x.shape[0]} blocks")


if __name__ == "__main__":
    main()
