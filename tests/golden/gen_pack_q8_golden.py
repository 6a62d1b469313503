#!/usr/bin/env python3
"""Write golden vectors for pack_q8 by running the reference's own packer.

Run once, in the build container only (the reference tree is not present on
GPU machines):

    python tests/golden/gen_pack_q8_golden.py /root/reference

It imports ``pack_q8`` from qwen3_mojo/scripts/quantize.py:31-43 of the
reference tree given on the command line, feeds it the bf16 inputs built
below, and stores inputs (bf16 bit patterns) and outputs (packed u16 rows)
in tests/golden/pack_q8_golden.npz.  Only data is stored: no reference code
travels with the fixture.

Cases (each a bf16 [n, m] matrix):
  normal  8 x 512  N(0, 0.02) rounded to bf16, seed 0
  sweep   128 x 512 every finite bf16 value, grouped 64 at a time by
          magnitude (so every scale regime occurs: zero, f16-subnormal,
          normal, overflowing-to-inf), shuffled within each group, seed 1
  edge    hand-built groups: zero, scale-0 (tiny), scale-0 boundary,
          f16-subnormal scales with clipping, exact ties for half-to-even,
          scale overflow to inf, single nonzero, all equal, negative max
  tiny    1 x 64 (smallest legal shape)
  odd     3 x 192 N(0, 1) seed 2
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "pack_q8_golden.npz")


def f32_to_bf16_bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def bits_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def case_normal():
    rng = np.random.default_rng(0)
    return f32_to_bf16_bits(rng.standard_normal((8, 512), dtype=np.float32) * np.float32(0.02))


def case_sweep():
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bits_to_f32(allb)
    finite = allb[np.isfinite(f)]
    mag = np.abs(bits_to_f32(finite))
    order = np.argsort(mag, kind="stable")
    vals = finite[order]
    pad = 65536 - vals.size
    vals = np.concatenate([vals, np.zeros(pad, dtype=np.uint16)])
    groups = vals.reshape(-1, 64)
    rng = np.random.default_rng(1)
    for g in groups:
        rng.shuffle(g)
    return groups.reshape(128, 512)


def _group(vals):
    v = np.zeros(64, dtype=np.float32)
    v[: len(vals)] = vals
    return v


def case_edge():
    rng = np.random.default_rng(3)
    groups = []
    groups.append(_group([]))                                   # all zero
    groups.append(rng.uniform(-3e-6, 3e-6, 64).astype(np.float32))  # scale -> 0
    groups.append(_group([3e-6, -1e-6, 0.0, 2e-7]))             # scale 0 with zeros
    for amax in (3.70e-6, 3.78e-6, 3.79e-6, 3.80e-6, 3.9e-6, 7.6e-6):  # boundary
        g = rng.uniform(-amax, amax, 64).astype(np.float32)
        g[5] = amax
        groups.append(g)
    for amax in (1e-5, 1e-4, 3e-4, 1e-3, 5e-3, 7.7e-3, 7.8e-3):      # subnormal scale
        g = rng.uniform(-amax, amax, 64).astype(np.float32)
        g[7] = -amax
        groups.append(g)
    k = np.arange(-127, 127, dtype=np.float32) + np.float32(0.5)  # ties, scale 1.0
    for c0 in range(0, k.size, 63):
        anchor = -127.0 if (c0 // 63) % 2 else 127.0
        groups.append(_group(list(k[c0:c0 + 63]) + [anchor]))
    groups.append(_group([63.5] + list(np.arange(-31.75, 31.75, 0.5, dtype=np.float32)[:63])))  # scale 0.5
    for amax in (8.3e6, 8.32e6, 8.3211e6, 8.33e6, 1e30):        # f16 scale overflow
        g = rng.uniform(-amax, amax, 64).astype(np.float32)
        g[0] = amax
        groups.append(g)
    groups.append(_group([0.0] * 20 + [-0.75]))                 # single nonzero
    groups.append(np.full(64, 0.3, dtype=np.float32))           # all equal
    groups.append(np.full(64, -2.5, dtype=np.float32))          # all equal negative
    g = rng.standard_normal(64).astype(np.float32)
    g[11] = -7.0                                                # negative max
    groups.append(g)
    g = rng.standard_normal(64).astype(np.float32) * np.float32(1e-2)
    groups.append(g)
    n_groups = len(groups)
    per_row = 4
    rows = (n_groups + per_row - 1) // per_row
    while len(groups) < rows * per_row:
        groups.append(_group([]))
    mat = np.stack(groups).reshape(rows, per_row * 64)
    return f32_to_bf16_bits(mat)


def case_tiny():
    rng = np.random.default_rng(4)
    return f32_to_bf16_bits(rng.standard_normal((1, 64), dtype=np.float32))


def case_odd():
    rng = np.random.default_rng(2)
    return f32_to_bf16_bits(rng.standard_normal((3, 192), dtype=np.float32))


def main():
    if len(sys.argv) != 2:
        sys.exit("usage: gen_pack_q8_golden.py <reference-root>")
    ref_root = sys.argv[1]
    # the reference tree is read-only input: importing from it must not
    # leave compiled bytecode (__pycache__) behind in it
    sys.dont_write_bytecode = True
    sys.path.insert(0, os.path.join(ref_root, "qwen3_mojo", "scripts"))
    import torch
    from quantize import GROUP, pack_q8  # reference packer (quantize.py:28,31)

    assert GROUP == 64
    out = {}
    for name, fn in (("normal", case_normal), ("sweep", case_sweep),
                     ("edge", case_edge), ("tiny", case_tiny), ("odd", case_odd)):
        bits = fn()
        t = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
        packed = pack_q8(t)
        pk = packed.numpy().view(np.uint16).copy()
        out[f"{name}_in"] = bits
        out[f"{name}_out"] = pk
        print(name, bits.shape, "->", pk.shape)
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
