#!/usr/bin/env python3
"""Write tests/golden/bruteforce.npz: golden vectors for the FP64 oracle.

The expected outputs come from a pure-Python brute-force attention (explicit
loops, math.fsum, math.exp) that shares no code with oracle/attention.py.
Inputs are multiples of 1/8 in [-2, 2], exactly representable in BF16, so
every Q.K dot product is exact in FP64; the only rounding is in exp/log and
the final sums.  Semantics are those of the reference harness's FP64 check,
benchmarks/bshd.py:90-100: logits = scale * q.k, key j hidden from query i when
j > i (top-left causal), LSE = natural-log logsumexp, O = softmax . V.

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import struct
from pathlib import Path

import numpy as np

D = 128
OUT = Path(__file__).resolve().parent / "bruteforce.npz"
# The ABI carries the scale as float32; use that value of 1/sqrt(128) exactly.
S128 = struct.unpack("<f", struct.pack("<f", 1 / math.sqrt(D)))[0]

# (batch, heads, sq, sk, causal, scale)
CASES = [
    (1, 1, 1, 1, False, S128),
    (1, 1, 1, 1, True, S128),
    (1, 2, 5, 7, False, S128),
    (1, 2, 5, 7, True, S128),
    (2, 1, 9, 4, False, S128),
    (2, 1, 9, 4, True, S128),
    (1, 1, 6, 6, True, 0.5),
    (1, 3, 17, 31, False, S128),
    (1, 3, 17, 31, True, S128),
]


def value(i: int) -> float:
    """Deterministic multiples of 1/8 in [-2, 2]."""
    return ((i * 7919 + 13) % 33 - 16) / 8.0


def bf16_bits(x: float) -> int:
    """BF16 bits of a float that is exactly representable in BF16."""
    u = struct.unpack(">I", struct.pack(">f", x))[0]
    assert u & 0xFFFF == 0, x
    return u >> 16


def tensor(b, s, h, salt):
    return [[[[value(((bi * s + si) * h + hi) * D + d + salt) for d in range(D)]
              for hi in range(h)] for si in range(s)] for bi in range(b)]


def brute(q, k, v, scale, causal):
    b, sq, h, sk = len(q), len(q[0]), len(q[0][0]), len(k[0])
    o = [[[[0.0] * D for _ in range(h)] for _ in range(sq)] for _ in range(b)]
    lse = [[[0.0] * sq for _ in range(h)] for _ in range(b)]
    for bi in range(b):
        for hi in range(h):
            for i in range(sq):
                logits = []
                for j in range(sk):
                    if causal and j > i:
                        continue
                    dot = math.fsum(q[bi][i][hi][d] * k[bi][j][hi][d] for d in range(D))
                    logits.append((j, dot * scale))
                m = max(x for _, x in logits)
                w = [(j, math.exp(x - m)) for j, x in logits]
                total = math.fsum(e for _, e in w)
                for d in range(D):
                    o[bi][i][hi][d] = math.fsum(e * v[bi][j][hi][d] for j, e in w) / total
                lse[bi][hi][i] = m + math.log(total)
    return o, lse


def main():
    arrays, meta = {}, []
    for n, (b, h, sq, sk, causal, scale) in enumerate(CASES):
        q, k, v = tensor(b, sq, h, 0), tensor(b, sk, h, 1000003), tensor(b, sk, h, 2000029)
        o, lse = brute(q, k, v, scale, causal)
        for name, t in (("q", q), ("k", k), ("v", v)):
            arrays[f"c{n}_{name}"] = np.array(
                [[[[bf16_bits(x) for x in row] for row in s] for s in bb] for bb in t], dtype=np.uint16)
        arrays[f"c{n}_o"] = np.array(o, dtype=np.float64)
        arrays[f"c{n}_lse"] = np.array(lse, dtype=np.float64)
        meta.append(dict(batch=b, heads=h, sq=sq, sk=sk, causal=causal, scale=scale))
        print(f"case {n}: b{b} h{h} {sq}x{sk} causal={causal} scale={scale}")
    arrays["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
