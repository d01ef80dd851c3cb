"""Restatement of the synthetic-data generator (TEST INFRASTRUCTURE ONLY).

The measured workloads draw every input from SplitMix64 (Steele, Lea and
Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014; the
64-bit finaliser constants of Vigna's splitmix64.c): output k of the generator
seeded with S is mix(S + (k + 1) * 0x9E3779B97F4A7C15).  Streams are ranges of
2^40 outputs.  A uniform is the top 53 bits times 2^-53; a normal is the
Box-Muller cosine branch over outputs 2i and 2i + 1 in binary64.

Written with Python integers and the `math` module, element by element, so it
shares no code with the product's numpy (workloads.py) or HIP (synth.hip)
versions.  Pinned by the published SplitMix64 outputs for seed 1234567
(tests/test_synth.py) and by distribution checks there.
"""
from __future__ import annotations

import math

_M64 = (1 << 64) - 1


def splitmix(seed: int, k: int) -> int:
    z = (seed + (k + 1) * 0x9E3779B97F4A7C15) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def uniform(seed: int, stream: int, i: int) -> float:
    return (splitmix(seed, (stream << 40) + i) >> 11) * 2.0 ** -53


def normal(seed: int, stream: int, i: int) -> float:
    u0 = uniform(seed, stream, 2 * i)
    u1 = uniform(seed, stream, 2 * i + 1)
    return math.sqrt(-2.0 * math.log(1.0 - u0)) * math.cos(2.0 * math.pi * u1)


def element(seed: int, stream: int, i: int, std: float = 1.0, outlier_stream: int = -1,
            outlier_frac: float = 0.0) -> float:
    """Element i as pam_synth_normal defines it, before rounding to the output type."""
    x = normal(seed, stream, i) * std
    if outlier_stream >= 0 and uniform(seed, outlier_stream, i) < outlier_frac:
        x *= 8.0
    return x
