"""T5 relative-position buckets, restated for the oracle.

TEST INFRASTRUCTURE ONLY (imported by tests/ and the CPU baseline, never by the product).

`relative_bucket` follows app/models/t5.js:14-23, itself a float32 emulation of HF
T5Attention._relative_position_bucket (transformers modeling_t5.py:217-262):
  bidirectional: nb = num_buckets/2, bucket = nb if rel > 0 else 0, n = |rel|
  unidirectional: nb = num_buckets, bucket = 0, n = -min(rel, 0)
  max_exact = nb/2; n < max_exact -> bucket + n; else
  bucket + min(max_exact + trunc(f32(f32(f32(log(f32(n/max_exact))) / f32(log(max_distance/max_exact)))
                                     * (nb - max_exact))), nb - 1)
with each f32 a round to float32 and log correctly rounded (Math.fround(Math.log(x))).

`bucket_thresholds` is the closed form in exact arithmetic: with max_exact = 8, nb = 16 and
max_distance = 128, bucket 8 + k starts at n = ceil(8 * 2**(k/2)), i.e. at 8, 12, 16, 23, 32, 46,
64, 91 (and everything >= 91 is bucket 15).
"""

from __future__ import annotations

import math

import numpy as np


def _f32(x: float) -> float:
    return float(np.float32(x))


def relative_bucket(rel: int, bidirectional: bool = True, num_buckets: int = 32, max_distance: int = 128) -> int:
    nb = num_buckets
    bucket = 0
    if bidirectional:
        nb //= 2
        if rel > 0:
            bucket = nb
        n = abs(rel)
    else:
        n = -min(rel, 0)
    max_exact = nb // 2
    if n < max_exact:
        return bucket + n
    lg = _f32(math.log(_f32(n / max_exact)))
    den = _f32(math.log(max_distance / max_exact))
    large = max_exact + int(_f32(_f32(lg / den) * (nb - max_exact)))
    return bucket + min(large, nb - 1)


def bucket_lut(Lq: int, Lk: int, bidirectional: bool = True, num_buckets: int = 32, max_distance: int = 128) -> np.ndarray:
    """int32 [Lq + Lk - 1]: bucket of rel = j - i at index rel + Lq - 1."""
    return np.array([relative_bucket(r, bidirectional, num_buckets, max_distance) for r in range(-(Lq - 1), Lk)],
                    dtype=np.int32)


def bucket_thresholds(num_buckets: int = 32, max_distance: int = 128, bidirectional: bool = True) -> list[int]:
    """First |rel| of each logarithmic bucket, from the exact-arithmetic closed form:
    bucket(n) = max_exact + floor(log(n/max_exact) / log(max_distance/max_exact) * (nb - max_exact)),
    so bucket max_exact + k begins at the smallest integer n with
    n >= max_exact * (max_distance/max_exact) ** (k / (nb - max_exact))."""
    nb = num_buckets // 2 if bidirectional else num_buckets
    max_exact = nb // 2
    out = []
    for k in range(nb - max_exact):
        x = max_exact * (max_distance / max_exact) ** (k / (nb - max_exact))
        n = math.ceil(x - 1e-9)
        out.append(n)
    return out
