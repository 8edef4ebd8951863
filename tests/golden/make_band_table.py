"""Exhaustive record of ceil(log2(x)) for every positive normal float32 x.

The reference computes a row's scale exponent as ceil(tl.log2(row_max))
(/root/reference/ozaki_triton.py:174); under the Triton interpreter tl.log2 is
numpy's float32 log2.  For each binade 2^k <= x < 2^(k+1) this script checks
that ceil(log2 x) is k for the mantissas j in [0, J] and k + 1 for all larger
ones, and writes J per k to ceil_log2_band.json.  Also records the integer
exponents e in [-149, 127] where numpy's float32 exp2(e) is not exactly 2^e.

Run: python tests/golden/make_band_table.py   (about a minute, numpy only)
"""
import json
import math
import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ceil_log2_band.json")


def main():
    band = {}
    j = np.arange(1 << 23, dtype=np.uint32)
    for k in range(-126, 128):
        x = (((k + 127) << 23) | j).view(np.float32)
        E = np.ceil(np.log2(x)).astype(np.int64)
        lo = E == k
        J = int(np.nonzero(lo)[0].max())
        assert lo[: J + 1].all(), k
        assert (E[J + 1:] == k + 1).all(), k
        band[str(k)] = J
    e = np.arange(-149, 128)
    inexact = [int(t) for t in e if np.exp2(np.float32(t)) != np.float32(math.ldexp(1.0, int(t)))]
    with open(OUT, "w") as f:
        json.dump({"numpy": np.__version__, "band_J": band, "exp2_inexact": inexact}, f,
                  indent=0, sort_keys=True)
    print(f"wrote {OUT}: {sum(1 for v in band.values() if v)} banded exponents, "
          f"exp2 inexact at {inexact}")


if __name__ == "__main__":
    main()
