"""Writes q4_kat.json: hand-derived known-answer vectors for the 4-bit codec.

The expected codes, bytes and fp16 bit patterns below are worked out by hand
from the reference's definition (usaf/quantization.py:47-132), not produced by
the oracle; numpy's IEEE float16 arithmetic is used only where noted (the
double-rounding case), as a library routine independent of the oracle.

    python tests/golden/make_q4_kat.py      # rewrites tests/golden/q4_kat.json
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

RAMP_BYTES = [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]  # codes 0..15, even index in the low nibble


def s8(b):
    return b - 256 if b >= 128 else b


def kats():
    out = []
    # 1. ramp 0..15 x8: min 0, max 15 -> scale exactly 1.0, codes = values.
    x = [float(i % 16) for i in range(128)]
    out.append(dict(name="ramp", group_size=128, x=x,
                    packed=[[s8(b) for b in RAMP_BYTES * 8]],
                    scale=[0x3C00], zero=[0x0000],
                    dequant_f16=[int(np.float16(v).view(np.uint16)) for v in x]))
    # 2. zero padding joins min/max: group 0 = 1 + ramp/2 (scale 0.5, zero 1.0);
    #    group 1 = [3, 4] + 126 zero pads -> min 0, max 4, scale fp32(4/15) = 0x3E888889,
    #    codes 3/s = 11.2499994 -> 11 and 4/s = 14.9999992 -> 15, pads -> 0.
    g0 = [1.0 + 0.5 * (i % 16) for i in range(128)]
    x = g0 + [3.0, 4.0]
    out.append(dict(name="pad_tail", group_size=128, x=x,
                    packed=[[s8(b) for b in RAMP_BYTES * 8], [s8(11 | (15 << 4))] + [0] * 63],
                    scale=[0x3800, 0x3444], zero=[0x3C00, 0x0000], dequant_f16=None))
    # 3. constant group: max-min = 0 -> scale clamps to 1e-12, which is 0 in fp16;
    #    zero = fp16(0.1f) = 0x2E66; all codes 0; dequant = 0*0 + z = z.
    out.append(dict(name="constant", group_size=128, x=[0.1] * 128,
                    packed=[[0] * 64], scale=[0x0000], zero=[0x2E66], dequant_f16=[0x2E66] * 128))
    # 4. numel < group_size: eff_gs = 5, one group of 3 bytes.  min -1, max 3,
    #    scale fp32(4/15); codes (x+1)/s = 0, 3.7499998 -> 4, 7.4999995 -> 7,
    #    11.2499994 -> 11, 14.9999992 -> 15.
    out.append(dict(name="tiny", group_size=128, x=[-1.0, 0.0, 1.0, 2.0, 3.0],
                    packed=[[s8(0 | (4 << 4)), s8(7 | (11 << 4)), s8(15)]],
                    scale=[0x3444], zero=[0xBC00], dequant_f16=None))
    # 5. odd group size 3: groups [1,2,3], [4,5,6]; scale fp32(2/15) = 0.13333334,
    #    codes 0, 1/s = 7.4999997 -> 7, 2/s = 14.9999995 -> 15 -> bytes [0x70, 0x0F].
    out.append(dict(name="odd_gs3", group_size=3, x=[1.0, 2.0, 3.0, 4.0, 5.0, 6.0],
                    packed=[[0x70, 0x0F], [0x70, 0x0F]],
                    scale=[0x3044, 0x3044], zero=[0x3C00, 0x4400], dequant_f16=None))
    # 6. the reference's odd-group dequant reads nibble i of the flat code bytes
    #    (interleave, flatten, slice), so group 1 starts at the pad nibble of group 0:
    #    bytes [[0x21,0x03],[0x54,0x06]] -> nibbles 1,2,3,0,4,5,6,0 -> groups
    #    [1,2,3] and [0,4,5]; scale [1, 2], zero [0, 100] -> [1,2,3,100,108,110].
    out.append(dict(name="odd_gs3_dequant_layout", group_size=3, x=None,
                    packed=[[0x21, 0x03], [0x54, 0x06]],
                    scale=[0x3C00, 0x4000], zero=[0x0000, 0x5640],
                    dequant_f16=[int(np.float16(v).view(np.uint16)) for v in [1, 2, 3, 100, 108, 110]]))
    # 7. two roundings: find (q, s, z) where fp16(fp16(q*s)+z) differs from the
    #    single rounding fp16(q*s+z); expected values from numpy float16 ops.
    rng = np.random.default_rng(7)
    cases = []
    while len(cases) < 32:
        q = int(rng.integers(1, 16))
        s = np.float16(rng.uniform(1e-3, 2e-2))
        z = np.float16(rng.uniform(-0.2, 0.0))
        two = np.float16(np.float16(np.float16(q) * s) + z)
        one = np.float16(np.float64(q) * np.float64(s) + np.float64(z))
        if two != one:
            cases.append((q, int(s.view(np.uint16)), int(z.view(np.uint16)), int(two.view(np.uint16)),
                          int(one.view(np.uint16))))
    out.append(dict(name="double_rounding", group_size=None, cases=cases))
    return out


if __name__ == "__main__":
    path = os.path.join(HERE, "q4_kat.json")
    with open(path, "w") as f:
        json.dump(kats(), f, indent=1)
    print(f"wrote {path}")
