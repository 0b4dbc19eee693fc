"""Extract the Q4_0 cases of the reference's quantisation fixture into a small
numpy archive used by the tests.

Source: ref/quant_fixture.bin of the lfm2-ampere repository (written by its
tests/make_quant_fixture.py from real attn_q weight blocks of the model, read
by its tests/test_quant.cu).  Format: b"LKQF", u32 case count, then per case
u32 kind (0 = Q4_0, 1 = Q6_K), u32 nblocks, u32 nplanes, f32 reserved, the
planes (u32 size + bytes each: Q4_0 has qs [nblocks][16] and fp16 d
[nblocks]), u32 nx + f32 x[nx], f32 expected_exact, f32 expected_fp32.
Only the data is copied (weights, input, expected dot products).

Usage: python tests/golden/make_q4_0_fixture.py [path/to/quant_fixture.bin]
"""
import os
import struct
import sys

import numpy as np

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/ref/quant_fixture.bin"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q4_0_dot.npz")


def main():
    b = open(SRC, "rb").read()
    assert b[:4] == b"LKQF", "not a quantisation fixture"
    off = 4
    (n,) = struct.unpack_from("<I", b, off); off += 4
    arrays = {}
    k = 0
    for _ in range(n):
        kind, nblocks, nplanes, _res = struct.unpack_from("<IIIf", b, off); off += 16
        planes = []
        for _ in range(nplanes):
            (sz,) = struct.unpack_from("<I", b, off); off += 4
            planes.append(b[off:off + sz]); off += sz
        (nx,) = struct.unpack_from("<I", b, off); off += 4
        x = np.frombuffer(b, np.float32, nx, off).copy(); off += 4 * nx
        exact, fp32 = struct.unpack_from("<ff", b, off); off += 8
        if kind != 0:
            continue
        arrays[f"qs{k}"] = np.frombuffer(planes[0], np.uint8).reshape(nblocks, 16).copy()
        arrays[f"d{k}"] = np.frombuffer(planes[1], np.uint16).copy()
        arrays[f"x{k}"] = x
        arrays[f"expected{k}"] = np.array([exact, fp32], np.float32)
        k += 1
    assert off == len(b), "trailing bytes"
    arrays["n"] = np.array(k, np.int32)
    np.savez(OUT, **arrays)
    print(f"wrote {OUT}: {k} Q4_0 cases")


if __name__ == "__main__":
    main()
