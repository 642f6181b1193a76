"""Writes the golden fixtures under tests/golden/ from closed forms.

Nothing here runs or imports the reference.  Every expected value is either a
published constant or exact integer arithmetic:

* splitmix64_kat.json -- the first outputs of SplitMix64 from state 0, as
  published with the generator (Steele, Lea and Flood, OOPSLA 2014; Vigna's
  public-domain splitmix64.c prints 0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4,
  0x06c45d188009454f for seed 0).
* reference_arange_cases.json -- the reference VM's full-kernel cases
  (/root/reference/test/test_vm.py:447-537 and :539-627): A = arange(m*k),
  B = arange(k*n) stored column-major, C = 1, alpha = beta = 1.  D is computed
  with Python integers, so it is exact.
* wgm_8x8_wgm4.json -- the work-group remap closed form of
  /root/reference/test/test_vm.py:734-737 on an 8 x 8 grid with wgm = 4.
* fill_vectors.json -- sample values of the seeded input generator at chosen
  indices, computed with Python integers and exact float arithmetic (uniform),
  so the C, numpy and shim implementations can be checked against data.

Run: python tests/golden/make_golden.py
"""
import json
import math
import os
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
M64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15


def mix64(z):
    z &= M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def word_at(key, i):
    return mix64(key + (i + 1) * GAMMA)


def stream_key(seed, mid):
    return mix64(seed ^ ((0xD1B54A32D192ED03 * (mid + 1)) & M64))


def uniform(seed, mid, i):
    w = word_at(stream_key(seed, mid), i)
    u = (w >> 40) / float(1 << 24)  # exact in binary64 and binary32
    v = u * 2.0 - 1.0               # exact: a multiple of 2^-23 in [-1, 1)
    assert struct.unpack("f", struct.pack("f", v))[0] == v
    return v


def arange_case(m, n, k):
    A = [[float(i + l * m) for l in range(k)] for i in range(m)]     # column-major arange
    B = [[float(l + j * k) for j in range(n)] for l in range(k)]
    D = [[int(sum(int(A[i][l]) * int(B[l][j]) for l in range(k))) + 1 for j in range(n)] for i in range(m)]
    # store D column-major as a flat list
    return [D[i][j] for j in range(n) for i in range(m)]


def main():
    with open(os.path.join(HERE, "splitmix64_kat.json"), "w") as f:
        json.dump({"state": 0, "outputs_hex": ["0xe220a8397b1dcdaf", "0x6e789e6aa1b965f4", "0x06c45d188009454f"]},
                  f, indent=1)
    cases = []
    for atom, (m, n, k) in (("16x16x4", (16, 16, 64)), ("32x32x2", (32, 32, 64))):
        cases.append({"atom": atom, "m": m, "n": n, "k": k, "alpha": 1.0, "beta": 1.0, "c": 1.0,
                      "d_colmajor": arange_case(m, n, k)})
    with open(os.path.join(HERE, "reference_arange_cases.json"), "w") as f:
        json.dump(cases, f)
    table = []
    for wy in range(8):
        for wx in range(8):
            z = wx + wy * 8
            table.append([wx, wy, (z % 4) + (z // 4 // 8) * 4, (z // 4) % 8])
    with open(os.path.join(HERE, "wgm_8x8_wgm4.json"), "w") as f:
        json.dump({"nwgx": 8, "nwgy": 8, "wgm": 4, "map": table}, f)
    vectors = []
    for seed, mid in ((0, 0), (1, 1), (2, 0), (2, 1), (3, 2), (4, 0)):
        idx = [0, 1, 2, 3, 63, 64, 1000, 4095, 4096, 16777215, 16777216, 67108863]
        vectors.append({"seed": seed, "matrix_id": mid, "dist": 0, "index": idx,
                        "value": [uniform(seed, mid, i) for i in idx],
                        "word_hex": [hex(word_at(stream_key(seed, mid), i)) for i in idx]})
    with open(os.path.join(HERE, "fill_vectors.json"), "w") as f:
        json.dump(vectors, f, indent=1)
    print("golden fixtures written")


if __name__ == "__main__":
    main()
