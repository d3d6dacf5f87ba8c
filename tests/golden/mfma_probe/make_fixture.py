"""Probe of v_mfma_f32_32x32x16_f16's arithmetic and the fixture made from it.

Step 1 (here, no GPU): write the test vectors.
    python tests/golden/mfma_probe/make_fixture.py vectors VEC.bin
Step 2 (on an MI355X): run the probe (probe.cpp: one test per wave, every
row of A equal to a, every column of B equal to b and every element of C
equal to c, so each output is c + sum_k a_k b_k as the matrix core computes
it; it also checks that all 16 outputs of a lane agree).
    hipcc --offload-arch=gfx950 -O2 probe.cpp -o probe && ./probe VEC.bin OUT.bin
Step 3 (here): keep a sample of the cases with the GPU's outputs.
    python tests/golden/mfma_probe/make_fixture.py fixture VEC.bin OUT.bin

The vectors, 165,761 cases (the fixture keeps 6,693 of them):
  kind 0  ordinary: a, b ~ U[-1, 1), c ~ U[-2, 2)
  kind 1  cancelling: c = -(a . b) (1 + U[-1e-3, 1e-3)) + U[-1e-4, 1e-4)
  kind 2  wide exponents: a, b, c = +-2^U(...) over 19 / 40 binades
  kind 3  c in {+-1, 1.5, 3, 0.75} plus products near its half-ulp
  kind 4  c = 0, cancelling products of mixed exponents
  kind 5  structured: +2^30 / 1 / -2^30 placed at every position triple;
          c = 2^30 or 1 against them; 2^30 + v and c = 2^30 + v for v
          around the FP32 ulp of 2^30 (which terms are summed together,
          the rounding of each step)
  kind 6  zero operands (+0, -0 in a or b) beside a product with bits below
          the frame a zero's exponent would set, and an accumulator with low
          bits against zero products only
"""

import json
import pathlib
import struct
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
FIXTURE = HERE.parent / "mfma_32x32x16_f16.npz"


def vectors():
    rng = np.random.default_rng(7)
    A, B, C, K = [], [], [], []

    def add(a, b, c, kind):
        A.append(np.asarray(a, np.float16))
        B.append(np.asarray(b, np.float16))
        C.append(np.float32(c))
        K.append(kind)

    n = 30000
    for _ in range(n):
        add(rng.uniform(-1, 1, 16), rng.uniform(-1, 1, 16), rng.uniform(-2, 2), 0)
    for _ in range(n):
        a, b = rng.uniform(-1, 1, 16), rng.uniform(-1, 1, 16)
        s = float(np.dot(a.astype(np.float16).astype(np.float64), b.astype(np.float16).astype(np.float64)))
        add(a, b, -s * (1 + rng.uniform(-1e-3, 1e-3)) + rng.uniform(-1e-4, 1e-4), 1)
    for _ in range(n):
        a = rng.choice([-1, 1], 16) * 2.0 ** rng.uniform(-12, 7, 16)
        b = rng.choice([-1, 1], 16) * 2.0 ** rng.uniform(-12, 7, 16)
        add(a, b, rng.choice([-1, 1]) * 2.0 ** rng.uniform(-20, 20), 2)
    for _ in range(n):
        e = rng.integers(-30, -20, 16)
        a = rng.choice([-1, 1], 16) * 2.0 ** (e // 2) * rng.uniform(1, 2, 16)
        b = 2.0 ** (e - e // 2) * rng.uniform(1, 2, 16)
        add(a, b, rng.choice([1.0, -1.0, 1.5, 3.0, 0.75]), 3)
    for _ in range(n):
        add(rng.choice([-1, 1], 16) * 2.0 ** rng.uniform(-6, 6, 16), np.abs(rng.uniform(0.5, 1, 16)), 0.0, 4)

    def placed(pairs, c, kind):
        a, b = np.zeros(16), np.zeros(16)
        for k, (x, y) in pairs.items():
            a[k], b[k] = x, y
        add(a, b, c, kind)

    big, nbig, one = (2.0 ** 15, 2.0 ** 15), (-2.0 ** 15, 2.0 ** 15), (1.0, 1.0)
    for i in range(16):
        for j in range(16):
            for k in range(16):
                if len({i, j, k}) == 3:
                    placed({i: big, j: one, k: nbig}, 0.0, 5)
    for j in range(16):
        for k in range(16):
            if j != k:
                placed({j: one, k: nbig}, 2.0 ** 30, 5)
                placed({j: big, k: nbig}, 1.0, 5)
    for v in (1, 16, 32, 48, 63, 64, 65, 96, 127, 128, 129, 160, 192, 200, 255, 256, 320, 384, 448):
        for i in range(16):
            for j in range(16):
                if i != j:
                    placed({i: big, j: (float(v), 1.0)}, 0.0, 5)
                    placed({i: big, j: (-float(v), 1.0)}, 0.0, 5)
        for j in range(16):
            placed({j: (float(v), 1.0)}, 2.0 ** 30, 5)
            placed({j: (-float(v), 1.0)}, 2.0 ** 30, 5)
    small = (2.0 ** -10 * (1 + 2.0 ** -10), 2.0 ** -10)  # 2^-20 + 2^-30
    for z in range(16):
        for s in range(16):
            if z != s:
                for partner in (2.0 ** 15, 2.0 ** 5, 1.0):
                    placed({z: (0.0, partner), s: small}, 0.0, 6)
                    placed({z: (-0.0, partner), s: small}, 0.0, 6)
                    placed({z: (partner, 0.0), s: small}, 0.0, 6)
    low = np.float32(2.0 ** -20 * (1.5 + 2.0 ** -20))
    for z in range(16):
        placed({z: (0.0, 2.0 ** 15)}, low, 6)
        placed({z: (2.0 ** 15, 0.0)}, low, 6)
    placed({}, low, 6)
    return (np.stack(A).view(np.uint16), np.stack(B).view(np.uint16), np.array(C, np.float32),
            np.array(K, np.int8))


def write_vectors(path):
    a, b, c, k = vectors()
    with open(path, "wb") as f:
        f.write(struct.pack("<i", len(c)))
        f.write(a.tobytes())
        f.write(b.tobytes())
        f.write(c.tobytes())
    print(f"{len(c)} cases -> {path}")


def write_fixture(vec_path, out_path):
    a, b, c, k = vectors()
    raw = pathlib.Path(vec_path).read_bytes()
    n = struct.unpack("<i", raw[:4])[0]
    assert n == len(c) and np.array_equal(np.frombuffer(raw, np.uint16, 16 * n, 4).reshape(n, 16), a)
    d = np.fromfile(out_path, np.float32)
    assert d.shape == (n,)
    rng = np.random.default_rng(1)
    keep = []
    for kind, count in ((0, 500), (1, 500), (2, 500), (3, 500), (4, 500), (5, 2000), (6, None)):
        idx = np.flatnonzero(k == kind)
        keep.append(idx if count is None else np.sort(rng.choice(idx, count, replace=False)))
    keep = np.concatenate(keep)
    np.savez_compressed(FIXTURE, a=a[keep], b=b[keep], c=c[keep], d=d[keep], kind=k[keep])
    print(f"{len(keep)} cases -> {FIXTURE}")


if __name__ == "__main__":
    if sys.argv[1:2] == ["vectors"]:
        write_vectors(sys.argv[2])
    elif sys.argv[1:2] == ["fixture"]:
        write_fixture(sys.argv[2], sys.argv[3])
    else:
        sys.exit(__doc__)
