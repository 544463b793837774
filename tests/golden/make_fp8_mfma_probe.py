"""Writes ``fp8_mfma_probe.npz``: e4m3 dot products as the f8f6f4 MFMA forms them.

Run on a machine with an MI355X, from the repository root:

    hipcc --offload-arch=gfx950 -O2 -Xclang -target-feature -Xclang -packed-fp32-ops \
        tests/golden/fp8_mfma_probe.hip -o /tmp/fp8_mfma_probe
    python tests/golden/make_fp8_mfma_probe.py /tmp/fp8_mfma_probe [output.npz]

Inputs (seeded): 16-row x 16-column cases of 128 e4m3 codes per row / column --
codes uniform over the finite values (products spanning 2^-18 .. 2^17), one
dominant product per row among small ones, codes from a narrow exponent band,
two nonzero products per row, and one large product followed by runs of small
equal ones. The fixture holds the codes (``a``, ``b``: [case, 16, 128] uint8) and
the MFMA's results (``d``: [case, 16, 16] float32, d[r][c] = a[r] . b[c]).
"""

import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def cases(seed=0):
    rng = np.random.default_rng(seed)
    finite = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)
    small = finite[(finite & 0x7F) < 0x20]
    large = finite[(finite & 0x7F) > 0x70]
    out = []
    for _ in range(16):  # uniform codes
        out.append((rng.choice(finite, (16, 128)), rng.choice(finite, (16, 128))))
    for _ in range(10):  # one dominant product per row
        a, b = rng.choice(small, (16, 128)), rng.choice(small, (16, 128))
        for r in range(16):
            k = rng.integers(0, 128)
            a[r, k] = rng.choice(large)
            b[r, k] = rng.choice(large)
        out.append((a, b))
    for _ in range(2):  # narrow exponent band
        lo = rng.integers(0x30, 0x50)
        band = finite[((finite & 0x7F) >= lo) & ((finite & 0x7F) < lo + 16)]
        out.append((rng.choice(band, (16, 128)), rng.choice(band, (16, 128))))
    for _ in range(8):  # two products per row
        a = np.zeros((16, 128), np.uint8)
        for r in range(16):
            k1, k2 = rng.integers(0, 128, 2)
            a[r, k1], a[r, k2] = rng.choice(finite), rng.choice(finite)
        out.append((a, rng.choice(finite, (16, 128))))
    for _ in range(4):  # a large product, then 8 r equal small ones in row r
        a = np.zeros((16, 128), np.uint8)
        b = np.full((16, 128), 0x38, np.uint8)  # 1.0
        big, sm = rng.choice(large), rng.choice(finite[(finite & 0x7F) < 0x40])
        for r in range(16):
            a[r, 0] = big
            a[r, 1:1 + 8 * r] = sm
        b[:, 0] = rng.choice(large, 16)
        out.append((a, b))
    a = np.stack([c[0] for c in out]).astype(np.uint8)
    b = np.stack([c[1] for c in out]).astype(np.uint8)
    return a, b


def main(probe_bin, out_path=None):
    a, b = cases()
    n = a.shape[0]
    with tempfile.TemporaryDirectory() as tmp:
        src, dst = os.path.join(tmp, "in.dat"), os.path.join(tmp, "out.dat")
        with open(src, "wb") as f:
            f.write(np.int32(n).tobytes())
            f.write(a.tobytes())
            f.write(b.tobytes())
        subprocess.run([probe_bin, src, dst], check=True)
        d = np.fromfile(dst, np.float32).reshape(n, 16, 16)
    np.savez_compressed(out_path or os.path.join(HERE, "fp8_mfma_probe.npz"), a=a, b=b, d=d)
    print(f"wrote {n} cases")


if __name__ == "__main__":
    main(*sys.argv[1:3])
