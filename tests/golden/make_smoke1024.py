"""Regenerates the reference's 1024-node smoke graph (GATBIN1) in memory.

Restates implementation/tools/prepare_smoke.py:9-25: numpy default_rng(20260928),
N=1024, D=128, C=40, row i has degree degrees[i % 14] made of the self-loop
followed by degree-1 distinct random sources, features N(0, 0.5) as float32.
The committed fixture implementation/data/smoke1024.gatbin has SHA256
b3e93c7f57e14c132746d4113e3c59c528602f171d26525fe74bd48e32c8b9e3
(implementation/runs/implementation-smoke-F83Zo7Xy/artifact.sha256); the test
suite checks that these bytes hash to it.
"""
import hashlib
import struct

import numpy as np

SMOKE1024_SHA256 = "b3e93c7f57e14c132746d4113e3c59c528602f171d26525fe74bd48e32c8b9e3"


def smoke1024_bytes() -> bytes:
    rng = np.random.default_rng(20260928)
    n, d, c = 1024, 128, 40
    degrees = [1, 2, 7, 15, 16, 17, 31, 32, 33, 63, 64, 65, 96, 127]
    row = [0]
    col = []
    for i in range(n):
        deg = degrees[i % len(degrees)]
        nbr = rng.choice(n, size=deg - 1, replace=False).astype(np.uint32).tolist()
        col.extend([i] + nbr)
        row.append(len(col))
    x = rng.normal(0, 0.5, size=(n, d)).astype("<f4")
    head = struct.pack("<8sQQII", b"GATBIN1\0", n, len(col), d, c)
    return head + np.asarray(row, "<u8").tobytes() + np.asarray(col, "<u4").tobytes() + x.tobytes()


def smoke1024():
    """Returns dict(n, e, din, classes, row, col, x) parsed from the bytes."""
    b = smoke1024_bytes()
    n, e, din, classes = struct.unpack_from("<QQII", b, 8)
    off = 32
    row = np.frombuffer(b, "<u8", n + 1, off).copy()
    off += 8 * (n + 1)
    col = np.frombuffer(b, "<u4", e, off).copy()
    off += 4 * e
    x = np.frombuffer(b, "<f4", n * din, off).reshape(n, din).copy()
    return dict(n=n, e=e, din=din, classes=classes, row=row, col=col, x=x)


if __name__ == "__main__":
    print(hashlib.sha256(smoke1024_bytes()).hexdigest() == SMOKE1024_SHA256)
