"""Random GGUF blocks for formats the reference ships no quantizer for
(Q5_0, Q4_1, Q3_K): random qs/qh/hmask/scale bytes (every bit pattern) with
f16 scales of magnitude dmax/32..dmax of both signs, and for Q4_1 mins in
(-2 dmax, 2 dmax).  Q3_K's super-block scale d sits at bytes 108..109."""
import numpy as np

import oracle as O


def rand_blocks(rng, dt, n, k, dmax=2.0 ** -4):
    if dt == O.Q3_K:
        nsb = k // 256
        b = rng.integers(0, 256, size=(n * nsb, 110), dtype=np.uint8)
        d = (rng.uniform(dmax / 32, dmax, n * nsb) * rng.choice([-1.0, 1.0], n * nsb)).astype(np.float16)
        b[:, 108:110] = d.view(np.uint8).reshape(-1, 2)
        return b.reshape(-1)
    nb = k // 32
    bb = O.BLOCK[dt][1]
    b = rng.integers(0, 256, size=(n * nb, bb), dtype=np.uint8)
    d = (rng.uniform(dmax / 32, dmax, n * nb) * rng.choice([-1.0, 1.0], n * nb)).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    if dt == O.Q4_1:
        m = rng.uniform(-2 * dmax, 2 * dmax, n * nb).astype(np.float16)
        b[:, 2:4] = m.view(np.uint8).reshape(-1, 2)
    return b.reshape(-1)


def float_bytes(rng, dt, n, k, sigma=0.05):
    """F32 / F16 / BF16 weight bytes of N(0, sigma^2) values (bf16 by
    truncating the f32 bits)."""
    w = (rng.standard_normal((n, k)) * sigma).astype(np.float32)
    if dt == O.F32:
        return w.view(np.uint8).reshape(-1)
    if dt == O.F16:
        return w.astype(np.float16).view(np.uint8).reshape(-1)
    return (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)


def rand_ternary(rng, dt, n, k, dmax=2.0 ** -4):
    """Random Q1_0 / Q2_0 / STQ1_0 blocks (random code bytes, f16 scale of
    dmax/32..dmax), or an I2_S tensor (random codes, then one f32 scale)."""
    if dt == O.I2_S:
        b = rng.integers(0, 256, size=n * k // 4 + 4, dtype=np.uint8)
        b[-4:] = np.frombuffer(np.float32(rng.uniform(dmax / 32, dmax)).tobytes(), np.uint8)
        return b
    qk, bb = O.BLOCK[dt]
    nb = n * (k // qk)
    b = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    d = rng.uniform(dmax / 32, dmax, nb).astype(np.float16).view(np.uint8).reshape(-1, 2)
    if dt == O.STQ1_0:
        b[:, 40:42] = d
    else:
        b[:, 0:2] = d
    return b.reshape(-1)
