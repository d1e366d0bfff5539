"""Seeded synthetic inputs with the distributions of BASELINE.json's configs:
int8 W uniform in [-127, 127], fp32 per-row scales uniform in [1e-3, 2e-2],
bf16 x ~ N(0, 1) (round to nearest even), RMSNorm gains ~ 1 + 0.1 N(0, 1)."""
import numpy as np


def bf16(x):
    a = np.asarray(x, dtype=np.float32)
    u = np.ascontiguousarray(a).reshape(-1).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).reshape(a.shape)
    return r[()] if a.ndim == 0 else r


def f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def weights(rng, out_f, in_f):
    return rng.integers(-127, 128, size=(out_f, in_f), dtype=np.int8)


def scales(rng, n):
    return rng.uniform(1e-3, 2e-2, size=n).astype(np.float32)


def activations(rng, *shape):
    return bf16(rng.standard_normal(shape).astype(np.float32))


def gains(rng, n):
    return bf16(1.0 + 0.1 * rng.standard_normal(n).astype(np.float32))
