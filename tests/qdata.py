"""Seeded generators of valid GGUF weight blocks for the parity tests.

Every byte pattern of these formats is a valid block once its f16 scale fields are finite,
so the weights are uniform random payload bytes with scale fields drawn at the magnitudes
an N(0, 0.02) tensor quantizes to.  Activations are N(0, 1) f32.
"""
import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K, ACT_Q8 = 0, 1, 2, 8, 12, 14, 15, 100
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


def f16_bytes(vals):
    return np.asarray(vals, np.float16).view(np.uint8).reshape(-1, 2)


def rand_weights(quant, rows, k, seed, full_range=False):
    """rows x k weights in `quant`, as a flat uint8 array (GGUF row-major)."""
    rng = np.random.default_rng(seed)
    be, bb = BLOCK[quant]
    nb = rows * (k // be)
    b = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if quant == Q8_0:
        b[:, 0:2] = f16_bytes(rng.uniform(2e-4, 6e-4, nb))
        lo = -128 if full_range else -127
        b[:, 2:] = rng.integers(lo, 128, size=(nb, 32)).astype(np.int8).view(np.uint8)
    elif quant == Q4_0:
        b[:, 0:2] = f16_bytes(rng.uniform(2e-3, 8e-3, nb))
    elif quant == Q4_K:
        b[:, 0:2] = f16_bytes(rng.uniform(1e-4, 4e-4, nb))
        b[:, 2:4] = f16_bytes(rng.uniform(5e-4, 2e-3, nb))
    elif quant == Q6_K:
        if not full_range:
            b[:, 192:208] = rng.integers(-64, 64, size=(nb, 16)).astype(np.int8).view(np.uint8)
        b[:, 208:210] = f16_bytes(rng.uniform(1e-4, 3e-4, nb))
    return b.reshape(-1)


def rand_act(k, seed, m=None):
    rng = np.random.default_rng(seed)
    shape = (k,) if m is None else (m, k)
    return rng.standard_normal(shape).astype(np.float32)


def row_bytes(quant, k):
    be, bb = BLOCK[quant]
    return (k // be) * bb


BF16 = 30
FLOAT_BYTES = {F32: 4, F16: 2, BF16: 2}


def rand_float_weights(quant, rows, k, seed, scale=0.02):
    """rows x k N(0, scale) weights stored as F32, F16 or BF16 (rounded to nearest even), as a flat
    uint8 array."""
    rng = np.random.default_rng(seed)
    w = (scale * rng.standard_normal((rows, k))).astype(np.float32)
    if quant == F32:
        return w.view(np.uint8).reshape(-1)
    if quant == F16:
        return w.astype(np.float16).view(np.uint8).reshape(-1)
    b = w.view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16  # round to nearest even on the upper 16 bits
    return b.astype(np.uint16).view(np.uint8).reshape(-1)


def float_values(quant, data, rows, k):
    """The f32 values of rand_float_weights' bytes."""
    data = np.ascontiguousarray(data, np.uint8)
    if quant == F32:
        return data.view(np.float32).reshape(rows, k)
    if quant == F16:
        return data.view(np.float16).astype(np.float32).reshape(rows, k)
    return (data.view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(rows, k)
