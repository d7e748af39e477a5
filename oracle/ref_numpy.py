"""Independent vectorised numpy restatement of the block formats (second oracle).

TEST INFRASTRUCTURE ONLY.  It exists so that oracle.c is checked against a second,
independently written reading of the public GGUF/ggml layouts (closed forms):
a transposed index or a dropped term in either one shows up as a mismatch.

Block layouts (little endian):
  Q8_0   34 B : f16 d | i8 q[32]                      y = d q
  Q4_0   18 B : f16 d | u8 qs[16]                     y[j] = d (lo - 8), y[j+16] = d (hi - 8)
  Q4_K  144 B : f16 d | f16 dmin | u8 sc[12] | u8 qs[128]
  Q6_K  210 B : u8 ql[128] | u8 qh[64] | i8 sc[16] | f16 d
  Q8_K  292 B : f32 d | i8 q[256] | i16 bsums[16]
  ACT_Q8 36 B : f32 d | i8 q[32]      (the reference's Q8 activation block, pinned by the
                                       golden llama fixture: the scale stays f32)
"""
import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K, ACT_Q8 = 0, 1, 2, 8, 12, 14, 15, 100
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), ACT_Q8: (32, 36), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}


def _f16(b2):
    return b2.copy().view(np.float16).astype(np.float32).reshape(b2.shape[:-1])


def _f32(b4):
    return b4.copy().view(np.float32).reshape(b4.shape[:-1])


def blocks(quant, data, rows, k):
    be, bb = BLOCK[quant]
    return np.ascontiguousarray(data, dtype=np.uint8).reshape(rows, k // be, bb)


def q4k_scales(sc):
    """sc: [..., 12] uint8 -> (scale[..., 8], min[..., 8]) as int32."""
    sc = sc.astype(np.int32)
    s = np.empty(sc.shape[:-1] + (8,), np.int32)
    m = np.empty_like(s)
    s[..., :4] = sc[..., 0:4] & 63
    m[..., :4] = sc[..., 4:8] & 63
    s[..., 4:] = (sc[..., 8:12] & 0xF) | ((sc[..., 0:4] >> 6) << 4)
    m[..., 4:] = (sc[..., 8:12] >> 4) | ((sc[..., 4:8] >> 6) << 4)
    return s, m


def unpack_ints(quant, data, rows, k):
    """Integer weights per element plus per-group integer scales (for the int partial sums).
    Returns (q[rows, k] int32, group) where group is the partial-sum width."""
    b = blocks(quant, data, rows, k)
    if quant == Q8_0:
        return b[..., 2:].view(np.int8).astype(np.int32).reshape(rows, k), 32
    if quant == Q4_0:
        qs = b[..., 2:].astype(np.int32)
        q = np.concatenate([(qs & 0xF) - 8, (qs >> 4) - 8], axis=-1)
        return q.reshape(rows, k), 32
    if quant == Q4_K:
        qs = b[..., 16:].astype(np.int32).reshape(rows, k // 256, 4, 32)
        q = np.stack([qs & 0xF, qs >> 4], axis=3)  # [r, b, i, lo/hi, 32] -> element 64i + 32h + l
        return q.reshape(rows, k), 32
    if quant == Q6_K:
        ql = b[..., :128].astype(np.int32).reshape(rows, k // 256, 2, 64)
        qh = b[..., 128:192].astype(np.int32).reshape(rows, k // 256, 2, 32)
        parts = [
            (ql[..., :32] & 0xF) | ((qh & 3) << 4),
            (ql[..., 32:] & 0xF) | (((qh >> 2) & 3) << 4),
            (ql[..., :32] >> 4) | (((qh >> 4) & 3) << 4),
            (ql[..., 32:] >> 4) | (((qh >> 6) & 3) << 4),
        ]
        q = np.stack(parts, axis=3) - 32  # [r, b, half, part, 32] -> element 128n + 32p + l
        return q.reshape(rows, k), 16
    raise ValueError(quant)


def dequantize(quant, data, rows, k):
    if quant == F32:
        return np.frombuffer(np.ascontiguousarray(data).tobytes(), np.float32).reshape(rows, k).copy()
    b = blocks(quant, data, rows, k)
    if quant in (Q8_0, Q4_0):
        q, _ = unpack_ints(quant, data, rows, k)
        return (q.reshape(rows, k // 32, 32) * _f16(b[..., 0:2])[..., None]).reshape(rows, k).astype(np.float32)
    if quant in (ACT_Q8, Q8_K):
        be = BLOCK[quant][0]
        q = b[..., 4:4 + be].view(np.int8).astype(np.float32)
        return (q * _f32(b[..., 0:4])[..., None]).reshape(rows, k)
    if quant == Q4_K:
        q, _ = unpack_ints(quant, data, rows, k)
        s, m = q4k_scales(b[..., 4:16])
        d = _f16(b[..., 0:2])[..., None]
        dm = _f16(b[..., 2:4])[..., None]
        q = q.reshape(rows, k // 256, 8, 32).astype(np.float32)
        y = (d * s)[..., None] * q - (dm * m)[..., None]
        return y.reshape(rows, k).astype(np.float32)
    if quant == Q6_K:
        q, _ = unpack_ints(quant, data, rows, k)
        sc = b[..., 192:208].view(np.int8).astype(np.float32)
        d = _f16(b[..., 208:210])[..., None]
        y = q.reshape(rows, k // 256, 16, 16) * (d * sc)[..., None]
        return y.reshape(rows, k).astype(np.float32)
    raise ValueError(quant)


def act_ints(act_quant, xq, k):
    b = blocks(act_quant, xq, 1, k)
    be = BLOCK[act_quant][0]
    return b[..., 4:4 + be].view(np.int8).astype(np.int64).reshape(k), _f32(b[..., 0:4]).reshape(-1)


def partials(quant, data, rows, k, act_quant, xq):
    """Exact int32 partial sums S[row, group] = sum over the group of q_w * q_x (Q6_K: q6-32)."""
    q, g = unpack_ints(quant, data, rows, k)
    a, _ = act_ints(act_quant, xq, k)
    return np.einsum("rgl,gl->rg", q.reshape(rows, k // g, g).astype(np.int64), a.reshape(k // g, g)).astype(np.int32)


def quantize_act_q8(x):
    """ACT_Q8 quantizer: per 32, f32 d = amax/127, q = rint(x * (1/d))."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    q = np.rint(x * inv[:, None]).astype(np.int8)
    out = np.empty((x.shape[0], 36), np.uint8)
    out[:, 0:4] = d.view(np.uint8).reshape(-1, 4)
    out[:, 4:] = q.view(np.uint8)
    return out.reshape(-1)


def quantize_q8_k(x):
    """Q8_K quantizer (ggml quantize_row_q8_K_ref)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 256)
    nb = x.shape[0]
    out = np.zeros((nb, 292), np.uint8)
    ax = np.abs(x)
    j = np.argmax(ax, axis=1)  # first index of the maximum magnitude
    mx = x[np.arange(nb), j]
    nz = ax[np.arange(nb), j] != 0
    with np.errstate(divide="ignore", invalid="ignore"):
        iscale = np.where(nz, np.float32(-127) / np.where(nz, mx, 1), 0).astype(np.float32)
    q = np.minimum(np.rint(iscale[:, None] * x), 127).astype(np.int8)
    q[~nz] = 0
    with np.errstate(divide="ignore"):
        d = np.where(nz, np.float32(1) / np.where(nz, iscale, 1), 0).astype(np.float32)
    bs = q.astype(np.int16).reshape(nb, 16, 16).sum(axis=2).astype(np.int16)
    out[:, 0:4] = d.view(np.uint8).reshape(-1, 4)
    out[:, 4:260] = q.view(np.uint8)
    out[:, 260:292] = bs.view(np.uint8).reshape(nb, 32)
    return out.reshape(-1)
