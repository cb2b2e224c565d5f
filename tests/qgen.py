"""Synthetic quantized weights and the closed form of the GPU's GEMV arithmetic.

The GPU kernels represent an activation row x exactly as integers,
    x~ = rint(x * 2^(22-E)),  max|x| = f * 2^E with f in [0.5, 1),
accumulate S = sum_k x~_k q_k exactly, and return fl(fl(S * 2^(E-22)) * scale).
``gemv_closed_form`` evaluates that definition in int64 / float64 numpy, so a
GPU result can be checked bit for bit (independently of the reference's own
rounding, which the oracle comparison covers).
"""
import numpy as np

F32, INT8, INT4 = 0, 1, 2


def rand_qtensor(rng, fmt, o, i, std=0.02):
    """BASELINE config-2 distributions: uniform codes, scales |N(0,std)|/qmax."""
    if fmt == INT4:
        payload = rng.integers(0, 256, size=(o, (i + 1) // 2), dtype=np.uint8)
        scales = (np.abs(rng.normal(0, std, o)) / 7).astype(np.float32)
    elif fmt == INT8:
        payload = rng.integers(-127, 128, size=(o, i), dtype=np.int8)
        scales = (np.abs(rng.normal(0, std, o)) / 127).astype(np.float32)
    else:
        payload = rng.normal(0, std, (o, i)).astype(np.float32)
        scales = None
    return payload, scales


def codes(fmt, payload, o, i):
    """Integer codes [o, i] (int4: two's-complement nibbles, low nibble = even index)."""
    if fmt == INT8:
        return np.asarray(payload, np.int8).reshape(o, i).astype(np.int64)
    p = np.asarray(payload, np.uint8).reshape(o, -1)
    lo = (p & 0xF).astype(np.int64)
    hi = (p >> 4).astype(np.int64)
    nib = np.stack([lo, hi], -1).reshape(o, -1)[:, :i]
    return np.where(nib > 7, nib - 16, nib)


def digitize(x):
    """(x~ int64 [M,K], e int per row) as the GPU's activation digitisation."""
    x = np.asarray(x, np.float32)
    xt = np.zeros(x.shape, np.int64)
    es = []
    for m in range(x.shape[0]):
        mx = np.float32(np.abs(x[m]).max()) if x.shape[1] else np.float32(0)
        E = 0 if mx == 0 else int(np.frexp(mx)[1])
        xt[m] = np.rint(np.ldexp(x[m].astype(np.float64), 22 - E)).astype(np.int64)
        es.append(E - 22)
    return xt, es


def gemv_closed_form(fmt, payload, scales, o, i, x):
    x = np.asarray(x, np.float32).reshape(-1, i)
    if fmt == F32:
        raise ValueError("f32 weights have no closed form here")
    q = codes(fmt, payload, o, i)
    xt, es = digitize(x)
    out = np.zeros((x.shape[0], o), np.float32)
    for m in range(x.shape[0]):
        S = q @ xt[m]  # exact int64
        v = np.ldexp(S.astype(np.float64), es[m]).astype(np.float32)
        out[m] = (v * scales).astype(np.float32)
    return out
