"""CPU checks of the integer identities the matrix-core expert kernels rely
on (undertow_amd/csrc/ut_gemv_mfma.h), each against the definition it must
reproduce rather than against a restatement of the kernel:

- nibble sign extension without carries, ((u ^ 8) + 120) ^ 128 per byte,
  equals unpack_i4 (undertow-quant/src/kernels.rs:10-19: ((nib << 4) as i8) >> 4);
- masking the low / high nibbles of a packed word gives the even / odd
  columns (low nibble = even column, qtensor.rs:1-12);
- three balanced base-256 digits, taken from x~ + 0x808080 with each byte's
  top bit flipped, sum back to x~ for every |x~| <= 2^22;
- one 16-row x 128-column step with the operands in the permuted column
  order gives the exact integer sums of the natural order.
"""
import numpy as np


def unpack_i4(nib):
    v = (np.asarray(nib, np.int64) << 4) & 0xFF
    return np.where(v >= 128, v - 256, v) >> 4


def sext_bytes(t):
    """The kernel's per-word formula, bytes as int8 (t: uint32 array)."""
    t = np.asarray(t, np.uint64)
    w = (((t & 0x0F0F0F0F) + 0x78787878) ^ 0x80808080) & 0xFFFFFFFF
    b = np.stack([(w >> (8 * i)) & 0xFF for i in range(4)], -1).astype(np.int64)
    return np.where(b >= 128, b - 256, b)


def test_nibble_sign_extension_matches_unpack_i4():
    u = np.arange(16, dtype=np.uint64)
    word = u | (u << 8) | (u << 16) | (u << 24)
    got = sext_bytes(word ^ 0x08080808)
    assert (got == unpack_i4(u)[:, None]).all()


def test_low_high_nibbles_are_even_odd_columns():
    rng = np.random.default_rng(1)
    w = rng.integers(0, 2**32, 1000, dtype=np.uint64)
    cols = np.stack([(w >> (4 * j)) & 0xF for j in range(8)], -1)  # column j = nibble j
    t = w ^ 0x88888888
    lo, hi = sext_bytes(t), sext_bytes(t >> 4)
    assert (lo == unpack_i4(cols[:, 0::2])).all()
    assert (hi == unpack_i4(cols[:, 1::2])).all()


def base256_digits(xt):
    u = (np.asarray(xt, np.int64) + 0x808080) & 0xFFFFFFFF
    d = np.stack([(u >> (8 * p)) & 0xFF for p in range(3)], -1) ^ 0x80
    return np.where(d >= 128, d - 256, d)


def test_base256_digits_reconstruct():
    rng = np.random.default_rng(2)
    xt = np.concatenate([rng.integers(-2**22, 2**22 + 1, 100000),
                         [-2**22, 2**22, 0, -1, 1, 127, 128, -128, -129, 0x7FFF, -0x8000]])
    d = base256_digits(xt)
    assert d.min() >= -128 and d.max() <= 127
    assert (d[:, 0] + 256 * d[:, 1] + 65536 * d[:, 2] == xt).all()


def test_permuted_step_gives_exact_sums():
    """16 weight rows x 128 columns, M = 4 activation rows: A (per lane group
    kg, 32 columns as two 16-byte operands in the even/odd order) times B
    (the staged digit planes in the same order) summed over planes equals
    sum_k q[row, k] * x~[m, k] exactly."""
    rng = np.random.default_rng(3)
    R, K, M = 16, 128, 4
    packed = rng.integers(0, 256, (R, K // 2), dtype=np.uint64)
    nib = np.stack([packed & 0xF, packed >> 4], -1).reshape(R, K)  # column k
    q = unpack_i4(nib)
    xt = rng.integers(-2**22, 2**22 + 1, (M, K))
    want = q @ xt.T  # [R, M]
    # staged order: per 8-column group the even columns, then the odd ones
    perm = np.concatenate([g * 8 + np.array([0, 2, 4, 6, 1, 3, 5, 7]) for g in range(K // 8)])
    dig = base256_digits(xt)  # [M, K, 3]
    B = dig[:, perm, :]       # staged bytes, position -> column perm[pos]
    # A bytes of each row in the kernel's operand order
    words = packed.reshape(R, K // 8, 4)
    words = words[..., 0] | (words[..., 1] << 8) | (words[..., 2] << 16) | (words[..., 3] << 24)
    t = words ^ 0x88888888
    lo, hi = sext_bytes(t), sext_bytes(t >> 4)  # [R, K/8, 4]
    A = np.concatenate([lo, hi], -1).reshape(R, K)  # position order
    C = np.einsum("rk,mkp->rmp", A, B)
    got = C[..., 0] + 256 * C[..., 1] + 65536 * C[..., 2]
    assert (got == want).all()
