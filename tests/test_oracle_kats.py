"""The reference's unit known-answer tests, restated as data against the oracle.

Each test names the reference test it restates.  Together with the golden
fixtures these pin every oracle function used as a parity checker.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def ref_matrix(o, i):
    # qtensor.rs:593-598
    k = np.arange(o * i, dtype=np.float32)
    v = (np.sin(k * np.float32(0.7)) * np.float32(0.9)) + ((k % 7) - 3).astype(np.float32) * np.float32(0.01)
    return v.astype(np.float32).reshape(o, i)


# ---------------------------------------------------------------- kernels.rs
def test_unpack_covers_full_nibble_range():
    # kernels.rs:87-96: every code -8..7 round-trips through both nibbles
    for v in range(-8, 8):
        nib = v & 0x0F
        row = np.array([nib, (nib << 4) & 0xFF], np.uint8)
        deq = O.dequantize(O.INT4, row, np.array([1.0], np.float32), 1, 4)
        assert deq[0, 0] == v and deq[0, 3] == v


def test_i4_matmul_handles_odd_tail():
    # kernels.rs:98-108: codes [2,-3,5], scale 0.5, x=[1,2,3] -> 5.5
    packed = np.array([(2 & 0xF) | (((-3) & 0xF) << 4), 5 & 0xF], np.uint8)
    out = O.matmul(O.INT4, packed, np.array([0.5], np.float32), 1, 3, np.array([1, 2, 3], np.float32))
    assert abs(out[0, 0] - 5.5) < 1e-6


def test_i8_matmul_hand_computed():
    # kernels.rs:110-120
    q = np.array([10, -20, 127, 1], np.int8)
    out = O.matmul(O.INT8, q, np.array([0.1, 0.01], np.float32), 2, 2, np.array([2, 3], np.float32))
    assert abs(out[0, 0] - np.float32(0.1) * -40) < 1e-6
    assert abs(out[0, 1] - np.float32(0.01) * 257) < 1e-6


# -------------------------------------------------------------------- lib.rs
def test_f32_matmul_identity_and_hand_computed():
    # lib.rs:151-167
    w = np.eye(3, dtype=np.float32)
    assert O.matmul(O.F32, w, None, 3, 3, np.array([1, 2, 3], np.float32)).tolist() == [[1, 2, 3]]
    w = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    x = np.array([[1, 1, 1], [0, 1, 2]], np.float32)
    assert O.matmul(O.F32, w, None, 2, 3, x).reshape(-1).tolist() == [6, 15, 8, 17]


def test_rmsnorm_unit_weight():
    # lib.rs:169-178
    out = O.rmsnorm(np.array([3, 4], np.float32), np.ones(2, np.float32), 0.0)
    r = math.sqrt(12.5)
    assert abs(out[0] - 3 / r) < 1e-6 and abs(out[1] - 4 / r) < 1e-6


def test_rmsnorm_accumulates_in_f64():
    # lib.rs:95: the mean of squares is an f64 sum.  1e8 and 1 differ by more
    # than f32 can add exactly, so an f32 accumulator would lose the 1.
    x = np.array([1e4, 1.0, 1.0, 1.0], np.float32)
    ms = (1e8 + 3.0) / 4.0
    r = np.float32(1.0) / np.sqrt(np.float32(ms) + np.float32(1e-6))
    want = x * r
    assert np.array_equal(O.rmsnorm(x, np.ones(4, np.float32), 1e-6), want.astype(np.float32))


def test_softmax_sums_to_one():
    # lib.rs:180-186
    p = O.softmax(np.array([1, 2, 3, 4], np.float32))
    assert abs(p.sum() - 1) < 1e-6 and p[3] > p[2] > p[1] > p[0]


# ---------------------------------------------------------------- qtensor.rs
@pytest.mark.parametrize("fmt,o,i,qmax", [(O.INT8, 8, 33, 127), (O.INT4, 5, 17, 7)])
def test_roundtrip_error_bound(fmt, o, i, qmax):
    # qtensor.rs:600-634
    w = ref_matrix(o, i)
    q, s = O.quantize(w, fmt)
    back = O.dequantize(fmt, q, s, o, i)
    half = np.abs(w).max(1, keepdims=True) / qmax / 2 + 1e-9
    assert (np.abs(w - back) <= half * 1.01).all()


def test_quantized_matmul_matches_dequant_reference():
    # qtensor.rs:636-656
    o, i, s = 6, 21, 3
    w = ref_matrix(o, i)
    x = np.cos(np.arange(s * i, dtype=np.float32) * np.float32(0.31)).reshape(s, i)
    for fmt in (O.INT8, O.INT4):
        q, sc = O.quantize(w, fmt)
        deq = O.dequantize(fmt, q, sc, o, i)
        expect = O.matmul(O.F32, deq, None, o, i, x)
        got = O.matmul(fmt, q, sc, o, i, x)
        assert (np.abs(got - expect) <= 1e-4 * np.maximum(np.abs(expect), 1)).all()


def test_zero_rows_are_safe():
    # qtensor.rs:671-688
    o, i = 3, 8
    w = ref_matrix(o, i)
    w[1] = 0
    for fmt in (O.INT8, O.INT4):
        q, s = O.quantize(w, fmt)
        assert s[1] == 0
        assert (O.dequantize(fmt, q, s, o, i)[1] == 0).all()
        out = O.matmul(fmt, q, s, o, i, np.ones(i, np.float32))
        assert out[0, 1] == 0 and np.isfinite(out).all()


def test_non_finite_weights_rejected():
    # qtensor.rs:690-697
    w = ref_matrix(2, 4)
    w[1, 1] = np.nan
    with pytest.raises(ValueError):
        O.quantize(w, O.INT8)
    w[1, 1] = np.inf
    with pytest.raises(ValueError):
        O.quantize(w, O.INT4)


def test_row_ops_match_dequant():
    # qtensor.rs:711-741
    o, i = 7, 13
    w = ref_matrix(o, i)
    x = np.sin(np.arange(i, dtype=np.float32) * 3 * np.float32(0.17))
    for fmt in (O.F32, O.INT8, O.INT4):
        q, s = O.quantize(w, fmt)
        deq = O.dequantize(fmt, q, s, o, i)
        acc = O.add_scaled_row(fmt, q, s, o, i, 3, 2.5, np.zeros(i, np.float32))
        assert np.abs(acc - 2.5 * deq[3]).max() < 1e-5
        out = O.matvec_rows(fmt, q, s, o, i, 2, 4, x)
        e = deq[2:6] @ x
        assert np.abs(out - e).max() < 1e-4


def test_quantize_rounds_half_away_from_zero_and_clamps():
    # qtensor.rs:167-202: s = max/qmax; round() is half-away-from-zero
    w = np.array([[7.0, 3.5, -3.5, 0.5, -0.5, 2.5]], np.float32)
    q, s = O.quantize(w, O.INT4)
    assert s[0] == np.float32(1.0)
    codes = O.dequantize(O.INT4, q, s, 1, 6)[0]
    assert codes.tolist() == [7, 4, -4, 1, -1, 3]
    # nibble packing: even index in the low nibble
    assert q[0, 0] == ((7 & 0xF) | ((4 & 0xF) << 4))


def test_dequant_is_scale_times_code_bit_exact():
    # qtensor.rs:265-272 + 516-543: 0 + (1*scale)*q == fl(scale*q)
    rng = np.random.default_rng(3)
    w = rng.standard_normal((9, 31)).astype(np.float32)
    for fmt in (O.INT8, O.INT4):
        q, s = O.quantize(w, fmt)
        deq = O.dequantize(fmt, q, s, 9, 31)
        if fmt == O.INT8:
            codes = q.astype(np.float32)
        else:
            lo = (q & 0xF).astype(np.int8)
            hi = (q >> 4).astype(np.int8)
            lo = np.where(lo > 7, lo - 16, lo)
            hi = np.where(hi > 7, hi - 16, hi)
            codes = np.stack([lo, hi], -1).reshape(9, -1)[:, :31].astype(np.float32)
        assert np.array_equal(deq, (s[:, None] * codes).astype(np.float32))


# ------------------------------------------------------- deepseek router.rs
def _router(logits, bias=None, k=2, n_group=1, topk_group=1, norm=False, scale=1.0):
    ids, w = O.route(np.asarray(logits, np.float32), bias, k, n_group, topk_group, norm, scale)
    return ids.tolist(), w


def sig(x):
    return np.float32(1) / (np.float32(1) + np.exp(np.float32(-x), dtype=np.float32))


def test_router_picks_largest_logits_without_bias():
    ids, w = _router([0.1, 2.0, -1.0, 1.0], k=2)
    assert ids == [1, 3] and abs(w[0] - sig(2.0)) < 1e-7


def test_router_bias_changes_selection_but_not_weights():
    ids, w = _router([1.0, 0.0, 0.9], bias=np.array([0, 0, 0.5], np.float32), k=1)
    assert ids == [2] and abs(w[0] - sig(0.9)) < 1e-7


def test_router_norm_and_scale_applied():
    ids, w = _router([3.0, 2.0, -3.0, -3.0], k=2, norm=True, scale=2.5)
    s0, s1 = sig(3.0), sig(2.0)
    d = s0 + s1 + 1e-20
    assert abs(w[0] - 2.5 * s0 / d) < 1e-6 and abs(w[1] - 2.5 * s1 / d) < 1e-6


def test_router_group_limitation_masks_losing_groups():
    ids, _ = _router([2.0, 1.9, 3.0, -5.0, -1.0, -1.0, 2.0, 1.8], k=4, n_group=4, topk_group=2)
    assert ids == [0, 6, 1, 7]


# ---------------------------------------------------------- core router.rs
def test_topk_edge_cases():
    # core/router.rs:215-238
    assert O.topk_indices(np.zeros(0, np.float32), 5) == []
    assert O.topk_indices([1.0, 2.0, 3.0], 0) == []
    assert O.topk_indices([1.0, 5.0, 2.0, 5.0], 1) == [1]
    assert O.topk_indices([2.0, 3.0, 1.0], 10) == [1, 0, 2]
    assert O.topk_indices([-5.0, -1.0, -1.0, -3.0], 2) == [1, 2]


def _brute_topk(values, k):
    out = []
    for _ in range(min(k, len(values))):
        best = None
        for i, v in enumerate(values):
            if i in out:
                continue
            if best is None or not values[best] >= v:
                best = i
        out.append(best)
    return out


@pytest.mark.parametrize("k", [16, 80])
def test_topk_parity_with_brute_force(k):
    # core/router.rs:240-278: N=512 with many exact ties
    vals = [np.float32(((i * 37) % 50)) * np.float32(0.1) for i in range(512)]
    assert O.topk_indices(np.array(vals, np.float32), k) == _brute_topk(vals, k)


# ------------------------------------------------------------ sample.rs
def test_argmax_first_max_and_nan():
    # sample.rs:353-361, 368-371
    assert O.argmax([0.1, 3.0, -1.0, 2.9]) == 1
    assert O.argmax([1.0, 5.0, 5.0]) == 1
    assert O.argmax([np.nan, 5.0]) == 0  # v[0] NaN: no `>` compare succeeds
    assert O.argmax([1.0, np.nan, 2.0]) == 2


# --------------------------------------------------------- attention.rs
def test_rope_pos0_is_identity():
    # attention.rs:294-299: pairs move to split-half positions
    assert O.rope_interleave([1, 2, 3, 4], 0, 4, 10000.0).tolist() == [1, 3, 2, 4]


def test_rope_preserves_norm():
    v = np.array([0.3, -1.2, 2.0, 0.5, -0.7, 1.1], np.float32)
    r = O.rope_interleave(v, 17, 6, 10000.0)
    assert abs((v * v).sum() - (r * r).sum()) < 1e-4


def test_rope_relative_position_invariance():
    dim = 8
    q = np.sin(np.arange(dim, dtype=np.float32) * np.float32(0.7))
    k = np.cos(np.arange(dim, dtype=np.float32) * np.float32(1.3))

    def dot_at(pq, pk):
        return float((O.rope_interleave(q, pq, dim, 1e4) * O.rope_interleave(k, pk, dim, 1e4)).sum())

    assert abs(dot_at(0, 5) - dot_at(7, 12)) < 1e-4


def test_mla_attend_matches_numpy_float64():
    # closed form of attention.rs:214-234 evaluated in float64
    rng = np.random.default_rng(11)
    R, H, L, P, T = 2, 3, 16, 4, 9
    qabs = rng.standard_normal((R, H, L)).astype(np.float32)
    qr = rng.standard_normal((R, H, P)).astype(np.float32)
    lat = rng.standard_normal((T, L)).astype(np.float32)
    kr = rng.standard_normal((T, P)).astype(np.float32)
    pos_base = T - R
    got = O.mla_attend(qabs, qr, lat, kr, pos_base, 0.25)
    for s in range(R):
        n = pos_base + s + 1
        for h in range(H):
            sc = (lat[:n].astype(np.float64) @ qabs[s, h] + kr[:n].astype(np.float64) @ qr[s, h]) * 0.25
            p = np.exp(sc - sc.max())
            p /= p.sum()
            want = p @ lat[:n].astype(np.float64)
            assert np.abs(got[s, h] - want).max() < 1e-5


def test_moe_experts_matches_per_expert_matmuls():
    rng = np.random.default_rng(5)
    hidden, inter, E, M, k = 24, 10, 6, 3, 2
    for fmt in (O.INT8, O.INT4):
        gs, us, ds, gq, uq, dq = [], [], [], [], [], []
        for _ in range(E):
            for lst_q, lst_s, shape in ((gq, gs, (inter, hidden)), (uq, us, (inter, hidden)), (dq, ds, (hidden, inter))):
                q, s = O.quantize(rng.standard_normal(shape).astype(np.float32), fmt)
                lst_q.append(q.reshape(-1).view(np.uint8))
                lst_s.append(s)
        ids = np.array([[1, 4], [4, 0], [5, 1]], np.int64)
        w = rng.random((M, k)).astype(np.float32)
        x = rng.standard_normal((M, hidden)).astype(np.float32)
        got = O.moe_experts(fmt, hidden, inter, np.concatenate(gq), np.concatenate(gs),
                            np.concatenate(uq), np.concatenate(us), np.concatenate(dq),
                            np.concatenate(ds), ids, w, x)
        for s in range(M):
            acc = np.zeros(hidden, np.float32)
            for c in range(k):
                e = ids[s, c]
                g = O.matmul(fmt, gq[e], gs[e], inter, hidden, x[s])[0]
                u = O.matmul(fmt, uq[e], us[e], inter, hidden, x[s])[0]
                h = (g / (np.float32(1) + np.exp(-g, dtype=np.float32))) * u
                d = O.matmul(fmt, dq[e], ds[e], hidden, inter, h.astype(np.float32))[0]
                acc = (acc + w[s, c] * d).astype(np.float32)
            assert np.abs(got[s] - acc).max() <= 1e-5 * max(1.0, np.abs(acc).max())
