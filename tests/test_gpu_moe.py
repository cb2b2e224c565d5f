"""Router top-k, routed-expert block, argmax and MLA attention on the GPU vs the oracle.

Bars: top-k indices and argmax bit-exact whenever the
top-2 gap exceeds 1e-3; expert outputs within 1e-4 * max(|oracle|, 1)
(the reference's SIMD-vs-scalar bound, avx512.rs:335-366); attention within
1e-5 of the oracle's sequential f32 loops.
"""
import numpy as np
import pytest

from conftest import dev, host
from oracle import oracle as O
from qgen import F32, INT4, INT8, rand_qtensor

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ router
@pytest.mark.parametrize("E,k,ng,tg", [(256, 8, 8, 4), (8, 2, 4, 2), (16, 4, 4, 2), (64, 6, 1, 1),
                                       (8, 2, 1, 1), (4, 2, 4, 2), (512, 8, 8, 4), (1024, 8, 8, 4),
                                       (160, 8, 5, 2), (100, 6, 4, 2), (128, 8, 16, 4),
                                       (64, 8, 64, 8), (2048, 8, 8, 4), (96, 8, 3, 1)])
@pytest.mark.parametrize("bias", [False, True])
def test_route_matches_oracle(ctx, E, k, ng, tg, bias):
    import undertow_amd as U
    rng = np.random.default_rng(E * 10 + k)
    rows = 9
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    b = (-0.1 + 0.2 * np.arange(E) / max(E - 1, 1)).astype(np.float32) if bias else None
    ids, w = U.route(ctx, dev(logits), None if b is None else dev(b), k, ng, tg, True, 2.5)
    ids, w = host(ids), host(w)
    for r in range(rows):
        oid, ow = O.route(logits[r], b, k, ng, tg, True, 2.5)
        assert ids[r].tolist() == oid.tolist()
        assert np.abs(w[r] - ow).max() <= 1e-6


def test_route_reference_kats(ctx):
    """router.rs:132-186 restated: group limitation picks [0, 6, 1, 7]."""
    import undertow_amd as U
    logits = np.array([[2.0, 1.9, 3.0, -5.0, -1.0, -1.0, 2.0, 1.8]], np.float32)
    ids, _ = U.route(ctx, dev(logits), None, 4, 4, 2, False, 1.0)
    assert host(ids)[0].tolist() == [0, 6, 1, 7]
    ids, w = U.route(ctx, dev(np.array([[1.0, 0.0, 0.9]], np.float32)),
                     dev(np.array([0, 0, 0.5], np.float32)), 1, 1, 1, False, 1.0)
    assert host(ids)[0].tolist() == [2]
    assert abs(host(w)[0, 0] - 1 / (1 + np.exp(-0.9))) < 1e-6


def test_route_ties_pick_lowest_index(ctx):
    import undertow_amd as U
    logits = np.zeros((1, 32), np.float32)
    ids, _ = U.route(ctx, dev(logits), None, 8, 1, 1, True, 1.0)
    assert host(ids)[0].tolist() == list(range(8))


@pytest.mark.parametrize("E,ng,tg", [(256, 8, 4), (8, 4, 2), (1024, 8, 4)])
def test_route_ties_across_groups(ctx, E, ng, tg):
    """Equal group scores rank by group index; equal scores inside the
    eligible groups by expert index; masked (-inf) experts never win over
    eligible ones."""
    import undertow_amd as U
    rng = np.random.default_rng(E)
    rows = [np.zeros(E, np.float32),
            np.repeat(rng.standard_normal(E // 4).astype(np.float32), 4),
            np.tile(np.array([1.0, 0.5, 0.5, 1.0], np.float32), E // 4)]
    logits = np.stack(rows)
    k = min(8, E)
    ids, w = U.route(ctx, dev(logits), None, k, ng, tg, True, 1.0)
    ids, w = host(ids), host(w)
    for r in range(len(rows)):
        oid, ow = O.route(logits[r], None, k, ng, tg, True, 1.0)
        assert ids[r].tolist() == oid.tolist()
        assert np.abs(w[r] - ow).max() <= 1e-6


def test_route_k_above_expert_count(ctx):
    """k > E: the E experts in order, then id -1 / weight 0 slots."""
    import undertow_amd as U
    logits = np.array([[0.5, -1.0, 2.0, 0.1]], np.float32)
    ids, w = U.route(ctx, dev(logits), None, 6, 1, 1, True, 1.0)
    ids, w = host(ids)[0], host(w)[0]
    oid, ow = O.route(logits[0], None, 6, 1, 1, True, 1.0)
    assert ids[:4].tolist() == oid[:4].tolist() and ids[4:].tolist() == [-1, -1]
    assert np.abs(w[:4] - ow[:4]).max() <= 1e-6 and w[4:].tolist() == [0.0, 0.0]


# ------------------------------------------------------------------ argmax
def test_argmax_rows(ctx):
    import undertow_amd as U
    rng = np.random.default_rng(2)
    rows = [rng.standard_normal(129280).astype(np.float32) for _ in range(3)]
    rows.append(np.array([np.nan, 5.0, 1.0] + [0.0] * 61, np.float32))
    rows.append(np.array([1.0, np.nan, 2.0, 2.0] + [-np.inf] * 60, np.float32))
    t = np.full((3, 129280), -np.inf, np.float32)
    t[0, 77] = 3.0
    t[0, 99999] = 3.0  # tie: first index wins
    t[1, :] = np.nan
    t[1, 0] = 0.5      # v[0] finite, rest NaN -> 0
    t[2, 129279] = 1.0
    for r in rows[:3]:
        got = host(U.argmax_rows(ctx, dev(r[None])))[0]
        assert got == O.argmax(r)
    for r in rows[3:]:
        assert host(U.argmax_rows(ctx, dev(r[None])))[0] == O.argmax(r)
    got = host(U.argmax_rows(ctx, dev(t)))
    assert got.tolist() == [O.argmax(t[i]) for i in range(3)] == [77, 0, 129279]


# ------------------------------------------------------------- expert block
def make_experts(ctx, rng, fmt, E, H, I):
    import undertow_amd as U
    tbl = U.ExpertTable(ctx, E, H, I)
    host_w = []
    for e in range(E):
        g = rand_qtensor(rng, fmt, I, H)
        u = rand_qtensor(rng, fmt, I, H)
        d = rand_qtensor(rng, fmt, H, I)
        tbl.set(e, U.QTensor(ctx, fmt, *g, I, H), U.QTensor(ctx, fmt, *u, I, H),
                U.QTensor(ctx, fmt, *d, H, I))
        host_w.append((g, u, d))
    return tbl, host_w


def oracle_moe(fmt, H, I, host_w, ids, w, x):
    E = len(host_w)

    def payload(j):
        return np.concatenate([np.asarray(hw[j][0]).reshape(-1).view(np.uint8) for hw in host_w])

    def scales(j, rows):
        if fmt == F32:
            return np.zeros(E * rows, np.float32)
        return np.concatenate([np.asarray(hw[j][1]).reshape(-1) for hw in host_w])

    return O.moe_experts(fmt, H, I, payload(0), scales(0, I), payload(1), scales(1, I),
                         payload(2), scales(2, H), ids.astype(np.int64), w, x)


@pytest.mark.parametrize("fmt", [INT4, INT8])
@pytest.mark.parametrize("M", [1, 2, 3, 4, 6])
def test_moe_experts_small(ctx, fmt, M):
    rng = np.random.default_rng(40 + M + fmt)
    E, H, I, k = 8, 256, 128, 2
    tbl, host_w = make_experts(ctx, rng, fmt, E, H, I)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(M)]).astype(np.int32)
    ids[0] = [3, 5]
    if M > 1:
        ids[1] = [5, 0]  # shared expert across rows
    w = rng.random((M, k)).astype(np.float32)
    x = rng.standard_normal((M, H)).astype(np.float32)
    got = host(tbl.moe_experts(dev(ids), dev(w), dev(x)))
    want = oracle_moe(fmt, H, I, host_w, ids, w, x)
    tol = 1e-4 * np.maximum(np.abs(want), 1.0)
    assert (np.abs(got - want) <= tol).all(), np.abs(got - want).max()
    # per-row values do not depend on the other rows
    for s in range(M):
        one = host(tbl.moe_experts(dev(ids[s:s + 1]), dev(w[s:s + 1]), dev(x[s:s + 1])))
        assert np.array_equal(one[0], got[s])


@pytest.mark.parametrize("M", [1, 3, 7])
def test_moe_experts_many_choices(ctx, M):
    """k = 10 choices (the combine's general path past 8) and M*k > 64 at
    M = 7 (the plan built before gate/up instead of inside it)."""
    rng = np.random.default_rng(70 + M)
    E, H, I, k = 16, 512, 64, 10
    tbl, host_w = make_experts(ctx, rng, INT4, E, H, I)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(M)]).astype(np.int32)
    w = rng.random((M, k)).astype(np.float32)
    x = rng.standard_normal((M, H)).astype(np.float32)
    got = host(tbl.moe_experts(dev(ids), dev(w), dev(x)))
    want = oracle_moe(INT4, H, I, host_w, ids, w, x)
    tol = 1e-4 * np.maximum(np.abs(want), 1.0)
    assert (np.abs(got - want) <= tol).all(), np.abs(got - want).max()
    for s_ in range(M):
        one = host(tbl.moe_experts(dev(ids[s_:s_ + 1]), dev(w[s_:s_ + 1]), dev(x[s_:s_ + 1])))
        assert np.array_equal(one[0], got[s_])


@pytest.mark.parametrize("E,ids", [(4, [2, 2, 0, 3, 0, 1]), (8, [5, 5, 1, 5]), (8, [6, 1, 4, 2])])
def test_moe_one_row_repeated_ids(ctx, E, ids):
    """Repeated expert ids in one row, and more choices than experts: the
    plan gives such choices a shared slot, each choice still adds its own
    weight times that slot's row in choice order.  The row equals the
    oracle's and, bit for bit, the same row inside a two-row call."""
    rng = np.random.default_rng(len(ids) * 10 + E)
    H, I = 256, 128
    tbl, host_w = make_experts(ctx, rng, INT4, E, H, I)
    k = len(ids)
    idm = np.array([ids], np.int32)
    w = rng.random((1, k)).astype(np.float32)
    x = rng.standard_normal((1, H)).astype(np.float32)
    got = host(tbl.moe_experts(dev(idm), dev(w), dev(x)))
    want = oracle_moe(INT4, H, I, host_w, idm, w, x)
    tol = 1e-4 * np.maximum(np.abs(want), 1.0)
    assert (np.abs(got - want) <= tol).all(), np.abs(got - want).max()
    two = host(tbl.moe_experts(dev(np.repeat(idm, 2, 0)), dev(np.repeat(w, 2, 0)),
                               dev(np.repeat(x, 2, 0))))
    assert np.array_equal(two[0], got[0]) and np.array_equal(two[1], got[0])


def test_moe_experts_f32_weights(ctx):
    import undertow_amd as U
    rng = np.random.default_rng(9)
    E, H, I, k, M = 4, 64, 32, 2, 2
    tbl, host_w = make_experts(ctx, rng, F32, E, H, I)
    ids = np.array([[1, 3], [3, 0]], np.int32)
    w = rng.random((M, k)).astype(np.float32)
    x = rng.standard_normal((M, H)).astype(np.float32)
    got = host(tbl.moe_experts(dev(ids), dev(w), dev(x)))
    want = oracle_moe(F32, H, I, host_w, ids, w, x)
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("H,I", [(768, 512), (2560, 256), (512, 272)])
def test_moe_int8_matrix_core_shapes(ctx, H, I):
    """int8 experts at 2-4 rows take the matrix-core gate/up (H % 256 == 0)
    and down (I % 256 == 0, I <= 2048); the shapes cover an odd segment
    count (768: three 256-column segments), x staged in two chunks (2560 >
    2048 columns), and a row tail with down on the dot-product kernel (272).
    Rows equal one-row calls, which run the dot-product kernels, bit for bit."""
    rng = np.random.default_rng(H + I)
    E, k = 8, 3
    tbl, host_w = make_experts(ctx, rng, INT8, E, H, I)
    for M in (2, 3, 4):
        ids = np.stack([rng.permutation(E)[:k] for _ in range(M)]).astype(np.int32)
        w = rng.random((M, k)).astype(np.float32)
        x = rng.standard_normal((M, H)).astype(np.float32)
        got = host(tbl.moe_experts(dev(ids), dev(w), dev(x)))
        want = oracle_moe(INT8, H, I, host_w, ids, w, x)
        tol = 1e-4 * np.maximum(np.abs(want), 1.0)
        assert (np.abs(got - want) <= tol).all(), (M, np.abs(got - want).max())
        for s in range(M):
            one = host(tbl.moe_experts(dev(ids[s:s + 1]), dev(w[s:s + 1]), dev(x[s:s + 1])))
            assert np.array_equal(one[0], got[s]), (M, s)


def test_moe_one_slot_int8_split_down(ctx):
    """A one-slot int8 MLP (every row on one expert: the dense FFN's form)
    at hidden 7168, inter 10240: at 2-4 rows gate/up runs on the matrix
    cores and down splits K into five 2,048-column slices on the matrix
    cores, whose exact partials the finish launch sums; each row equals a
    one-row call (dot-product kernels) bit for bit, and the oracle."""
    rng = np.random.default_rng(77)
    E, H, I, k = 1, 7168, 10240, 1
    tbl, host_w = make_experts(ctx, rng, INT8, E, H, I)
    for M in (2, 3, 4):
        ids = np.zeros((M, k), np.int32)
        w = rng.random((M, k)).astype(np.float32)
        x = rng.standard_normal((M, H)).astype(np.float32)
        got = host(tbl.moe_experts(dev(ids), dev(w), dev(x)))
        want = oracle_moe(INT8, H, I, host_w, ids, w, x)
        tol = 1e-4 * np.maximum(np.abs(want), 1.0)
        assert (np.abs(got - want) <= tol).all(), (M, np.abs(got - want).max())
        for s in range(M):
            one = host(tbl.moe_experts(dev(ids[s:s + 1]), dev(w[s:s + 1]), dev(x[s:s + 1])))
            assert np.array_equal(one[0], got[s]), (M, s)


@pytest.mark.parametrize("fmt,Ms", [(INT4, (1, 2, 4)), (INT8, (1, 2, 3, 4))])
def test_moe_experts_deepseek_shape(ctx, fmt, Ms):
    """hidden 7168, inter 2048, top-8 of 16 loaded experts
    (M = 1 takes the streaming gate/up kernel), int4 and the int8 variant at
    the same shapes (undertow-quant/src/kernels.rs:21-44)."""
    rng = np.random.default_rng(1234)
    E, H, I, k = 16, 7168, 2048, 8
    tbl, host_w = make_experts(ctx, rng, fmt, E, H, I)
    for M in Ms:
        ids = np.stack([rng.permutation(E)[:k] for _ in range(M)]).astype(np.int32)
        w = rng.random((M, k)).astype(np.float32)
        x = rng.standard_normal((M, H)).astype(np.float32)
        got = host(tbl.moe_experts(dev(ids), dev(w), dev(x)))
        want = oracle_moe(fmt, H, I, host_w, ids, w, x)
        tol = 1e-4 * np.maximum(np.abs(want), 1.0)
        assert (np.abs(got - want) <= tol).all(), (M, np.abs(got - want).max())
        # a one-row call (the gate/up launch plans and digitises x itself)
        # gives the multi-row call's row bit for bit
        if M > 1:
            for s in range(M):
                one = host(tbl.moe_experts(dev(ids[s:s + 1]), dev(w[s:s + 1]), dev(x[s:s + 1])))
                assert np.array_equal(one[0], got[s]), (M, s)


@pytest.mark.parametrize("fmt,H,I,Ms", [(INT4, 512, 256, (1, 2, 3, 5)), (INT8, 512, 128, (1, 2)),
                                         (INT4, 7168, 2048, (1, 2))])
@pytest.mark.parametrize("bias", [False, True])
def test_moe_route_experts_matches_route_then_experts(ctx, fmt, H, I, Ms, bias):
    """ut_moe_route_experts (routing inside the gate/up launch at one row
    with DeepSeek-V3's router: 256 experts, 8 groups, top-4 groups, top-8)
    gives ut_route's choices and ut_moe_experts' output bit for bit, and
    the oracle's within the expert bar.  The 256-entry table reuses 16
    distinct weight sets (each id is still its own slot)."""
    import undertow_amd as U
    rng = np.random.default_rng(500 + H + fmt + bias)
    E, k, ng, tg = 256, 8, 8, 4
    n_w = 16
    tbl = U.ExpertTable(ctx, E, H, I)
    host_w = []
    qts = []
    for j in range(n_w):
        g = rand_qtensor(rng, fmt, I, H)
        u = rand_qtensor(rng, fmt, I, H)
        d = rand_qtensor(rng, fmt, H, I)
        qts.append((U.QTensor(ctx, fmt, *g, I, H), U.QTensor(ctx, fmt, *u, I, H),
                    U.QTensor(ctx, fmt, *d, H, I)))
        host_w.append((g, u, d))
    for e in range(E):
        tbl.set(e, *qts[e % n_w])
    b = (rng.standard_normal(E) * 0.1).astype(np.float32) if bias else None
    for M in Ms:
        logits = rng.standard_normal((M, E)).astype(np.float32)
        x = rng.standard_normal((M, H)).astype(np.float32)
        out, ids, w = tbl.moe_route_experts(dev(logits), None if b is None else dev(b), dev(x),
                                            k, ng, tg, True, 2.5)
        rid, rw = U.route(ctx, dev(logits), None if b is None else dev(b), k, ng, tg, True, 2.5)
        ref = tbl.moe_experts(rid, rw, dev(x))
        assert np.array_equal(host(ids), host(rid)), M
        assert np.array_equal(host(w), host(rw)), M
        assert np.array_equal(host(out), host(ref)), M
        hid, hw = host(ids), host(w)
        for r in range(M):
            oid, ow = O.route(logits[r], b, k, ng, tg, True, 2.5)
            assert hid[r].tolist() == oid.tolist(), (M, r)
            assert np.abs(hw[r] - ow).max() <= 1e-6, (M, r)
        # id e holds weight set e % 16 (the oracle computes each choice on
        # its own, so two ids sharing a set stay two choices)
        want = oracle_moe(fmt, H, I, host_w, (hid % n_w).astype(np.int32), hw, x)
        tol = 1e-4 * np.maximum(np.abs(want), 1.0)
        assert (np.abs(host(out) - want) <= tol).all(), (M, np.abs(host(out) - want).max())


@pytest.mark.parametrize("fmt", [INT4, INT8])
def test_moe_one_row_equals_two_rows_repeated(ctx, fmt):
    """One row and two rows take different gate/up kernels (the one-row
    kernel plans and digitises x itself).  Over many calls, with the routing
    inside the call and without, the one-row result equals each row of the
    two-row call on the duplicated row bit for bit, and the oracle within the
    expert bar."""
    import undertow_amd as U
    rng = np.random.default_rng(77 + fmt)
    E, H, I, k = 16, 1024, 512, 8
    tbl, host_w = make_experts(ctx, rng, fmt, E, H, I)
    for it in range(40):
        ids = rng.permutation(E)[:k].astype(np.int32)[None]
        w = rng.random((1, k)).astype(np.float32)
        x = rng.standard_normal((1, H)).astype(np.float32)
        one = host(tbl.moe_experts(dev(ids), dev(w), dev(x)))
        two = host(tbl.moe_experts(dev(np.repeat(ids, 2, 0)), dev(np.repeat(w, 2, 0)),
                                   dev(np.repeat(x, 2, 0))))
        assert np.array_equal(one[0], two[0]) and np.array_equal(one[0], two[1]), it
        if it % 10 == 0:
            want = oracle_moe(fmt, H, I, host_w, ids, w, x)
            assert (np.abs(one - want) <= 1e-4 * np.maximum(np.abs(want), 1.0)).all(), it
    logits = rng.standard_normal((1, E)).astype(np.float32)
    x = rng.standard_normal((1, H)).astype(np.float32)
    for it in range(20):
        out, ids, w = tbl.moe_route_experts(dev(logits), None, dev(x), k, 4, 2, True, 2.5)
        ref = tbl.moe_experts(ids, w, dev(np.repeat(x, 1, 0)))
        assert np.array_equal(host(out), host(ref)), it
        logits = rng.standard_normal((1, E)).astype(np.float32)
    ctx.synchronize()


@pytest.mark.parametrize("E,ng,tg", [(256, 8, 4), (256, 1, 1), (224, 7, 3), (256, 8, 8)])
@pytest.mark.parametrize("bias", [False, True])
def test_moe_route_experts_ties_match_route(ctx, E, ng, tg, bias):
    """The one-row routing inside the gate/up launch (four keys per lane)
    against ut_route's wave router on logits with many ties: values on a
    coarse grid (equal sigmoids inside and across groups, tied group
    scores), all-equal rows, and a NaN.  Ids, weights and outputs bit for
    bit; ids also against the oracle."""
    import undertow_amd as U
    rng = np.random.default_rng(E + ng + bias)
    H, I, k, n_w = 256, 64, 8, 8
    tbl = U.ExpertTable(ctx, E, H, I)
    qts = []
    for j in range(n_w):
        g, u, d = (rand_qtensor(rng, INT8, I, H), rand_qtensor(rng, INT8, I, H),
                   rand_qtensor(rng, INT8, H, I))
        qts.append((U.QTensor(ctx, INT8, *g, I, H), U.QTensor(ctx, INT8, *u, I, H),
                    U.QTensor(ctx, INT8, *d, H, I)))
    for e in range(E):
        tbl.set(e, *qts[e % n_w])
    b = (rng.integers(-2, 3, E) * 0.05).astype(np.float32) if bias else None
    rows = [rng.integers(-3, 4, E).astype(np.float32) * 0.5 for _ in range(12)]
    rows.append(np.zeros(E, np.float32))
    rows.append(np.full(E, 2.0, np.float32))
    nan_row = rng.integers(-3, 4, E).astype(np.float32)
    nan_row[37] = np.nan
    rows.append(nan_row)
    x = dev(rng.standard_normal((1, H)).astype(np.float32))
    for i, lg in enumerate(rows):
        logits = dev(lg[None])
        bd = None if b is None else dev(b)
        out, ids, w = tbl.moe_route_experts(logits, bd, x, k, ng, tg, True, 2.5)
        rid, rw = U.route(ctx, logits, bd, k, ng, tg, True, 2.5)
        ref = tbl.moe_experts(rid, rw, x)
        assert np.array_equal(host(ids), host(rid)), i
        assert np.array_equal(host(w), host(rw), equal_nan=True), i
        assert np.array_equal(host(out), host(ref), equal_nan=True), i
        if not np.isnan(lg).any():
            oid, _ = O.route(lg, b, k, ng, tg, True, 2.5)
            assert host(ids)[0].tolist() == oid.tolist(), i
    ctx.synchronize()


@pytest.mark.parametrize("fmt", [INT4, INT8])
@pytest.mark.parametrize("H", [1024, 7168])
def test_moe_bf16_activations_equal_widened_f32(ctx, fmt, H):
    """bf16 activations (ut_moe_experts_bf16 / ut_moe_route_experts_bf16):
    bit-identical to the f32 entry points on the exactly widened values, at
    one row (the gate/up launch widens while staging), two to four rows
    (widened first) and five (two passes); the oracle within the expert bar
    on the widened x."""
    import torch
    rng = np.random.default_rng(91 + fmt + H)
    E, I, k = 16, 512, 8
    tbl, host_w = make_experts(ctx, rng, fmt, E, H, I)
    for M in (1, 2, 3, 4, 5, 1):
        ids = np.stack([rng.permutation(E)[:k] for _ in range(M)]).astype(np.int32)
        w = rng.random((M, k)).astype(np.float32)
        xb = dev(rng.standard_normal((M, H)).astype(np.float32)).to(torch.bfloat16)
        xw = xb.float()
        got = host(tbl.moe_experts(dev(ids), dev(w), xb))
        ref = host(tbl.moe_experts(dev(ids), dev(w), xw))
        assert np.array_equal(got, ref), M
        want = oracle_moe(fmt, H, I, host_w, ids, w, host(xw))
        assert (np.abs(got - want) <= 1e-4 * np.maximum(np.abs(want), 1.0)).all(), M
        logits = dev(rng.standard_normal((M, E)).astype(np.float32))
        out, rid, rw = tbl.moe_route_experts(logits, None, xb, k, 4, 2, True, 2.5)
        out2, rid2, rw2 = tbl.moe_route_experts(logits, None, xw, k, 4, 2, True, 2.5)
        assert np.array_equal(host(rid), host(rid2)) and np.array_equal(host(rw), host(rw2))
        assert np.array_equal(host(out), host(out2)), M
    ctx.synchronize()


def test_moe_bf16_activations_checked(ctx):
    """Misaligned bf16 rows and a hidden size that is not a multiple of 8
    are refused on the host before any launch."""
    import torch
    import undertow_amd as U
    rng = np.random.default_rng(5)
    tbl, _ = make_experts(ctx, rng, INT8, 4, 256, 64)
    ids, w = dev(np.array([[0, 1]], np.int32)), dev(np.ones((1, 2), np.float32))
    buf = torch.zeros(257, dtype=torch.bfloat16, device="cuda:0")
    with pytest.raises(U.UtError, match="alignment"):
        tbl.moe_experts(ids, w, buf[1:].view(1, 256))
    tbl2, _ = make_experts(ctx, rng, INT8, 2, 36, 16)
    with pytest.raises(U.UtError, match="alignment"):
        tbl2.moe_experts(ids, w, torch.zeros((1, 36), dtype=torch.bfloat16, device="cuda:0"))
    ctx.synchronize()


@pytest.mark.parametrize("H", [64, 256])  # 256: the gate/up launch resolves the plan
def test_moe_bad_expert_is_reported(ctx, H):
    import undertow_amd as U
    rng = np.random.default_rng(3)
    tbl, _ = make_experts(ctx, rng, INT8, 4, H, 32)
    ids = np.array([[1, 9]], np.int32)
    out = tbl.moe_experts(dev(ids), dev(np.ones((1, 2), np.float32)),
                          dev(np.ones((1, H), np.float32)))
    with pytest.raises(U.UtError) as ei:
        ctx.synchronize()
    assert ei.value.code == U.runtime.UT_ERR_BAD_EXPERT
    assert np.isfinite(host(out)).all()
    ctx.synchronize()  # the flag is cleared once reported


# --------------------------------------------------------------- attention
@pytest.mark.parametrize("R,H,L,P,T", [(1, 4, 64, 16, 5), (2, 4, 64, 16, 40), (4, 8, 16, 8, 300),
                                       (2, 128, 512, 64, 1024), (1, 128, 512, 64, 600),
                                       (3, 6, 32, 8, 17), (4, 128, 512, 64, 4096),
                                       (2, 128, 512, 64, 9000), (1, 128, 512, 64, 33)])
def test_mla_attend_matches_oracle(ctx, R, H, L, P, T):
    """DeepSeek-V3 shapes (128 heads, 512 + 64) run on the bf16 matrix cores
    with each f32 operand split into bf16 hi + lo parts (products keep about
    16 significant bits): bar 1e-4 of the largest output, against 1e-5 for
    the f32 kernel that adds in the reference's order."""
    import undertow_amd as U
    rng = np.random.default_rng(R * 100 + T)
    qabs = rng.standard_normal((R, H, L)).astype(np.float32)
    qr = rng.standard_normal((R, H, P)).astype(np.float32)
    lat = rng.standard_normal((T, L)).astype(np.float32)
    kr = rng.standard_normal((T, P)).astype(np.float32)
    pos_base = T - R
    scale = float(1 / np.sqrt(192.0))
    got = host(U.mla_attend(ctx, dev(qabs), dev(qr), dev(lat), dev(kr), pos_base, scale))
    want = O.mla_attend(qabs, qr, lat, kr, pos_base, scale)
    mfma = H % 32 == 0 and L == 512 and P == 64
    tol = (1e-4 if mfma else 1e-5) * max(1.0, np.abs(want).max())
    assert np.abs(got - want).max() <= tol, np.abs(got - want).max()
    if mfma:
        # the split-cache entry (cache converted once) gives the same bits
        kc = U.mla_cache_split(ctx, dev(lat), dev(kr))
        got2 = host(U.mla_attend_split(ctx, dev(qabs), dev(qr), kc, pos_base, scale))
        assert np.array_equal(got2, got)
    # row independence: row s alone at pos_base + s sees the same context
    for s in range(R):
        one = host(U.mla_attend(ctx, dev(qabs[s:s + 1]), dev(qr[s:s + 1]), dev(lat), dev(kr),
                                pos_base + s, scale))
        assert np.array_equal(one[0], got[s])


HEADS_CHECKED = [0, 1, 31, 32, 63, 64, 100, 127]


@pytest.mark.parametrize("R,T", [(1, 32768), (2, 32768), (4, 32768), (4, 16400), (3, 16385)])
def test_mla_long_context_matches_oracle(ctx, R, T):
    """Config 3's longest context: past 16384 positions the matrix-core
    kernel's slices grow past 256 positions (512 at 32768, 61 slices of 272
    at 16400).  All
    128 heads run on the GPU; the oracle's sequential loops check eight of
    them (its (row, head) pairs are independent)."""
    import undertow_amd as U
    H, L, P = 128, 512, 64
    rng = np.random.default_rng(R * 7 + T)
    qabs = rng.standard_normal((R, H, L)).astype(np.float32)
    qr = rng.standard_normal((R, H, P)).astype(np.float32)
    lat = rng.standard_normal((T, L)).astype(np.float32)
    kr = rng.standard_normal((T, P)).astype(np.float32)
    pos_base = T - R
    scale = float(1 / np.sqrt(192.0))
    kc = U.mla_cache_split(ctx, dev(lat), dev(kr))
    got = host(U.mla_attend_split(ctx, dev(qabs), dev(qr), kc, pos_base, scale))
    hs = HEADS_CHECKED
    want = O.mla_attend(np.ascontiguousarray(qabs[:, hs]), np.ascontiguousarray(qr[:, hs]), lat, kr,
                        pos_base, scale)
    tol = 1e-4 * max(1.0, np.abs(want).max())
    assert np.abs(got[:, hs] - want).max() <= tol, np.abs(got[:, hs] - want).max()
    assert np.isfinite(got).all()
    for s in range(R):
        one = host(U.mla_attend_split(ctx, dev(qabs[s:s + 1]), dev(qr[s:s + 1]), kc, pos_base + s,
                                      scale))
        assert np.array_equal(one[0], got[s])


def test_mla_split_cache_round_trip(ctx):
    """hi + lo of the split cache reproduces the f32 cache to 2^-16 relative
    (hi = bf16(x) rounded to nearest, lo = bf16(x - hi))."""
    import torch
    import undertow_amd as U
    rng = np.random.default_rng(5)
    T, L, P = 37, 512, 64
    lat = (rng.standard_normal((T, L)) * np.exp(rng.uniform(-20, 20, (T, 1)))).astype(np.float32)
    kr = rng.standard_normal((T, P)).astype(np.float32)
    kc = U.mla_cache_split(ctx, dev(lat), dev(kr))
    bits = host(kc).astype(np.uint16).astype(np.uint32) << 16
    parts = bits.view(np.float32).astype(np.float64)  # [T, 2, L+P]
    x = np.concatenate([lat, kr], 1).astype(np.float64)
    hi, lo = parts[:, 0], parts[:, 1]
    # hi is x rounded to bf16 (8 significant bits)
    assert np.all(np.abs(hi - x) <= np.abs(x) * 2.0 ** -8)
    assert np.all(np.abs(hi + lo - x) <= np.abs(x) * 2.0 ** -16)


def test_mla_attend_split_rejects_other_shapes(ctx):
    import undertow_amd as U
    q = dev(np.zeros((1, 4, 64), np.float32))
    qr = dev(np.zeros((1, 4, 16), np.float32))
    kc = U.mla_cache_split(ctx, dev(np.zeros((8, 64), np.float32)), dev(np.zeros((8, 16), np.float32)))
    with pytest.raises(U.UtError) as ei:
        U.mla_attend_split(ctx, q, qr, kc, 4, 0.1)
    assert ei.value.code == U.runtime.UT_ERR_SHAPE



def test_kernel_timing(ctx):
    """Bench tooling: per-launch event timing."""
    rng = np.random.default_rng(5)
    tbl, _ = make_experts(ctx, rng, INT8, 4, 256, 32)
    ids = dev(np.array([[0, 2]], np.int32))
    w = dev(np.ones((1, 2), np.float32))
    x = dev(rng.standard_normal((1, 256)).astype(np.float32))
    ctx.enable_timing(True)
    for _ in range(3):
        tbl.moe_experts(ids, w, x)
    ctx.synchronize()
    n, ms = ctx.kernel_time("moe_gate_up")
    nd, msd = ctx.kernel_time("moe_down")
    ctx.enable_timing(False)
    assert n == 3 and nd == 3 and ms > 0 and msd > 0


@pytest.mark.parametrize("I", [96, 160])
def test_moe_matrix_core_gate_up_row_tail(ctx, I):
    """The matrix-core gate/up takes 64 h rows per workgroup at 2-4 rows
    when the routed experts have the launch to themselves; with I % 64 == 32
    the last workgroup's second tile lies past I and its waves clamp their
    rows.  Every row equals the one-row call (the dot-product kernels) bit
    for bit and the oracle within the expert bar."""
    rng = np.random.default_rng(I)
    E, H, k = 8, 512, 4
    tbl, host_w = make_experts(ctx, rng, INT4, E, H, I)
    for M in (2, 3, 4):
        ids = np.stack([rng.permutation(E)[:k] for _ in range(M)]).astype(np.int32)
        w = rng.random((M, k)).astype(np.float32)
        x = rng.standard_normal((M, H)).astype(np.float32)
        got = host(tbl.moe_experts(dev(ids), dev(w), dev(x)))
        assert np.isfinite(got).all(), M
        want = oracle_moe(INT4, H, I, host_w, ids, w, x)
        tol = 1e-4 * np.maximum(np.abs(want), 1.0)
        assert (np.abs(got - want) <= tol).all(), (M, np.abs(got - want).max())
        for s in range(M):
            one = host(tbl.moe_experts(dev(ids[s:s + 1]), dev(w[s:s + 1]), dev(x[s:s + 1])))
            assert np.array_equal(one[0], got[s]), (M, s)
