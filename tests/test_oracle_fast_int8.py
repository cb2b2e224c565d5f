"""The oracle's restatement of the opt-in fast-int8 path (undertow-quant/src/
lib.rs:31-59, avx512.rs:221-242, neon.rs:139-184), pinned by the reference's
own bound and by closed forms that a plausible slip (banker's rounding, NaN
not mapped to 0, scale and inverse swapped, the scales multiplied in another
order) fails.
"""
import numpy as np
import pytest

from oracle import oracle as O


def f32_sym(rng, n):
    return rng.uniform(-1.0, 1.0, n).astype(np.float32)


@pytest.mark.parametrize("o,i", [(4, 64), (7, 130), (3, 16)])
def test_fast_int8_close_to_scalar(o, i):
    # neon.rs:257-278 (fast_int8_kernel_close_to_scalar): within 3 % of the
    # largest exact output
    rng = np.random.default_rng(0xFA57 + o * i)
    w = f32_sym(rng, o * i).reshape(o, i)
    x = f32_sym(rng, 2 * i).reshape(2, i)
    q, s = O.quantize(w, O.INT8)
    fast = O.matmul_fast_i8(q, s, o, i, x)
    exact = O.matmul(O.INT8, q, s, o, i, x)
    mag = max(np.abs(exact).max(), 1e-3)
    assert (np.abs(fast - exact) <= 0.03 * mag).all()


def test_quantize_activations_rounding_and_edges():
    # max 127 -> inv 1: codes are the values rounded half away from zero
    q, s = O.quantize_activations(np.array([127, 2.5, -2.5, 0.5, -0.5, 1.49, -126.6], np.float32))
    assert s == np.float32(1.0)
    assert q.tolist() == [127, 3, -3, 1, -1, 1, -127]
    # NaN is skipped by the max and quantised to 0
    q, s = O.quantize_activations(np.array([np.nan, 2.0, -4.0], np.float32))
    assert s == np.float32(np.float32(4.0) / np.float32(127.0))
    assert q.tolist() == [0, 64, -127]
    # a zero row: scale 0, codes 0
    q, s = O.quantize_activations(np.zeros(5, np.float32))
    assert s == 0.0 and not q.any()


def test_codes_match_closed_form():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(1000) * 3).astype(np.float32)
    q, s = O.quantize_activations(x)
    m = np.float32(np.abs(x).max())
    inv = np.float32(127.0) / m
    t = (x * inv).astype(np.float32)
    want = np.clip(np.sign(t) * np.floor(np.abs(t) + np.float32(0.5)), -127, 127).astype(np.int8)
    assert np.array_equal(q, want) and s == m / np.float32(127.0)


def test_integer_activations_equal_the_exact_path():
    # integer activations with max 127 quantise to themselves (scale 1), so
    # with sums below 2^24 the fast path equals the exact int8 matmul bit for bit
    rng = np.random.default_rng(11)
    o, i = 9, 200
    x = rng.integers(-127, 128, (3, i)).astype(np.float32)
    x[:, 0] = 127.0
    q = rng.integers(-127, 128, (o, i)).astype(np.int8)
    s = (rng.random(o) * 0.01 + 0.001).astype(np.float32)
    fast = O.matmul_fast_i8(q.view(np.uint8), s, o, i, x)
    exact = O.matmul(O.INT8, q.view(np.uint8), s, o, i, x)
    assert np.array_equal(fast.view(np.uint32), exact.view(np.uint32))


def test_epilogue_order():
    # out = ((acc as f32) * a_scale) * scale, left to right
    rng = np.random.default_rng(5)
    o, i = 16, 96
    x = f32_sym(rng, i)[None]
    q = rng.integers(-127, 128, (o, i)).astype(np.int8)
    s = (rng.random(o) * 0.37 + 0.01).astype(np.float32)
    qa, a = O.quantize_activations(x[0])
    acc = (q.astype(np.int64) @ qa.astype(np.int64)).astype(np.float32)
    want = (acc * a).astype(np.float32) * s
    got = O.matmul_fast_i8(q.view(np.uint8), s, o, i, x)[0]
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_infinite_activation_gives_nan():
    # max = inf: inv = 0, every code 0 (inf * 0 is NaN -> 0), a_scale = inf,
    # so each output is 0 * inf
    q = np.ones((2, 3), np.int8)
    out = O.matmul_fast_i8(q.view(np.uint8), np.ones(2, np.float32), 2, 3,
                           np.array([[np.inf, 1.0, 2.0]], np.float32))
    assert np.isnan(out).all()


def test_oracle_model_fast_int8_keeps_agreement(golden_dir):
    """undertow-bench/tests/fast_int8.rs:24-61 on the oracle: the fixture
    converted to int8 experts and dense weights, forwarded with the
    process-global switch on (every int8 matmul of the model quantises its
    activations per row), keeps >= 75 % teacher-forcing argmax agreement
    with the transformers golden; the switch changes the logits, and off
    again restores the exact path bit for bit."""
    import json
    from models import checkpoint
    ref = json.loads((golden_dir / "oracle-tiny" / "reference.json").read_text())
    om = O.Model(checkpoint(fmt="int8"))
    exact = om.forward(ref["full_ids"])
    O.set_fast_int8(True)
    try:
        assert O.fast_int8_enabled()
        fast = om.forward(ref["full_ids"])
    finally:
        O.set_fast_int8(False)
    assert not O.fast_int8_enabled()
    agree = np.mean([int(fast[s].argmax()) == ref["tf_pred"][s] for s in range(len(ref["full_ids"]))])
    assert agree >= 0.75, agree
    assert not np.array_equal(fast, exact)
    # fast-int8 differs from the exact path by about the activation
    # quantisation error (lib.rs:31-34: ~1e-2 relative; 3 % of the mean
    # logit magnitude here)
    assert np.abs(fast - exact).mean() <= 0.06 * np.abs(exact).mean()
    assert np.array_equal(om.forward(ref["full_ids"]), exact)
