"""ut_moe_experts_noalloc: the expert block without any allocation, against
ut_moe_experts (the same kernels, so bit-identical) on two calls in a row,
the second with fewer rows, and at the DeepSeek-V3 expert shape."""
import numpy as np
import pytest

from conftest import dev, host

pytestmark = pytest.mark.gpu


def make_table(ctx, rng, E, H, I):
    import undertow_amd as U
    tbl = U.ExpertTable(ctx, E, H, I)
    for e in range(E):
        qs = []
        for o, i in ((I, H), (I, H), (H, I)):
            p = rng.integers(0, 256, size=(o, i // 2), dtype=np.uint8)
            s = (np.abs(rng.normal(0, 0.02, o)) / 7).astype(np.float32)
            qs.append(U.QTensor(ctx, U.INT4, p, s, o, i))
        tbl.set(e, *qs)
    return tbl


@pytest.mark.parametrize("E,H,I,k", [(16, 7168, 2048, 8), (8, 512, 256, 2)])
def test_noalloc_matches_moe_experts(ctx, E, H, I, k):
    import torch
    rng = np.random.default_rng(E + H)
    tbl = make_table(ctx, rng, E, H, I)
    for rows in (4, 1, 3):  # a smaller call after a larger one, then a middle one
        ids = np.stack([rng.permutation(E)[:k] for _ in range(rows)]).astype(np.int32)
        w = rng.random((rows, k)).astype(np.float32)
        x = rng.standard_normal((rows, H)).astype(np.float32)
        ids_d, w_d, x_d = dev(ids), dev(w), dev(x)
        want = host(tbl.moe_experts(ids_d, w_d, x_d))
        out = torch.full((rows, H), float("nan"), device="cuda:0")
        tbl.moe_experts_noalloc(ids_d, w_d, x_d, out)
        got = host(out)
        assert np.array_equal(got, want), (rows, np.abs(got - want).max())
    ctx.synchronize()


def test_noalloc_rejects_working_sets_beyond_its_array(ctx):
    import torch
    import undertow_amd as U
    rng = np.random.default_rng(2)
    tbl = U.ExpertTable(ctx, 256, 7168, 2048)
    qs = []
    for o, i in ((2048, 7168), (2048, 7168), (7168, 2048)):
        qs.append(U.QTensor(ctx, U.INT4, rng.integers(0, 256, size=(o, i // 2), dtype=np.uint8),
                            np.full(o, 1e-3, np.float32), o, i))
    tbl.set(0, *qs)
    k = 64
    ids = dev(np.zeros((4, k), np.int32))
    w = dev(np.ones((4, k), np.float32))
    x = dev(np.zeros((4, 7168), np.float32))
    out = torch.empty((4, 7168), device="cuda:0")
    with pytest.raises(U.UtError) as ei:
        tbl.moe_experts_noalloc(ids, w, x, out)
    assert ei.value.code == U.runtime.UT_ERR_ARG
    assert "exceeds" in str(ei.value)


def test_noalloc_refuses_a_second_context_on_the_device(ctx):
    """The array is one per device: the first context that calls owns it, a
    second context on the same GPU is refused rather than racing on it, and
    the owner keeps working."""
    import torch
    import undertow_amd as U
    rng = np.random.default_rng(5)
    tbl = make_table(ctx, rng, 8, 512, 256)
    ids = dev(np.stack([rng.permutation(8)[:2] for _ in range(2)]).astype(np.int32))
    w, x = dev(rng.random((2, 2)).astype(np.float32)), dev(rng.standard_normal((2, 512)).astype(np.float32))
    out = torch.empty((2, 512), device="cuda:0")
    tbl.moe_experts_noalloc(ids, w, x, out)  # ctx owns the device's array
    other = U.Context(0)
    tbl2 = make_table(other, rng, 8, 512, 256)
    with pytest.raises(U.UtError) as ei:
        tbl2.moe_experts_noalloc(ids, w, x, out)
    assert ei.value.code == U.runtime.UT_ERR_STATE
    del tbl2, other
    want = host(tbl.moe_experts(ids, w, x))
    tbl.moe_experts_noalloc(ids, w, x, out)
    assert np.array_equal(host(out), want)
