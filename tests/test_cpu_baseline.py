"""The timed CPU baseline (oracle/cpu_baseline.c, libcpu_model.so) against
the scalar oracle: the restated dispatched kernels must compute the
reference's function, within the reference's own SIMD-vs-scalar bound
(1e-4 relative, undertow-quant/src/avx512.rs:335-366), at every ISA the
dispatcher can pick."""
import ctypes as C

import numpy as np
import pytest

from models import C1, checkpoint, prompt_ids
from oracle import oracle as O
from qgen import INT4, INT8, rand_qtensor

SHAPES = [(1, 1), (3, 16), (5, 17), (8, 64), (7, 130), (16, 256), (2, 31), (64, 7168)]


@pytest.fixture(params=[2, 1, 0], ids=["avx512", "avx2", "scalar"])
def isa(request):
    L = O.cpu_baseline_lib()
    avail = int(L.ucb_isa())
    if request.param > avail:
        pytest.skip(f"ISA level {request.param} not available on this host")
    L.ucb_set_isa(request.param)
    yield request.param
    L.ucb_set_isa(-1)


@pytest.mark.parametrize("fmt", [INT4, INT8])
@pytest.mark.parametrize("o,i", SHAPES)
def test_ucb_matmul_matches_oracle(isa, fmt, o, i):
    L = O.cpu_baseline_lib()
    rng = np.random.default_rng(o * 7 + i + fmt)
    payload, scales = rand_qtensor(rng, fmt, o, i)
    x = rng.standard_normal((3, i)).astype(np.float32)
    out = np.zeros((3, o), np.float32)
    L.ucb_matmul(fmt, payload.ctypes.data, scales.ctypes.data, o, i, x.reshape(-1), 3,
                 out.reshape(-1), 2)
    want = O.matmul(fmt, payload, scales, o, i, x)
    assert (np.abs(out - want) <= 1e-4 * np.maximum(np.abs(want), 1.0)).all()


@pytest.mark.parametrize("fmt", [INT4, INT8])
def test_ucb_moe_experts_matches_oracle(isa, fmt):
    L = O.cpu_baseline_lib()
    rng = np.random.default_rng(3 + fmt)
    E, H, I, k, M = 6, 256, 96, 3, 2
    mats = [rand_qtensor(rng, fmt, o, i) for _ in range(E) for (o, i) in ((I, H), (I, H), (H, I))]
    cat = lambda j: np.concatenate([mats[3 * e + j][0].reshape(-1) for e in range(E)])
    cats = lambda j: np.concatenate([mats[3 * e + j][1] for e in range(E)])
    g, gs, u, us, d, ds = cat(0), cats(0), cat(1), cats(1), cat(2), cats(2)
    ids = np.array([[0, 4, 2], [4, 5, 0]], np.int64)
    w = rng.random((M, k)).astype(np.float32)
    x = rng.standard_normal((M, H)).astype(np.float32)
    out = np.zeros((M, H), np.float32)
    L.ucb_moe_experts(fmt, H, I, g.ctypes.data, gs.ctypes.data, u.ctypes.data, us.ctypes.data,
                      d.ctypes.data, ds.ctypes.data, M, k, ids.reshape(-1), w.reshape(-1),
                      x.reshape(-1), out.reshape(-1), 2)
    want = O.moe_experts(fmt, H, I, g, gs, u, us, d, ds, ids, w, x)
    assert (np.abs(out - want) <= 1e-4 * np.maximum(np.abs(want), 1.0)).all()


def test_ucb_mla_attend_matches_oracle():
    L = O.cpu_baseline_lib()
    rng = np.random.default_rng(9)
    R, H, Ld, P, T = 3, 8, 64, 16, 77
    qabs = rng.standard_normal((R, H, Ld)).astype(np.float32)
    qr = rng.standard_normal((R, H, P)).astype(np.float32)
    lat = rng.standard_normal((T, Ld)).astype(np.float32)
    kr = rng.standard_normal((T, P)).astype(np.float32)
    out = np.zeros((R, H, Ld), np.float32)
    L.ucb_mla_attend(qabs.reshape(-1), qr.reshape(-1), lat.reshape(-1), kr.reshape(-1), R, H, Ld, P,
                     T - R, 0.125, out.reshape(-1), 2)
    want = O.mla_attend(qabs, qr, lat, kr, T - R, 0.125)
    assert np.abs(out - want).max() <= 1e-5 * max(1.0, np.abs(want).max())


def test_cpu_model_matches_oracle():
    """libcpu_model.so: the oracle's model over the dispatched kernels."""
    CM = O.cpu_model_lib()
    sp = O.default_spec(**C1)
    ref = O.Checkpoint(sp)
    ref.convert(O.INT4, O.INT8)
    fast = O.Checkpoint(sp, L=CM)
    fast.convert(O.INT4, O.INT8)
    prompt = prompt_ids(16, C1["vocab_size"])
    want = O.Model(ref).forward(prompt)
    got = O.Model(fast).forward(prompt)
    err = np.abs(got - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
    assert O.Model(fast).greedy_decode(prompt, 16) == O.Model(ref).greedy_decode(prompt, 16)
