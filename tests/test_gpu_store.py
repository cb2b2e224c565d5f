"""The HBM tier of the expert store (DiskExpertStore + ExpertCache with the
cache in device memory) against a resident model, after the reference's
pipeline tests (undertow-bench/tests/pipeline.rs:67-95, 253-292):

- a starvation-level budget gives logits bit-identical to the resident
  store, and a second identical forward re-reads nearly every expert;
- a hot-expert profile recorded on one run and pinned on the next removes
  every miss without changing the numerics;
- MTP generation, the weighted policy and pilot-router prefetch leave the
  token stream unchanged.
"""
import json

import numpy as np
import pytest

from models import C1, C1_E256, checkpoint, gpu_model, prompt_ids, write_converted

pytestmark = pytest.mark.gpu


def fresh(ctx, ck):
    import undertow_amd as U
    from models import CFG_KEYS
    return U.Model(ctx, {k: getattr(ck.spec, k) for k in CFG_KEYS})


@pytest.fixture(scope="module")
def c1dir(ctx, tmp_path_factory):
    ck = checkpoint(C1, fmt="int4")
    d = tmp_path_factory.mktemp("c1_int4")
    write_converted(ck, d, expert_layers=[1, 2])
    return ck, d, gpu_model(ctx, ck)


def expert_bytes(ck):
    H, I = ck.spec.hidden_size, ck.spec.moe_intermediate_size
    return 2 * I * (H // 2) + H * (I // 2) + (2 * I + H) * 4


def test_starved_cache_is_bit_identical_to_resident(ctx, c1dir, golden_dir):
    ck, d, resident = c1dir
    ref = json.loads((golden_dir / "oracle-tiny" / "reference.json").read_text())
    ids = [t % C1["vocab_size"] for t in ref["full_ids"]] + prompt_ids(12, C1["vocab_size"])
    starved = fresh(ctx, ck)
    starved.load_dir_tiered(d, hbm_budget_bytes=2 * expert_bytes(ck))
    a = resident.forward(ids)
    b = starved.forward(ids)
    assert np.array_equal(a, b), "storage tier must not affect numerics"
    first = starved.store_stats()
    assert first["misses"] > 10, first
    b2 = starved.forward(ids)
    assert np.array_equal(a, b2)
    second = starved.store_stats()
    refetched = second["misses"] - first["misses"]
    assert refetched >= 0.8 * first["misses"], (first, second)
    assert second["evictions"] > 0


def test_profile_pinning_eliminates_misses(ctx, c1dir):
    import undertow_amd as U
    ck, d, resident = c1dir
    ids = prompt_ids(24, C1["vocab_size"], seed=4)
    recorder = fresh(ctx, ck)
    recorder.load_dir_tiered(d, hbm_budget_bytes=1 << 30)
    baseline = recorder.forward(ids)
    usage = recorder.expert_usage()
    assert usage.sum() > 0
    prof = U.ExpertProfile.from_usage("deepseek_moe", usage)
    pinned = fresh(ctx, ck)
    pinned.load_dir_tiered(d, hbm_budget_bytes=1 << 30, policy=U.WEIGHTED)
    nbytes = pinned.pin_experts(prof.hottest(), 1 << 30)
    assert nbytes > 0
    logits = pinned.forward(ids)
    assert np.array_equal(logits, baseline), "pinning must not change numerics"
    st = pinned.store_stats()
    assert st["misses"] == 0 and st["hits"] > 0, st
    assert st["pinned_experts"] == len(prof.hottest())


def test_generation_through_the_store(ctx, tmp_path):
    """Three layers (two MoE, so decode has a next MoE layer to pilot-route)."""
    import undertow_amd as U
    cfg = dict(C1, num_hidden_layers=3)
    ck = checkpoint(cfg, fmt="int4")
    write_converted(ck, tmp_path, expert_layers=[1, 2, 3])
    resident = gpu_model(ctx, ck)
    prompt = prompt_ids(16, C1["vocab_size"])
    want = resident.generate_greedy(prompt, 24)
    for policy, prefetch in ((U.LRU, False), (U.WEIGHTED, True)):
        m = fresh(ctx, ck)
        m.load_dir_tiered(tmp_path, hbm_budget_bytes=3 * expert_bytes(ck), policy=policy,
                          prefetch=prefetch)
        assert m.generate_greedy(prompt, 24) == want
        assert m.generate_mtp(prompt, 24, depth=2)[0] == want
        st = m.store_stats()
        assert st["misses"] > 0
        if prefetch:
            assert st["prefetch_issued"] > 0, st


def test_deepseek_router_shape_through_the_store(ctx, tmp_path):
    """256 experts, 8 groups, top-8 at hidden 256: a quarter of the experts
    fit the budget."""
    ck = checkpoint(C1_E256, fmt="int4")
    write_converted(ck, tmp_path, expert_layers=[1, 2])
    resident = gpu_model(ctx, ck)
    m = fresh(ctx, ck)
    m.load_dir_tiered(tmp_path, hbm_budget_bytes=64 * expert_bytes(ck), prefetch=True)
    prompt = prompt_ids(16, C1_E256["vocab_size"])
    assert np.array_equal(m.forward(prompt), resident.forward(prompt))
    assert m.generate_mtp(prompt, 16, depth=1) == resident.generate_mtp(prompt, 16, depth=1)


def test_missing_expert_shard_is_reported(ctx, tmp_path):
    import undertow_amd as U
    ck = checkpoint(C1, fmt="int4")
    write_converted(ck, tmp_path, expert_layers=[1, 2])
    (tmp_path / "experts-00002.safetensors").unlink()
    with pytest.raises(U.UtError) as ei:
        fresh(ctx, ck).load_dir_tiered(tmp_path, hbm_budget_bytes=1 << 20)
    assert ei.value.code == U.runtime.UT_ERR_IO


def test_synthesized_model_with_a_host_pool(ctx):
    """ut_model_synthesize_tiered: dense weights on the device, routed
    experts from a pinned host pool behind a three-expert budget."""
    import undertow_amd as U
    cfg = dict(C1, num_hidden_layers=3)
    ck = checkpoint(cfg, fmt="int4")
    m = fresh(ctx, ck)
    m.synthesize_tiered(7, hbm_budget_bytes=3 * expert_bytes(ck), host_pool_experts=5,
                        prefetch=True)
    prompt = prompt_ids(16, C1["vocab_size"])
    toks = m.generate_greedy(prompt, 16)
    assert len(toks) == 16
    assert m.generate_mtp(prompt, 16, depth=1)[0] == toks
    st = m.store_stats()
    assert st["misses"] > 0 and st["hits"] > 0 and st["bytes_read"] > 0
    usage = m.expert_usage()
    assert usage.shape == (4, 8) and usage[0].sum() == 0 and usage[1:].sum() > 0
    prof = U.ExpertProfile.from_usage("deepseek_moe", usage)
    assert prof.counts[0][2] == usage.max()
