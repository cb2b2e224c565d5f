"""BASELINE config 5 at full shape: DeepSeek-V3 671B's 61 layers (the first
3 dense, 58 MoE plus the MTP module's MoE layer), 256 routed experts top-8 at
hidden 7168 and expert width 2048, int4 experts behind the HBM tier of the
expert store, int8 dense weights in HBM (ut_model_synthesize_tiered: dense
weights synthesized on the device, the routed experts served from a small
pinned host pool).  The reference's pipeline invariants, checked at this
shape as properties (no CPU oracle runs a 671B-shaped model):

- a starvation-level expert budget gives logits bit-identical to a roomy
  one, and a second identical forward re-reads nearly every expert
  (undertow-bench/tests/pipeline.rs:67-95);
- a profile recorded on one run and pinned on the next removes every miss
  without changing the numerics (pipeline.rs:253-292);
- MTP speculation on the starved store emits exactly the greedy stream
  (pipeline.rs:298-338).
"""
import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

PROMPT = 8
NEW = 16
POOL = 32          # pinned host pool entries (22 MB each)
ROOMY = 96 << 30   # every expert an 8-token prompt routes to fits
STARVED = 3 << 30  # about 140 slots for 59 MoE layers x 8+ experts per row


def c5_cfg():
    from undertow_amd.configs import C5
    return dict(C5, max_position_embeddings=64)


def slot_bytes(cfg):
    H, I = cfg["hidden_size"], cfg["moe_intermediate_size"]
    return 2 * I * (H // 2) + H * (I // 2) + (2 * I + H) * 4


def make(ctx, budget, policy=None):
    import undertow_amd as U
    m = U.Model(ctx, c5_cfg())
    m.synthesize_tiered(1905, budget, POOL, policy=U.LRU if policy is None else policy)
    return m


@pytest.fixture(scope="module")
def c5_prompt():
    from models import prompt_ids
    return prompt_ids(PROMPT, c5_cfg()["vocab_size"], seed=55)


@pytest.fixture(scope="module")
def recorded(ctx, c5_prompt):
    """The roomy run: logits of the prompt and its routing profile."""
    print("config 5: roomy store, recording", flush=True)
    m = make(ctx, ROOMY)
    logits = m.forward(c5_prompt)
    st = m.store_stats()
    again = m.forward(c5_prompt)
    st2 = m.store_stats()
    usage = m.expert_usage()
    del m
    return logits, st, again, st2, usage


def test_c5_roomy_store_holds_the_working_set(recorded):
    logits, st, again, st2, usage = recorded
    cfg = c5_cfg()
    assert np.isfinite(logits).all() and logits.shape == (PROMPT, cfg["vocab_size"])
    assert np.array_equal(again, logits)
    assert st["misses"] > 0 and st["bytes_read"] == st["misses"] * slot_bytes(cfg), st
    # the second pass finds every expert it needs in HBM
    assert st2["misses"] == st["misses"] and st2["evictions"] == 0, (st, st2)
    L = cfg["num_hidden_layers"] + 1
    assert usage.shape == (L, cfg["n_routed_experts"])
    # dense layers route nothing; forward() runs every MoE layer and not
    # the MTP module's (its last row)
    assert usage[:cfg["first_k_dense_replace"]].sum() == 0 and usage[-1].sum() == 0
    assert (usage[cfg["first_k_dense_replace"]:-1].sum(1) > 0).all()


def test_c5_starved_store_is_bit_identical(ctx, c5_prompt, recorded):
    want = recorded[0]
    print("config 5: starved store", flush=True)
    m = make(ctx, STARVED)
    got = m.forward(c5_prompt)
    assert np.array_equal(got, want), "storage tier must not affect numerics"
    first = m.store_stats()
    assert first["misses"] > 20 and first["evictions"] > 0, first
    got2 = m.forward(c5_prompt)
    assert np.array_equal(got2, want)
    second = m.store_stats()
    refetched = second["misses"] - first["misses"]
    assert refetched >= 0.8 * first["misses"], (first, second)
    print("config 5: starved greedy and MTP-1", flush=True)
    greedy = m.generate_greedy(c5_prompt, NEW)
    toks, drafted, accepted = m.generate_mtp(c5_prompt, NEW, depth=1)
    assert toks == greedy and drafted > 0
    assert m.store_stats()["misses"] > second["misses"]


def test_c5_pinned_profile_removes_misses(ctx, c5_prompt, recorded):
    import undertow_amd as U
    want, usage = recorded[0], recorded[4]
    prof = U.ExpertProfile.from_usage("deepseek_v3", usage)
    keys = prof.hottest()
    print(f"config 5: pinning {len(keys)} experts", flush=True)
    m = make(ctx, ROOMY, policy=U.WEIGHTED)
    nbytes = m.pin_experts(keys, ROOMY)
    assert nbytes == len(keys) * slot_bytes(c5_cfg())
    got = m.forward(c5_prompt)
    assert np.array_equal(got, want), "pinning must not change numerics"
    st = m.store_stats()
    assert st["misses"] == 0 and st["hits"] > 0, st
    assert st["pinned_experts"] == len(keys)
