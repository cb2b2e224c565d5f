"""The MTP accept path, the draft head and the stop rule on the GPU, against
the CPU oracle (whose own pins are in tests/test_oracle_mtp.py).

- draft_logits (mtp.rs:74-133): with the identity MTP module of
  tests/models.py, the GPU's draft logits equal the oracle's (1e-3 max /
  1e-4 mean) and twice the GPU's own forward on the shifted sequence; on
  config 1's random model the native head's draft ids equal the oracle's
  wherever the top-2 gap exceeds 1e-3.
- the accept branch (mtp.rs:263-314): the identity module accepts most
  drafts natively at depth 1-3 (multi-row MTP feeds after accepts,
  chained drafts, partial rollbacks), with output equal to greedy and the
  drafted / accepted counts equal to the oracle's; caller drafts through the
  C ABI's draft callback run the reference's perfect-draft test
  (undertow-bench/tests/pipeline.rs:343-393) and every accept length.
- stop ids and on_token (core/model.rs:139-166): streams end where the
  oracle's end.
"""
import numpy as np
import pytest

from models import C1, C1_MLA, checkpoint, gpu_model, greedy_sim, identity_mtp_checkpoint, prompt_ids
from oracle import oracle as O

pytestmark = pytest.mark.gpu

# DeepSeek-V3 attention dims (matrix-core attention, int8 absorbs) at hidden
# 1024, one MoE layer plus the identity MTP module, int4 experts / int8 dense
IDENT_MLA = dict(C1_MLA, num_hidden_layers=1, first_k_dense_replace=0)


def gap_ok(logits):
    s = np.sort(logits, axis=-1)
    return (s[..., -1] - s[..., -2]) > 1e-3


@pytest.fixture(scope="module", params=["tiny_f32", "mla_int4"])
def ident(request, ctx):
    if request.param == "tiny_f32":
        ck = identity_mtp_checkpoint()
    else:
        ck = identity_mtp_checkpoint(IDENT_MLA, fmt="int4")
    return ck, gpu_model(ctx, ck), O.Model(ck)


def test_identity_draft_logits(ident):
    ck, m, om = ident
    V = ck.spec.vocab_size
    prompt = prompt_ids(9, V, seed=3)
    s, os_ = m.session(), om.session()
    s.prefill(prompt)
    os_.prefill(prompt)
    seq = list(prompt)
    nxt = 17
    for step in range(4):
        got, did = s.draft_logits(nxt)
        want, _ = os_.draft_logits(nxt)
        err = np.abs(got - want)
        assert err.max() <= 1e-3 and err.mean() <= 1e-4, (step, err.max(), err.mean())
        if gap_ok(want):
            assert did == int(np.argmax(want))
        shifted = m.forward(seq[1:] + [nxt])[-1] * np.float32(2.0)
        assert np.abs(got - shifted).max() <= 1e-4 * np.abs(shifted).max() + 1e-6, step
        s.prefill([nxt])
        os_.prefill([nxt])
        seq.append(nxt)
        nxt = (nxt * 7 + 3) % V


@pytest.mark.parametrize("depth", [1, 2, 3])
def test_identity_native_mtp_accepts(ident, depth):
    ck, m, om = ident
    prompt = prompt_ids(12, ck.spec.vocab_size, seed=5)
    greedy = m.generate_greedy(prompt, 24)
    assert greedy == om.greedy_decode(prompt, 24)[12:]
    toks, drafted, accepted = m.generate_mtp(prompt, 24, depth=depth)
    otoks, od, oa = om.speculative_loop(prompt, 24, depth=depth)
    assert toks == greedy == otoks
    assert accepted > 0
    assert (drafted, accepted) == (od, oa)


@pytest.fixture(scope="module")
def c1(ctx):
    ck = checkpoint(C1, fmt="int4")
    return ck, gpu_model(ctx, ck), O.Model(ck)


def test_c1_draft_ids_match_oracle(c1):
    """The native head on a random model: draft logits and ids along a
    stream, step by step, against the oracle."""
    ck, m, om = c1
    prompt = prompt_ids(16, C1["vocab_size"])
    stream = om.greedy_decode(prompt, 12)[16:]
    s, os_ = m.session(), om.session()
    s.prefill(prompt)
    os_.prefill(prompt)
    checked = 0
    for t in stream:
        got, did = s.draft_logits(t)
        want, _ = os_.draft_logits(t)
        err = np.abs(got - want)
        assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
        if gap_ok(want):
            assert did == int(np.argmax(want))
            checked += 1
        s.prefill([t])
        os_.prefill([t])
    assert checked >= len(stream) // 2


@pytest.mark.parametrize("depth", [1, 2, 3])
def test_perfect_and_wrong_drafts_through_callback(c1, depth):
    """pipeline.rs:343-393 through ut_speculative_loop's draft callback, then
    drafts made wrong at every position in turn."""
    ck, m, om = c1
    V = C1["vocab_size"]
    prompt = prompt_ids(16, V)
    max_new = 24
    stream = m.generate_greedy(prompt, max_new + 4)
    assert stream == om.greedy_decode(prompt, max_new + 4)[16:]

    def perfect(tokens, nxt, dep):
        k = len(tokens) - len(prompt)
        assert stream[k] == nxt and list(tokens[:16]) == prompt
        return stream[k + 1:k + 1 + dep]

    got = m.speculative_loop(prompt, max_new, depth=depth, draft_fn=perfect)
    assert got == om.speculative_loop(prompt, max_new, depth=depth, draft_fn=perfect)
    assert got == greedy_sim(stream, depth, lambda r: None, max_new)
    assert got[2] >= got[1] - (depth - 1) and got[1] > 0

    def wrong_factory():
        rounds = []

        def draft(tokens, nxt, dep):
            k = len(tokens) - len(prompt)
            d = list(stream[k + 1:k + 1 + dep])
            p = len(rounds) % (dep + 1)
            rounds.append(p)
            if p < dep:
                d[p] = (d[p] + 1) % V
            return d
        return draft

    got = m.speculative_loop(prompt, max_new, depth=depth, draft_fn=wrong_factory())
    assert got == om.speculative_loop(prompt, max_new, depth=depth, draft_fn=wrong_factory())
    assert got == greedy_sim(stream, depth, lambda r: r % (depth + 1), max_new)


@pytest.mark.parametrize("depth", [1, 3])
def test_verify_graph_replay_matches_eager(c1, ident, depth):
    """The MTP verify step (depth + 1 rows fed from the device ids) replayed
    from a captured graph, with the host's accept decision, rollbacks and
    position resets between the replays: caller drafts (perfect, then wrong
    at every position in turn) and native drafts on the identity module
    (which accepts most of them) give the eager streams and counts."""
    ck, m, om = c1
    V = C1["vocab_size"]
    prompt = prompt_ids(16, V)
    stream = m.generate_greedy(prompt, 28)

    def perfect(tokens, nxt, dep):
        k = len(tokens) - len(prompt)
        return stream[k + 1:k + 1 + dep]

    def wrong_factory():
        rounds = []

        def draft(tokens, nxt, dep):
            k = len(tokens) - len(prompt)
            d = list(stream[k + 1:k + 1 + dep])
            p = len(rounds) % (dep + 1)
            rounds.append(p)
            if p < dep:
                d[p] = (d[p] + 1) % V
            return d
        return draft

    ick, im, _ = ident
    iprompt = prompt_ids(9, ick.spec.vocab_size, seed=4)
    runs = [(m, lambda: m.speculative_loop(prompt, 24, depth=depth, draft_fn=perfect)),
            (m, lambda: m.speculative_loop(prompt, 24, depth=depth, draft_fn=wrong_factory())),
            (im, lambda: im.generate_mtp(iprompt, 20, depth=depth))]
    eager = [f() for _, f in runs]
    for mm, _ in runs:
        mm.enable_graphs(True)
    before = [mm.graph_stats() for mm, _ in runs]
    try:
        got = [f() for _, f in runs]
    finally:
        for mm, _ in runs:
            mm.enable_graphs(False)
    after = [mm.graph_stats() for mm, _ in runs]
    assert got == eager
    assert eager[2][2] > 0  # the identity module accepted native drafts
    for b, a in zip(before, after):
        assert a["failures"] == b["failures"]
    assert after[0]["replays"] - before[0]["replays"] > 0
    assert after[2]["replays"] - before[2]["replays"] > 0


def test_stop_ids_and_on_token(c1):
    ck, m, om = c1
    prompt = prompt_ids(16, C1["vocab_size"])
    stream = m.generate_greedy(prompt, 32)
    stop = stream[6]
    cut = stream.index(stop) + 1
    assert m.generate(prompt, 32, extra_stop_ids=[stop]) == om.generate(prompt, 32, stop_ids=[stop]) \
        == stream[:cut]
    seen = []
    assert m.generate(prompt, 32, on_token=lambda t: seen.append(t) or len(seen) < 5) == stream[:5]
    assert seen == stream[:5]
    # the model's own stop ids (DeepseekMoeModel::stop_ids) apply to every loop
    m.set_stop_ids([stop])
    try:
        assert m.generate_greedy(prompt, 32) == stream[:cut]
        for depth in (1, 3):
            toks, _, _ = m.generate_mtp(prompt, 32, depth=depth)
            assert toks == stream[:cut]

            def draft(tokens, nxt, dep, k0=len(prompt)):
                k = len(tokens) - k0
                return stream[k + 1:k + 1 + dep]

            toks, d, a = m.speculative_loop(prompt, 32, depth=depth, draft_fn=draft)
            otoks, od, oa = om.speculative_loop(prompt, 32, depth=depth, draft_fn=draft,
                                                stop_ids=[stop])
            assert toks == otoks == stream[:cut] and (d, a) == (od, oa) and a > 0
    finally:
        m.set_stop_ids([])


def test_draft_errors(c1):
    import undertow_amd as U
    ck, m, om = c1
    prompt = prompt_ids(16, C1["vocab_size"])
    with pytest.raises(U.UtError) as ei:
        m.speculative_loop(prompt, 8, depth=1, draft_fn=lambda t, n, d: [C1["vocab_size"]])
    assert ei.value.code == U.runtime.UT_ERR_BAD_TOKEN
    with pytest.raises(ZeroDivisionError):
        m.speculative_loop(prompt, 8, depth=2, draft_fn=lambda t, n, d: [1 // 0])
    s = m.session()
    s.prefill(prompt)
    s.draft_logits(3)
    with pytest.raises(U.UtError) as ei:
        s.draft_logits(3)  # nothing pending
    assert ei.value.code == U.runtime.UT_ERR_STATE


def test_long_prompt_first_draft(ctx):
    """A first MTP draft over more positions than the session's pinned id
    slot holds (16,376) goes through a staging buffer of its size."""
    ck = checkpoint(dict(max_position_embeddings=20000))
    m = gpu_model(ctx, ck)
    prompt = prompt_ids(16500, ck.spec.vocab_size, seed=13)
    toks, drafted, _ = m.generate_mtp(prompt, 4, depth=1)
    assert drafted > 0
    assert toks == m.generate_greedy(prompt, 4)


def _device_cfg(overrides):
    from undertow_amd.configs import C1 as DC1
    return dict(DC1, **overrides)


@pytest.mark.parametrize("over", [dict(num_hidden_layers=3),
                                  dict(num_hidden_layers=2, hidden_size=1024, num_attention_heads=128,
                                       kv_lora_rank=512, qk_nope_head_dim=128, qk_rope_head_dim=64,
                                       v_head_dim=128)],
                         ids=["c1_3layers", "mla_2layers"])
def test_restating_mtp_head_accepts_and_stays_lossless(ctx, over):
    """ut_model_synthesize_ex(UT_SYNTH_MTP_RESTATES): the MTP module restates
    the first MoE layer and the other layers' residual writes are damped,
    so the native head's drafts mostly match the verified tokens.  Greedy
    and MTP depth 1-3 emit the same stream (the verify keeps speculation
    lossless whatever the head predicts), the accept counts are consistent,
    and depth 1 accepts most drafts.  The flags are validated."""
    import undertow_amd as U
    cfg = _device_cfg(over)
    m = U.Model(ctx, cfg)
    m.synthesize(31, 0.02, U.INT4, U.INT8, mtp_restates=True)
    prompt = prompt_ids(24, cfg["vocab_size"], seed=8)
    greedy = m.generate_greedy(prompt, 48)
    for depth in (1, 2, 3):
        toks, drafted, accepted = m.generate_mtp(prompt, 48, depth=depth)
        assert toks == greedy, depth
        assert 0 <= accepted <= drafted and drafted > 0
        if depth == 1:
            assert accepted / drafted > 0.5, (accepted, drafted)
    plain = U.Model(ctx, cfg)
    plain.synthesize(31, 0.02, U.INT4, U.INT8)
    _, pd, pa = plain.generate_mtp(prompt, 48, depth=1)
    assert pa < accepted or pa / pd < 0.5
    bad = U.Model(ctx, cfg)
    with pytest.raises(U.UtError):
        bad.synthesize(31, 0.02, U.INT4, U.INT4, mtp_restates=True)
