"""The decode step end to end on the GPU: the reference's transformers golden
(oracle-tiny), BASELINE config 1 against the CPU oracle, greedy and MTP streams.

Bars: logits within 1e-3 max-abs and 1e-4 mean-abs of
the oracle; argmax exact wherever the top-2 gap exceeds 1e-3; greedy token
streams identical; MTP output identical to plain greedy (mtp.rs losslessness,
undertow-bench/tests/pipeline.rs:298-338).
"""
import json

import numpy as np
import pytest

from models import C1, C1_E256, C1_MLA, C1_MLA_V40, checkpoint, gpu_model, prompt_ids
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def gap_ok(logits):
    s = np.sort(logits, axis=-1)
    return (s[..., -1] - s[..., -2]) > 1e-3


@pytest.fixture(scope="module")
def ref(golden_dir):
    return json.loads((golden_dir / "oracle-tiny" / "reference.json").read_text())


def test_tiny_f32_matches_transformers_golden(ctx, ref):
    """undertow-bench/tests/oracle.rs:47-84 against the GPU path."""
    m = gpu_model(ctx, checkpoint())
    logits = m.forward(ref["full_ids"])
    tl = np.asarray(ref["tf_logits"], np.float32)
    err = np.abs(logits - tl)
    assert err.max() < 1e-3, err.max()
    assert logits.argmax(1).tolist() == ref["tf_pred"]
    max_new = len(ref["full_ids"]) - len(ref["prompt_ids"])
    assert ref["prompt_ids"] + m.generate_greedy(ref["prompt_ids"], max_new) == ref["full_ids"]


@pytest.mark.parametrize("fmt", ["f32", "int8", "int4"])
def test_tiny_matches_oracle(ctx, ref, fmt):
    ck = checkpoint(fmt=fmt)
    m = gpu_model(ctx, ck)
    om = O.Model(ck)
    ids = ref["full_ids"]
    got = m.forward(ids)
    want = om.forward(ids)
    err = np.abs(got - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
    ok = gap_ok(want)
    assert (got.argmax(1)[ok] == want.argmax(1)[ok]).all()
    assert m.generate_greedy(ref["prompt_ids"], 16) == om.greedy_decode(ref["prompt_ids"], 16)[len(ref["prompt_ids"]):]


@pytest.fixture(scope="module")
def c1(ctx):
    ck = checkpoint(C1, fmt="int4")
    return ck, gpu_model(ctx, ck), O.Model(ck)


def test_c1_logits_match_oracle(c1):
    ck, m, om = c1
    prompt = prompt_ids(16, C1["vocab_size"])
    got, want = m.forward(prompt), om.forward(prompt)
    err = np.abs(got - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
    ok = gap_ok(want)
    assert (got.argmax(1)[ok] == want.argmax(1)[ok]).all()


def test_c1_greedy_stream_identical(c1):
    ck, m, om = c1
    prompt = prompt_ids(16, C1["vocab_size"])
    want = om.greedy_decode(prompt, 64)[16:]
    assert m.generate_greedy(prompt, 64) == want


@pytest.fixture(scope="module")
def c1_mla(ctx):
    ck = checkpoint(C1_MLA, fmt="int4")
    return ck, gpu_model(ctx, ck), O.Model(ck)


def test_c1_mla_shape_logits_and_stream(c1_mla):
    """DeepSeek-V3 attention dims end to end: int8 kv_b absorbs, split-cache
    matrix-core attention, against the oracle's sequential f32 loops."""
    ck, m, om = c1_mla
    prompt = prompt_ids(16, C1_MLA["vocab_size"])
    got, want = m.forward(prompt), om.forward(prompt)
    err = np.abs(got - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
    ok = gap_ok(want)
    assert (got.argmax(1)[ok] == want.argmax(1)[ok]).all()
    assert m.generate_greedy(prompt, 16) == om.greedy_decode(prompt, 16)[16:]


@pytest.mark.parametrize("depth", [1, 2, 3])
def test_c1_mla_mtp_verify_rows(c1_mla, depth):
    """Verify steps of 2, 3 and 4 rows at hidden 1024 (the matrix-core
    expert kernels take 3 and 4 rows, beside the shared expert's own
    launches): the MTP stream equals greedy decode and the oracle's."""
    ck, m, om = c1_mla
    prompt = prompt_ids(16, C1_MLA["vocab_size"])
    toks, drafted, accepted = m.generate_mtp(prompt, 16, depth=depth)
    assert toks == m.generate_greedy(prompt, 16) == om.greedy_decode(prompt, 16)[16:]
    assert drafted > 0 and 0 <= accepted <= drafted


def test_c1_mla_value_head_tail(ctx):
    """A 40-dim value head (not a multiple of the absorbed V's 16 rows per
    workgroup): logits against the oracle, and one-row decode, two- and
    four-row verify streams equal to the oracle's greedy stream."""
    ck = checkpoint(C1_MLA_V40, fmt="int4")
    m, om = gpu_model(ctx, ck), O.Model(ck)
    prompt = prompt_ids(16, C1_MLA_V40["vocab_size"], seed=5)
    got, want = m.forward(prompt), om.forward(prompt)
    err = np.abs(got - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
    stream = om.greedy_decode(prompt, 12)[16:]
    assert m.generate_greedy(prompt, 12) == stream
    for depth in (1, 3):
        toks, drafted, accepted = m.generate_mtp(prompt, 12, depth=depth)
        assert toks == stream and drafted > 0


@pytest.mark.parametrize("which", ["c1", "c1_mla"])
def test_graph_replay_matches_eager(request, which):
    """One-row greedy steps replayed from a captured graph (every position
    read from device memory, attention grids sized for the capacity) give
    the eager stream token for token, over 45 replays with the host's
    readbacks and waits between them; a second call captures its own
    session's graph.  c1 takes the f32 split-T attention, c1_mla the
    matrix-core attention with the fused q_a/kv_a finish."""
    ck, m, om = request.getfixturevalue(which)
    cfg = C1 if which == "c1" else C1_MLA
    prompt = prompt_ids(16, cfg["vocab_size"])
    eager = m.generate_greedy(prompt, 48)
    eager2 = m.generate_greedy(prompt[:9], 40)
    before = m.graph_stats()
    m.enable_graphs(True)
    try:
        g1 = m.generate_greedy(prompt, 48)
        g2 = m.generate_greedy(prompt[:9], 40)
    finally:
        m.enable_graphs(False)
    after = m.graph_stats()
    assert g1 == eager
    assert g2 == eager2
    # the replays ran: one capture per call, every step from the third on
    assert after["failures"] == before["failures"]
    assert after["captures"] - before["captures"] == 2
    assert after["replays"] - before["replays"] == (48 - 3) + (40 - 3)
    assert eager == om.greedy_decode(prompt, 48)[16:]


@pytest.fixture(scope="module")
def c1_e256(ctx):
    ck = checkpoint(C1_E256, fmt="int4")
    return ck, gpu_model(ctx, ck), O.Model(ck)


def test_c1_deepseek_router_logits_stream_and_mtp(c1_e256):
    """256 experts, 8 groups, top-8: prefill (4-row chunks), decode (1 row)
    and MTP verify (2 rows) route inside the expert launch."""
    ck, m, om = c1_e256
    prompt = prompt_ids(16, C1_E256["vocab_size"])
    got, want = m.forward(prompt), om.forward(prompt)
    err = np.abs(got - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
    ok = gap_ok(want)
    assert (got.argmax(1)[ok] == want.argmax(1)[ok]).all()
    stream = om.greedy_decode(prompt, 32)[16:]
    assert m.generate_greedy(prompt, 32) == stream
    toks, drafted, accepted = m.generate_mtp(prompt, 32, depth=1)
    assert toks == stream and drafted > 0


def test_c1_mtp_matches_oracle_and_greedy(c1):
    ck, m, om = c1
    prompt = prompt_ids(16, C1["vocab_size"])
    toks, drafted, accepted = m.generate_mtp(prompt, 64, depth=1)
    otoks, od, oa = om.generate_mtp(prompt, 64)
    assert toks == otoks == m.generate_greedy(prompt, 64)
    assert (drafted, accepted) == (od, oa)


@pytest.mark.parametrize("depth", [2, 3])
def test_c1_mtp_deeper_drafts_are_lossless(c1, depth):
    ck, m, om = c1
    prompt = prompt_ids(16, C1["vocab_size"])
    toks, drafted, accepted = m.generate_mtp(prompt, 48, depth=depth)
    assert toks == m.generate_greedy(prompt, 48)
    assert drafted > 0 and 0 <= accepted <= drafted


def test_incremental_decode_matches_one_shot(c1):
    """pipeline.rs:100-136: incremental == full prefill (argmax exact, < 1e-3)."""
    ck, m, om = c1
    ids = prompt_ids(24, C1["vocab_size"], seed=9)
    full = m.forward(ids)
    s = m.session()
    inc = [s.prefill(ids[:10])[-1]]
    for t in ids[10:]:
        inc.append(s.decode(t))
    inc = np.stack(inc)
    assert np.abs(inc - full[9:]).max() < 1e-3
    assert (inc.argmax(1) == full[9:].argmax(1)).all()


def test_truncate_then_refill_matches(c1):
    """pipeline.rs:200-223."""
    ck, m, om = c1
    ids = prompt_ids(20, C1["vocab_size"], seed=11)
    s = m.session()
    a = s.prefill(ids)
    s.truncate(12)
    assert s.position == 12
    b = s.prefill(ids[12:])
    assert np.array_equal(a[12:], b)


def test_context_overflow_and_bad_token(ctx):
    import undertow_amd as U
    ck = checkpoint({"max_position_embeddings": 32})
    m = gpu_model(ctx, ck)
    s = m.session()
    s.prefill(list(range(30)))
    with pytest.raises(U.ContextOverflow):
        s.prefill([1, 2, 3])
    with pytest.raises(U.UtError) as ei:
        m.session().prefill([5, 999999])
    assert ei.value.code == U.runtime.UT_ERR_BAD_TOKEN
    # generation stops cleanly at the context end (pipeline.rs:450-459)
    out = m.generate_greedy(list(range(28)), 10)
    assert len(out) == 5


def test_handles_release_in_any_order():
    """Sessions keep their model and models their context alive, so handles
    can be released in any order (Python finalizers of a reference cycle)."""
    import undertow_amd as U
    c = U.Context(0)
    m = gpu_model(c, checkpoint())
    s = m.session()
    L = U.lib()
    L.ut_model_free(m._h)
    m._h = None
    L.ut_ctx_destroy(c._h)
    c._h = None
    logits = s.prefill([1, 2, 3])  # model and context are still alive
    assert np.isfinite(logits).all()
    s._release()


@pytest.mark.parametrize("inter", [96, 160])
def test_shared_mlp_beside_matrix_core_experts_row_tail(ctx, inter):
    """Hidden 512 with expert widths of 96 and 160 (I % 64 == 32): prefill
    chunks and MTP verify steps of 2-4 rows run the routed experts on the
    matrix cores with the shared MLP in the same launches, whose last
    workgroups end past I.  Logits within the model bar of the oracle and
    MTP depth 1-3 equal to greedy."""
    cfg = dict(C1, hidden_size=512, moe_intermediate_size=inter)
    ck = checkpoint(cfg, fmt="int4")
    m, om = gpu_model(ctx, ck), O.Model(ck)
    prompt = prompt_ids(11, C1["vocab_size"], seed=3)
    got, want = m.forward(prompt), om.forward(prompt)
    err = np.abs(got - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
    ok = gap_ok(want)
    assert (got.argmax(1)[ok] == want.argmax(1)[ok]).all()
    greedy = m.generate_greedy(prompt, 12)
    assert greedy == om.greedy_decode(prompt, 12)[len(prompt):]
    for depth in (1, 2, 3):
        assert m.generate_mtp(prompt, 12, depth=depth)[0] == greedy, depth


def test_concurrent_sessions_are_isolated(ctx, ref):
    """Sessions on four threads, each on its own context (stream, scratch,
    staging), share one resident model and run three forwards each with
    logits bit-identical to a forward on the model's own context
    (undertow-bench/tests/pipeline.rs:226-249)."""
    import threading
    import undertow_amd as U
    ck = checkpoint(C1, fmt="int4")
    m = gpu_model(ctx, ck)
    ids = [t % C1["vocab_size"] for t in ref["full_ids"]] + prompt_ids(12, C1["vocab_size"])
    want = m.forward(ids)
    ctxs = [U.Context(0, bind_torch_stream=False) for _ in range(4)]
    errors = []

    def worker(c):
        try:
            for _ in range(3):
                got = m.session(ctx=c).prefill(ids)
                if not np.array_equal(got, want):
                    errors.append(float(np.abs(got - want).max()))
        except Exception as e:  # reported below, on the main thread
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(c,)) for c in ctxs]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


def test_kv_budget_lowers_effective_context(ctx):
    """LoadOptions::kv_budget_bytes shrinks the usable context
    (loader.rs:311-325); a forward past the lowered bound is a typed
    overflow naming it, and forwards within it work
    (undertow-bench/tests/pipeline.rs:463-483)."""
    import undertow_amd as U
    ck = checkpoint(C1, fmt="int4")
    m = gpu_model(ctx, ck)
    full = m.max_context
    assert full == ck.spec.max_position_embeddings
    m.set_kv_budget(16 * 1024)
    s = ck.spec
    per = s.num_hidden_layers * (s.kv_lora_rank + s.qk_rope_head_dim) * 4 + s.hidden_size * 4 + 8
    eff = m.max_context
    assert eff == min(full, max(16 * 1024 // per, 1)) and eff < full
    long = [i % s.vocab_size for i in range(eff + 1)]
    with pytest.raises(U.ContextOverflow) as ei:
        m.forward(long)
    assert ei.value.code == U.runtime.UT_ERR_CONTEXT_OVERFLOW and f"> {eff}" in str(ei.value)
    a = m.forward(long[:min(eff, 8)])
    m.set_kv_budget(None)
    assert m.max_context == full
    assert np.array_equal(a, m.forward(long[:min(eff, 8)]))
    # a greedy stream stops at the lowered window
    m.set_kv_budget(16 * 1024)
    assert len(m.generate_greedy(long[:eff - 2], 50)) <= 3
    with pytest.raises(U.UtError):
        m.set_kv_budget(0)


@pytest.mark.parametrize("fmt,floor,min_prefix", [("int8", 0.85, 6), ("int4", 0.55, 3)])
def test_quantized_agreement_floors(ctx, ref, fmt, floor, min_prefix):
    """pipeline.rs:137-177 on the GPU: the converted oracle-tiny fixture
    keeps the reference's teacher-forcing agreement and greedy-prefix
    floors against the transformers golden."""
    from test_oracle_quant_agreement import agreement
    m = gpu_model(ctx, checkpoint(fmt=fmt))
    max_new = len(ref["full_ids"]) - len(ref["prompt_ids"])
    rate, prefix = agreement(ref, m.forward(ref["full_ids"]),
                             m.generate_greedy(ref["prompt_ids"], max_new))
    assert rate >= floor, (fmt, rate)
    assert prefix >= min_prefix, (fmt, prefix)


@pytest.mark.parametrize("fmt,cfg", [("int8", None), ("int4", C1)], ids=["tiny_int8", "c1_int4"])
def test_fast_int8_mode_in_the_model(ctx, ref, fmt, cfg):
    """ut_set_fast_int8 reaches every int8 matmul of the model, as the
    reference's process-global switch reaches every int8 QTensor::matmul
    (undertow-quant/src/lib.rs:35-59, qtensor.rs:385-398).  This backend
    runs the absorbed attention for every path, where kv_b goes through
    matvec_rows / add_scaled_row (exact in the reference too), so the bar is
    the oracle's absorbed path (session path 1) under its switch: logits
    within the model bar, greedy decode identical.  The reference's quality
    gate holds on the int8 fixture (undertow-bench/tests/fast_int8.rs:24-61:
    teacher-forcing agreement >= 0.75), and switching off restores the exact
    path bit for bit."""
    ck = checkpoint(cfg, fmt=fmt)
    m = gpu_model(ctx, ck)
    om = O.Model(ck)
    ids = ref["full_ids"] if cfg is None else prompt_ids(16, C1["vocab_size"])
    exact = m.forward(ids)
    ctx.set_fast_int8(True)
    O.set_fast_int8(True)
    try:
        got = m.forward(ids)
        want = om.session(path=1).prefill(ids)
        prompt = ids[:12]
        stream = m.generate_greedy(prompt, 12)
        os_ = om.session(path=1)
        nxt = int(os_.prefill(prompt)[-1].argmax())
        ostream = [nxt]
        while len(ostream) < 12:
            nxt = int(os_.decode(nxt).argmax())
            ostream.append(nxt)
    finally:
        ctx.set_fast_int8(False)
        O.set_fast_int8(False)
    err = np.abs(got - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
    assert stream == ostream
    assert not np.array_equal(got, exact)
    if cfg is None:
        agree = np.mean([int(got[s].argmax()) == ref["tf_pred"][s] for s in range(len(ids))])
        assert agree >= 0.75, agree
    assert np.array_equal(m.forward(ids), exact)
