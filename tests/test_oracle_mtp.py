"""The oracle's MTP draft head and speculative loop, pinned on the CPU.

draft_logits (mtp.rs:74-133) is pinned by construction: with the identity
MTP module of tests/models.py the draft logits at every pending position
equal twice the main model's logits on the sequence shifted by one token.
The speculative loop's accept branch (mtp.rs:263-314) is pinned by the
reference's perfect-draft test (undertow-bench/tests/pipeline.rs:343-393)
and, at depth 2-3, by drafts made wrong at a chosen position: every accept
length and every rollback length runs, and the emitted stream and counts
follow from the greedy sequence alone.  Stop ids and on_token follow
undertow_core::generate (core/model.rs:139-166).
"""
import numpy as np
import pytest

from models import C1, checkpoint, greedy_sim, identity_mtp_checkpoint, prompt_ids
from oracle import oracle as O


@pytest.fixture(scope="module")
def ident():
    ck = identity_mtp_checkpoint()
    return ck, O.Model(ck)


def test_identity_draft_logits_equal_shifted_forward(ident):
    ck, om = ident
    V = ck.spec.vocab_size
    prompt = prompt_ids(9, V, seed=3)
    s = om.session()
    s.prefill(prompt)
    seq = list(prompt)
    nxt = 17
    for step in range(4):
        # pending: the whole prompt first, then one position per step
        dl, _ = s.draft_logits(nxt)
        want = om.forward(seq[1:] + [nxt])[-1] * np.float32(2.0)
        tol = 1e-5 * np.abs(want).max()
        assert np.abs(dl - want).max() <= tol, (step, np.abs(dl - want).max(), tol)
        s.prefill([nxt])
        seq.append(nxt)
        nxt = (nxt * 7 + 3) % V


def test_identity_construction_detects_plausible_mistakes(ident):
    """The same comparison fails for the plausible mistakes: the unshifted
    sequence (t_next = tokens[i]), the main head's scale, and a feed that
    skips the pending prompt rows."""
    ck, om = ident
    V = ck.spec.vocab_size
    prompt = prompt_ids(9, V, seed=3)
    s = om.session()
    s.prefill(prompt)
    dl, _ = s.draft_logits(17)
    good = om.forward(prompt[1:] + [17])[-1] * np.float32(2.0)
    tol = 1e-5 * np.abs(good).max()
    assert np.abs(dl - good).max() <= tol
    for bad in (om.forward(prompt)[-1] * np.float32(2.0),          # unshifted tokens
                om.forward(prompt[1:] + [17])[-1],                  # main head's scale
                om.forward([17])[-1] * np.float32(2.0)):            # context not fed
        assert np.abs(dl - bad).max() > 100 * tol


def test_identity_native_mtp_accepts_and_is_lossless(ident):
    ck, om = ident
    prompt = prompt_ids(12, ck.spec.vocab_size, seed=5)
    greedy = om.greedy_decode(prompt, 24)[12:]
    for depth in (1, 2, 3):
        toks, drafted, accepted = om.speculative_loop(prompt, 24, depth=depth)
        assert toks == greedy
        assert drafted > 0 and accepted > 0, (depth, drafted, accepted)


@pytest.fixture(scope="module")
def c1o():
    ck = checkpoint(C1, fmt="int4")
    return ck, O.Model(ck)


@pytest.mark.parametrize("depth", [1, 2, 3])
def test_perfect_drafts_all_accept(c1o, depth):
    """pipeline.rs:343-393 at depth 1, extended to 2-3 draft tokens."""
    ck, om = c1o
    prompt = prompt_ids(16, C1["vocab_size"])
    max_new = 20
    stream = om.greedy_decode(prompt, max_new + 4)[16:]

    def draft(tokens, nxt, dep):
        k = len(tokens) - len(prompt)
        assert stream[k] == nxt and list(tokens[:16]) == prompt
        return stream[k + 1:k + 1 + dep]

    toks, drafted, accepted = om.speculative_loop(prompt, max_new, depth=depth, draft_fn=draft)
    assert toks == stream[:max_new]
    # every draft is accepted; a run cut by max_new leaves its tail unused
    assert drafted > 0 and drafted - (depth - 1) <= accepted <= drafted
    if depth == 1:
        assert accepted == drafted
    assert (toks, drafted, accepted) == greedy_sim(stream, depth, lambda r: None, max_new)


@pytest.mark.parametrize("depth", [2, 3])
def test_wrong_drafts_every_accept_length(c1o, depth):
    ck, om = c1o
    prompt = prompt_ids(16, C1["vocab_size"])
    V, max_new = C1["vocab_size"], 24
    stream = om.greedy_decode(prompt, max_new + 4)[16:]
    rounds = []

    def corrupt_at(r):
        return r % (depth + 1)  # 0..depth-1: wrong there; depth: all right

    def draft(tokens, nxt, dep):
        k = len(tokens) - len(prompt)
        d = list(stream[k + 1:k + 1 + dep])
        p = corrupt_at(len(rounds))
        rounds.append(p)
        if p < dep:
            d[p] = (d[p] + 1) % V
        return d

    toks, drafted, accepted = om.speculative_loop(prompt, max_new, depth=depth, draft_fn=draft)
    assert toks == stream[:max_new]
    assert (toks, drafted, accepted) == greedy_sim(stream, depth, corrupt_at, max_new)
    assert set(rounds) == set(range(depth + 1))


def test_stop_ids_and_on_token(c1o):
    """core/model.rs:139-166: a stop token is emitted and ends the stream;
    on_token returning False ends it after that token."""
    ck, om = c1o
    prompt = prompt_ids(16, C1["vocab_size"])
    stream = om.greedy_decode(prompt, 32)[16:]
    stop = stream[6]
    cut = stream.index(stop) + 1
    assert om.generate(prompt, 32, stop_ids=[stop]) == stream[:cut]
    seen = []
    assert om.generate(prompt, 32, on_token=lambda t: seen.append(t) or len(seen) < 5) == stream[:5]
    assert seen == stream[:5]
    for depth in (1, 3):
        toks, _, _ = om.speculative_loop(prompt, 32, depth=depth, stop_ids=[stop])
        assert toks == stream[:cut]

        def draft(tokens, nxt, dep, k0=len(prompt)):
            k = len(tokens) - k0
            return stream[k + 1:k + 1 + dep]

        toks, d, a = om.speculative_loop(prompt, 32, depth=depth, draft_fn=draft, stop_ids=[stop])
        assert toks == stream[:cut] and a > 0
