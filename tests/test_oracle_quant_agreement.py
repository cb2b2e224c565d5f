"""Quantized checkpoints stay close to the f32 reference: the reference's
floors (undertow-bench/tests/pipeline.rs:137-177) on the oracle.  The
oracle-tiny fixture converted to int8 experts + int8 dense keeps >= 85 % of
the transformers golden's teacher-forcing argmax decisions and a greedy
prefix of >= 6 tokens; int4 experts + int8 dense >= 55 % and >= 3.  A
conversion or kernel mistake (a wrong scale, a nibble order swap) takes
these to near zero."""
import json

import pytest

from models import checkpoint
from oracle import oracle as O

CASES = [("int8", 0.85, 6), ("int4", 0.55, 3)]


def agreement(ref, logits, greedy):
    ids = ref["full_ids"]
    rate = sum(int(logits[s].argmax()) == ref["tf_pred"][s] for s in range(len(ids))) / len(ids)
    p = len(ref["prompt_ids"])
    prefix = 0
    for a, b in zip(ref["prompt_ids"] + greedy, ids):
        if a != b:
            break
        prefix += 1
    return rate, prefix - p


@pytest.fixture(scope="module")
def ref(golden_dir):
    return json.loads((golden_dir / "oracle-tiny" / "reference.json").read_text())


@pytest.mark.parametrize("fmt,floor,min_prefix", CASES)
def test_oracle_quantized_agreement_floors(ref, fmt, floor, min_prefix):
    om = O.Model(checkpoint(fmt=fmt))
    max_new = len(ref["full_ids"]) - len(ref["prompt_ids"])
    greedy = om.greedy_decode(ref["prompt_ids"], max_new)[len(ref["prompt_ids"]):]
    rate, prefix = agreement(ref, om.forward(ref["full_ids"]), greedy)
    assert rate >= floor, (fmt, rate)
    assert prefix >= min_prefix, (fmt, prefix, greedy)
