"""The golden-stream harness on the CPU: the synthetic hybrid model
(tests/stream_model.py) with its mixers on the oracle reproduces the golden
token stream that the reference's own anchors produced
(tests/golden/stream_golden.json, written by tests/golden/make_stream.py),
token for token -- the model-level form of the oracle's bitwise pin."""
import json
import os

import numpy as np

import stream_model as sm

HERE = os.path.dirname(os.path.abspath(__file__))


def golden():
    with open(os.path.join(HERE, "golden", "stream_golden.json")) as f:
        g = json.load(f)
    g["prompts"] = [np.array(p, np.int64) for p in g["prompts"]]
    g["ids"] = np.array(g["ids"], np.int64)
    return g


def clear(g):
    """Per sequence: the steps before its first near-tie (top-1 minus top-2
    logit below near_tie), where a stream is decided by the model rather
    than by rounding noise."""
    return [int(c) for c in g["clear_prefix"]]


def test_stream_fixture_premise():
    """The fixture's clear prefixes agree with its margins, and are long
    enough to be a meaningful gate."""
    g = golden()
    mar = np.array(g["margins"])
    assert g["ids"].shape == mar.shape == (len(g["lens"]), g["n_new"])
    for s, c in enumerate(clear(g)):
        assert np.all(mar[s, :c] >= g["near_tie"])
        assert c == g["n_new"] or mar[s, c] < g["near_tie"]
    assert min(clear(g)) >= 16


def test_stream_oracle_reproduces_golden(orc):
    g = golden()
    model = sm.Model(g["model_seed"])
    ids, lg = sm.run_greedy(model, sm.OracleMixers(model, orc, len(g["lens"]), g["max_seq"]),
                            g["prompts"], g["n_new"])
    assert np.array_equal(ids, g["ids"])
    np.testing.assert_allclose(sm.margin(lg), g["margins"], atol=1e-4)
