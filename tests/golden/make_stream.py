"""Write tests/golden/stream_golden.json: the golden token stream of the
synthetic hybrid model (tests/stream_model.py) with its mixers on the
reference's own scalar anchors (c/gdn.h, c/attn.h wired as c/layer.h by
oracle/ref_shim.c, built by `make -C oracle ref`).

This mirrors the reference's standing golden (tests/m11/README.md: a short
prompt, 24 greedy tokens, reproduced exactly): three prompts of 15, 100
and 37 tokens prefilled as one ragged batch, then 24 greedy tokens each.
A step whose top-1 minus top-2 logit is below NEAR_TIE is a near-tie: any
change in the summation order of a mixer moves some bf16 mixer input by an
ulp, and the model's logits then move by up to ~0.005 (measured by flipping
random ulps of the mixer outputs), so past a near-tie the stream is a
function of rounding noise rather than of the model. NEAR_TIE is four
times that noise. The prompt seed is the one among the first SEEDS whose
three streams run longest before their first near-tie (the shortest of the
three counts); the ids and every step's margin are stored, and the GPU
tests compare streams up to each sequence's first near-tie and, teacher
forced, at every step that is not one.

Run in the build container only (the reference is not present on GPU
hosts):  python tests/golden/make_stream.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "apus-qwen3.6-35b-a3b_amd"),
                os.path.dirname(HERE)]

import oracle        # noqa: E402
import stream_model as sm  # noqa: E402

LENS = (15, 100, 37)
N_NEW = 24
NEAR_TIE = 0.02
SEEDS = 40
MAX_SEQ = 160


def prompts_for(seed):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, sm.V, n).astype(np.int64) for n in LENS]


def clear_prefix(mar):
    """Per sequence: the number of steps before the first near-tie."""
    return [int(np.argmax(m < NEAR_TIE)) if (m < NEAR_TIE).any() else len(m) for m in mar]


def main():
    ref = oracle.Reference()
    model = sm.Model()
    best = None
    for seed in range(1, SEEDS + 1):
        prompts = prompts_for(seed)
        ids, lg = sm.run_greedy(model, sm.OracleMixers(model, ref, len(LENS), MAX_SEQ), prompts,
                                N_NEW)
        mar = sm.margin(lg)
        cp = clear_prefix(mar)
        print(f"seed {seed}: clear prefixes {cp}", flush=True)
        if best is None or min(cp) > min(best[1]):
            best = (seed, cp, prompts, ids, mar)
    seed, cp, prompts, ids, mar = best
    out = dict(model_seed=20260830, prompt_seed=seed, lens=list(LENS), n_new=N_NEW,
               max_seq=MAX_SEQ, near_tie=NEAR_TIE, clear_prefix=cp,
               prompts=[p.tolist() for p in prompts], ids=ids.tolist(),
               margins=np.round(mar, 5).tolist(),
               source="reference anchors (oracle/_ref) as mixers of tests/stream_model.py")
    with open(os.path.join(HERE, "stream_golden.json"), "w") as f:
        json.dump(out, f)
    print("wrote stream_golden.json, prompt seed", seed, "clear prefixes", cp)


if __name__ == "__main__":
    main()
