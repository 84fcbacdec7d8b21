"""CPU checks of the attention decode split plan (no GPU): the scores
kernel's writer wavefront counts each run's 64-key groups before it stores
anything, and the streaming wavefronts publish one group per 64 keys of
each segment they walk. If the two enumerations ever differed, a
producer/consumer wait of the score ring would not be met (the kernel's
bounded waits would then expire and fail the call). The same walk checks
that every real key of every (sequence, kv head) pair lies in exactly one
segment, that the segments' statistics / partial slots are distinct, and
that the runs P.V and the combine fold for a pair (pair_runs) are exactly
the runs that hold one of its segments.

The plan is walked on the host by the library itself
(apus_hip_attn_split_check), through the same seg_at / run_groups /
pair_runs code the kernels run."""
import numpy as np
import pytest

import apus_hip


def _check(tq, pos0, nkv=2, cus=256):
    cu = np.concatenate([[0], np.cumsum(tq)]).astype(np.int32)
    r = apus_hip.attn_split_check(cu, np.asarray(pos0, np.int32), nkv=nkv, cus=cus)
    assert r["group_mismatch"] == 0, r
    assert r["writer_groups"] == r["stream_groups"], r
    for k in ("bad_keys", "bad_slots", "bad_pair_runs", "pv_bad_keys", "pv_bad_slots",
              "pv_bad_pair_runs"):
        assert r[k] == 0, (k, r)
    return r


def test_config2_shape():
    r = _check([1] * 64, [32767] * 64)
    # 64 pairs x 2 heads x 32768 padded keys / T1 groups of 64
    assert r["writer_groups"] == 64 * 2 * 32768 // 64


def test_single_key_pairs():
    """Sequences whose only key is the new token (pos0 = 0, one token)."""
    _check([1] * 7, [0] * 7)
    _check([1], [0])
    _check([4, 1, 1, 3], [0, 0, 5, 0])


@pytest.mark.parametrize("seed", range(12))
def test_random_ragged(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.choice([1, 3, 17, 128, 224, 225, 260]))
    tq = rng.integers(1, 5, B)
    # a mix of tiny, block-edge and long contexts
    kinds = rng.integers(0, 4, B)
    pos0 = np.where(kinds == 0, rng.integers(0, 70, B),
                    np.where(kinds == 1, 64 * rng.integers(1, 40, B) - tq,
                             np.where(kinds == 2, rng.integers(0, 9000, B),
                                      rng.integers(30000, 66000, B))))
    pos0 = np.maximum(pos0, 0)
    cus = int(rng.choice([1, 7, 80, 256]))
    _check(tq, pos0, cus=cus)


def test_b260_lognormal():
    """The B=260 attention case of the full-config tests (more sequences than
    the by-value metadata holds), at config 4's context distribution."""
    rng = np.random.default_rng(7)
    ctx = np.clip(np.exp(rng.normal(np.log(4096), 1.0, 260)), 256, 65536).astype(np.int64)
    tq = rng.integers(1, 5, 260)
    _check(tq, ctx - tq)


def test_rejects_bad_batches():
    with pytest.raises(apus_hip.ApusHipError):
        apus_hip.attn_split_check(np.array([0, 5], np.int32), np.array([0], np.int32))
