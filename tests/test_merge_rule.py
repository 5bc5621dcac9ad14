"""The split merge's rule on the CPU (no GPU): partial records (m, l, o) of one query head,
folded in the schedule of k_decode_merge (thread groups take records grp, grp + P, ...,
batches of kMergeBatch per memory round trip, groups rescaled to the common maximum and
added in group order), against the fp64 closed form of the same log-sum-exp merge:

    out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s,   M = max_s m_s

A record whose keys were all masked (a prefill part lying past a token's position) is
(m = -inf, l = 0, o = 0) and must weigh nothing. The restatement's weight rule is a
parameter, so the test also shows that the rule without the -inf guard turns a group
holding only such records into NaN (the mistake is planted here, on the CPU).
"""
import numpy as np
import pytest

BATCH = 8  # kMergeBatch


def weight_guarded(m, mb):
    return np.float32(0.0) if m == -np.inf else np.exp2(np.float32(m - mb))


def weight_unguarded(m, mb):
    with np.errstate(invalid="ignore"):
        return np.exp2(np.float32(m) - np.float32(mb))


def merge_schedule(ml, o, groups, weight=weight_guarded):
    """k_decode_merge's fold for one head: ml [S][2] f32, o [S][D] f32; `groups` thread groups."""
    S = len(ml)
    gm, gl, go = [], [], []
    for grp in range(groups):
        m_run, l_run, acc = np.float32(-np.inf), np.float32(0), np.zeros(o.shape[1], np.float32)
        for s0 in range(grp, S, BATCH * groups):
            batch = [s0 + u * groups for u in range(BATCH) if s0 + u * groups < S]
            mb = m_run
            for s in batch:
                mb = max(mb, ml[s][0])
            c = np.float32(1.0) if mb == m_run else np.exp2(np.float32(m_run - mb))
            acc, l_run = acc * c, l_run * c
            for s in batch:
                f = weight(ml[s][0], mb)
                acc = acc + o[s] * f
                l_run = l_run + ml[s][1] * f
            m_run = mb
        gm.append(m_run), gl.append(l_run), go.append(acc)
    M = max(gm)
    total, L = np.zeros(o.shape[1], np.float32), np.float32(0)
    for m_g, l_g, o_g in zip(gm, gl, go):
        sc = np.float32(0) if m_g == -np.inf else np.exp2(np.float32(m_g - M))
        total, L = total + o_g * sc, L + l_g * sc
    return total / L


def closed_form(ml, o):
    m = ml[:, 0].astype(np.float64)
    M = m[np.isfinite(m)].max()
    w = np.where(np.isfinite(m), np.exp2(m - M), 0.0)
    return (w[:, None] * o.astype(np.float64)).sum(0) / (w * ml[:, 1].astype(np.float64)).sum()


def records(rng, S, D, masked):
    """S records of an attention over random keys; the indexes in `masked` attended no key."""
    ml = np.zeros((S, 2), np.float32)
    o = np.zeros((S, D), np.float32)
    for s in range(S):
        if s in masked:
            ml[s] = (-np.inf, 0.0)
            continue
        sc = rng.standard_normal(7).astype(np.float32) * 3  # log2-unit scores of 7 keys
        m = sc.max()
        p = np.exp2(sc - m)
        v = rng.standard_normal((7, D)).astype(np.float32)
        ml[s] = (m, p.sum())
        o[s] = p @ v
    return ml, o


@pytest.mark.parametrize("S,groups,masked", [
    (2, 4, {1}),             # prefill part [256, 260) past positions 200..255: group 1 sees only -inf
    (2, 4, {0}),             # the first record masked
    (9, 4, {1, 5}),          # group 1 holds records 1 and 5 only, both masked
    (40, 4, set(range(0, 40, 4))),  # group 0 entirely masked over several batches
    (64, 16, {3, 7, 63}),
])
def test_merge_masked_records_weigh_nothing(S, groups, masked):
    rng = np.random.default_rng(S * 31 + groups)
    ml, o = records(rng, S, 16, masked)
    got = merge_schedule(ml, o, groups)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, closed_form(ml, o), rtol=2e-6, atol=2e-6)


def test_unguarded_weight_gives_nan():
    """The planted mistake: without the guard a group of only masked records yields NaN."""
    rng = np.random.default_rng(5)
    ml, o = records(rng, 2, 16, {1})
    assert np.isnan(merge_schedule(ml, o, 4, weight=weight_unguarded)).all()
    assert np.isfinite(merge_schedule(ml, o, 4)).all()


def test_merge_no_masked_matches_closed_form():
    rng = np.random.default_rng(11)
    ml, o = records(rng, 100, 32, set())
    np.testing.assert_allclose(merge_schedule(ml, o, 4), closed_form(ml, o), rtol=2e-6, atol=2e-6)
