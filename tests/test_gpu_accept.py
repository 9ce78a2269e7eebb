"""GPU parity of the fused verify-accept kernel against the oracle restatement
of engine/speculative.go:191-208 (greedy) and the repository's stochastic
speculative-sampling definition. Every call goes through the C ABI."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from yuuka_amd import hip, synth

pytestmark = pytest.mark.gpu


def _run(dev, stream, logits, drafts, params):
    B = params.batch
    lb = dev.upload(logits.astype(np.float32))
    db = dev.upload(np.asarray(drafts, np.int32).reshape(-1)) if params.drafts else None
    rb = dev.alloc(B * 16)
    dbg = dev.alloc(B * (params.drafts + 1) * 32)
    hip.verify_accept(stream, lb, db, rb, params, debug=dbg)
    stream.sync()
    return rb.read(np.int32).reshape(B, 4), dbg.read(np.float64).reshape(B, params.drafts + 1, 4)


def test_greedy_config1(dev, stream):
    c = synth.config1(0)
    p = hip.accept_params(hip.ACCEPT_GREEDY, 1, c["k"], c["V"])
    res, _ = _run(dev, stream, c["logits"], c["drafts"], p)
    a, nxt, rows = O.accept_greedy(c["logits"], c["drafts"])
    assert (res[0, 0], res[0, 1], res[0, 2]) == (a, nxt, rows[0])


@pytest.mark.parametrize("accept_len", [0, 1, 2, 3, 4])
def test_greedy_forced_acceptance_lengths(dev, stream, accept_len):
    rng = np.random.default_rng(accept_len)
    k, V = 4, 151936
    logits = rng.normal(0, 3, (k + 1, V)).astype(np.float32)
    am = logits.argmax(axis=1)
    drafts = [int(am[i]) if i < accept_len else int((am[i] + 1) % V) for i in range(k)]
    p = hip.accept_params(hip.ACCEPT_GREEDY, 1, k, V)
    res, _ = _run(dev, stream, logits, drafts, p)
    a, nxt, _ = O.accept_greedy(logits, drafts)
    assert a == accept_len and (res[0, 0], res[0, 1]) == (a, nxt)


def test_greedy_ties_nan_inf(dev, stream):
    V, k = 5000, 3
    logits = np.zeros((k + 1, V), np.float32)
    logits[0, [10, 4000, 4999]] = 7.0          # tie: lowest index wins
    logits[1, 0] = np.nan                       # NaN at index 0 wins
    logits[1, 5] = 100.0
    logits[2, :] = -np.inf                      # all -inf: index 0
    logits[2, 3] = np.nan
    logits[3, 17] = np.inf
    logits[3, 12] = np.nan
    for drafts in ([10, 0, 0], [10, 5, 0], [4000, 0, 0], [10, 0, 1]):
        p = hip.accept_params(hip.ACCEPT_GREEDY, 1, k, V)
        res, _ = _run(dev, stream, logits, drafts, p)
        a, nxt, rows = O.accept_greedy(logits, drafts)
        assert (res[0, 0], res[0, 1]) == (a, nxt), drafts


def test_greedy_batched_with_stride(dev, stream):
    rng = np.random.default_rng(9)
    B, k, V, stride = 3, 8, 32000, 32064
    logits = rng.normal(0, 3, (B, k + 1, stride)).astype(np.float32)
    drafts = np.zeros((B, k), np.int32)
    for b in range(B):
        am = logits[b, :, :V].argmax(axis=1)
        drafts[b] = [am[i] if i < 2 * b + 1 else (am[i] + 3) % V for i in range(k)]
    p = hip.accept_params(hip.ACCEPT_GREEDY, B, k, V, row_stride=stride)
    res, _ = _run(dev, stream, logits, drafts, p)
    for b in range(B):
        a, nxt, _ = O.accept_greedy(np.ascontiguousarray(logits[b, :, :V]), drafts[b])
        assert (res[b, 0], res[b, 1]) == (a, nxt)


def test_stochastic_matches_oracle_decisions(dev, stream):
    """Identical accept/reject decisions and resampled tokens whenever the
    probabilities agree to tolerance; a mismatch is tolerated only at a
    documented near-tie (|u - p| or the inverse-CDF boundary within 1e-9)."""
    rng = np.random.default_rng(21)
    k, V, T = 4, 151936, 0.8
    mismatches = 0
    for trial in range(24):
        logits = rng.normal(0, 3, (k + 1, V)).astype(np.float32)
        # make acceptance likely for a few rows: sharpen the draft's logit
        drafts = rng.integers(0, V, k).astype(np.int32)
        for i in range(k):
            if rng.random() < 0.6:
                logits[i, drafts[i]] = logits[i].max() + rng.uniform(-1, 3)
        p = hip.accept_params(hip.ACCEPT_STOCHASTIC, 1, k, V, temperature=T, seed=1234, step=trial)
        res, dbg = _run(dev, stream, logits, drafts, p)
        a, nxt, pd, ua = O.accept_stochastic(logits, drafts, T, 1234, trial, 0)
        for i in range(min(a, int(res[0, 0])) + 1):
            if i < k:
                assert dbg[0, i, 1] == ua[i]                    # same Philox draw, bit for bit
                assert abs(dbg[0, i, 0] - pd[i]) <= 1e-9 * max(pd[i], 1e-300) + 1e-15
        if (int(res[0, 0]), int(res[0, 1])) != (a, nxt):
            i = min(a, int(res[0, 0]))
            near = i < k and abs(ua[i] - pd[i]) < 1e-9
            assert near, (trial, res[0], a, nxt)
            mismatches += 1
    assert mismatches <= 1


def test_stochastic_zero_temperature_is_greedy(dev, stream):
    c = synth.config1(3)
    p = hip.accept_params(hip.ACCEPT_STOCHASTIC, 1, c["k"], c["V"], temperature=0.0)
    res, _ = _run(dev, stream, c["logits"], c["drafts"], p)
    a, nxt, _ = O.accept_greedy(c["logits"], c["drafts"])
    assert (res[0, 0], res[0, 1]) == (a, nxt)


def _check_truncated(dev, stream, logits, drafts, T, top_k, top_p, seed, step):
    """Device vs oracle for one request under top-k / top-p: the kept set must
    match (row totals agree to 1e-12), so must p(draft) and every decision,
    except at a near-tie of u and p(draft)."""
    k = len(drafts)
    V = logits.shape[-1]
    p = hip.accept_params(hip.ACCEPT_STOCHASTIC, 1, k, V, temperature=T, top_k=top_k, top_p=top_p,
                          seed=seed, step=step)
    res, dbg = _run(dev, stream, logits, drafts, p)
    a, nxt, pd, ua = O.accept_stochastic(logits, drafts, T, seed, step, 0, top_k, top_p)
    last = min(a, int(res[0, 0]))
    for i in range(last + 1):
        _, w, total, _ = O.target_weights(logits[i], T, top_k, top_p)
        assert abs(dbg[0, i, 2] - total) <= 1e-12 * total, (i, dbg[0, i, 2], total)
        if i < k:
            assert dbg[0, i, 1] == ua[i]
            assert abs(dbg[0, i, 0] - pd[i]) <= 1e-9 * max(pd[i], 1e-300) + 1e-15
    if (int(res[0, 0]), int(res[0, 1])) != (a, nxt):
        assert last < k and abs(ua[last] - pd[last]) < 1e-9, (res[0], a, nxt)
        return 1
    return 0


@pytest.mark.parametrize("top_k,top_p,T", [(0, 0.9, 0.7), (50, 1.0, 0.8), (400, 0.9, 0.7), (0, 0.5, 1.3)])
def test_stochastic_top_k_top_p_matches_oracle(dev, stream, top_k, top_p, T):
    """The config-3 sampler settings (T = 0.7, top-p 0.9) and top-k alone or
    combined, on N(0, 3) logits over the full vocabulary."""
    rng = np.random.default_rng(31 + top_k)
    k, V = 8, 151936
    mism = 0
    for trial in range(6):
        logits = rng.normal(0, 3, (k + 1, V)).astype(np.float32)
        drafts = rng.integers(0, V, k).astype(np.int32)
        order = np.argsort(-logits, axis=1, kind="stable")
        for i in range(k):  # drafts from the head of the distribution, so rows get accepted
            if rng.random() < 0.8:
                drafts[i] = order[i, int(rng.integers(0, 3))]
        mism += _check_truncated(dev, stream, logits, drafts, T, top_k, top_p, 77, trial)
    assert mism <= 1


def test_truncation_cut_inside_tie_groups(dev, stream):
    """Integer-valued logits make the top-k and top-p boundaries fall inside
    large groups of equal logits: the kept members are the lowest ids
    (sampling.go:84-92); -0 and +0 rank as equal."""
    rng = np.random.default_rng(5)
    k, V = 3, 5000
    for top_k, top_p in [(37, 1.0), (0, 0.3), (700, 0.6), (5, 0.99)]:
        logits = rng.integers(0, 8, (k + 1, V)).astype(np.float32)
        logits[:, ::7] = 0.0
        logits[:, 3::7] = -0.0
        logits[:, 11] = np.nan
        logits[:, 12] = -np.inf
        drafts = []
        for i in range(k):
            ties = np.flatnonzero(logits[i] == 7.0)
            drafts.append(int(ties[min(len(ties) - 1, (i + 1) * 9)]))
        for step in range(3):
            assert _check_truncated(dev, stream, logits, np.array(drafts, np.int32), 1.0, top_k, top_p, 3,
                                    step) == 0


def test_truncation_zero_and_negative_keys(dev, stream):
    """A cut among zero and negative logits, where the order key of -0 must
    equal that of +0."""
    k, V = 2, 3000
    logits = np.full((k + 1, V), -1.0, np.float32)
    logits[:, 100:200] = -0.0
    logits[:, 150:250] = 0.0
    logits[:, 5] = 2.0
    drafts = np.array([180, 240], np.int32)
    for top_k in (30, 120, 190, 260):
        assert _check_truncated(dev, stream, logits, drafts, 0.5, top_k, 1.0, 9, top_k) == 0


def test_truncated_acceptance_is_reproducible(dev, stream):
    """The radix-selection histograms are combined in a fixed order: two runs
    give bit-identical probabilities and decisions."""
    rng = np.random.default_rng(12)
    k, V = 8, 151936
    logits = rng.normal(0, 3, (k + 1, V)).astype(np.float32)
    drafts = np.argsort(-logits, axis=1)[:k, 1].astype(np.int32)
    p = hip.accept_params(hip.ACCEPT_STOCHASTIC, 1, k, V, temperature=0.7, top_p=0.9, seed=4, step=2)
    r1, d1 = _run(dev, stream, logits, drafts, p)
    r2, d2 = _run(dev, stream, logits, drafts, p)
    assert (r1 == r2).all() and np.array_equal(d1, d2)


def test_truncation_tie_group_spanning_late_id_steps(dev, stream):
    """Full vocabulary: a top tie group of 300 equal logits, 40 of them below
    id 8192 and the rest spread up to the last id, so the top-k / top-p cut
    falls on a member the kept-id sweep reaches only in a later 8192-id step.
    The kept set (lowest ids of the group) and every decision match the
    oracle's."""
    rng = np.random.default_rng(17)
    k, V = 4, 151936
    logits = rng.normal(0, 1, (k + 1, V)).astype(np.float32)
    ties = np.concatenate([rng.choice(8192, 40, replace=False),
                           8192 + rng.choice(V - 8192, 260, replace=False)])
    ties.sort()
    logits[:, ties] = 10.0
    drafts = np.array([ties[150], ties[20], ties[299], ties[90]], np.int32)
    for top_k, top_p in [(120, 1.0), (0, 0.5), (250, 0.3), (41, 1.0)]:
        for step in range(2):
            assert _check_truncated(dev, stream, logits, drafts, 1.0, top_k, top_p, 21, step) == 0
