"""Batched verify engine (yuuka_q35_step_batch / fork / prefill_request) and
the qwen35moe model against the CPU reference decoder, one oracle instance per
request on the same seeded weights. Same logit bar as the single-request
engine: |gpu - cpu| <= 1e-2 * (|cpu| + rms(row)) per element; accepted
prefixes must match the oracle's greedy decision except at a logged near-tie
of the top two logits. The oracle rolls back as the reference engine does
(state.go Snapshot, forward every row, Restore, replay the accepted rows)."""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from oracle import oracle as O
from yuuka_amd import model as Mdl

pytestmark = pytest.mark.gpu


def _close(got, want, what=""):
    want = np.atleast_2d(want)
    got = np.atleast_2d(got)
    for r in range(want.shape[0]):
        rms = float(np.sqrt(np.mean(want[r].astype(np.float64) ** 2)))
        err = np.abs(got[r].astype(np.float64) - want[r])
        assert np.all(err <= 1e-2 * (np.abs(want[r]) + rms)), (what, r, float(err.max()), rms)


def _top2_gap(row):
    s = np.sort(row)
    return float(s[-1] - s[-2])


def _greedy_cont(o, pending, n):
    snap, pos = o.snapshot()
    seq = [int(pending)]
    for _ in range(n):
        seq.append(O.argmax(o.forward([seq[-1]])))
    o.restore(snap, pos)
    return seq[1:]


def _all_rows(o, rows):
    snap, pos = o.snapshot()
    want = o.forward(rows, all_logits=True)
    o.restore(snap, pos)
    return want


def _step(eng, orcs, toks, forced=None, what=""):
    """One batched verify step checked per request against its oracle; the
    oracles then commit the engine's accepted prefixes."""
    n, rows = toks.shape
    want = [_all_rows(orcs[r], toks[r]) for r in range(n)]
    res = eng.step_batch(toks, 0, forced=forced)
    got = eng.logits(n * rows).reshape(n, rows, -1)
    for r in range(n):
        _close(got[r], want[r], f"{what} request {r}")
        drafts = toks[r, 1:]
        if forced is None:
            a, nxt, _ = O.accept_greedy(got[r], drafts)
            a_ref, nxt_ref, _ = O.accept_greedy(want[r], drafts)
            if (a, nxt) != (a_ref, nxt_ref):
                assert _top2_gap(want[r][min(a, a_ref)]) < 1e-2
        else:
            a = min(int(forced[r]), rows - 1)
            nxt = O.argmax(got[r][a])
        assert (int(res[r, 0]), int(res[r, 1])) == (a, nxt), (what, r)
        orcs[r].forward(toks[r, :a + 1])
        assert eng.request_position(r) == orcs[r].position, (what, r)
    return res


def _setup(dev, base, batch, max_rows=16, seed=11, lengths=(10, 17, 24)):
    cfg = replace(base, batch=batch, max_rows=max_rows)
    w = Mdl.make_weights(cfg, seed=seed)
    eng = Mdl.Engine(dev, cfg, w)
    rng = np.random.default_rng(seed)
    orcs, pend = [], []
    for r in range(batch):
        prompt = rng.integers(0, cfg.vocab, lengths[r % len(lengths)] + r).astype(np.int32)
        eng.prefill_request(r, prompt[:-1])
        o = O.Q35(cfg, w)
        o.forward(prompt[:-1])
        orcs.append(o)
        pend.append(int(prompt[-1]))
    return cfg, eng, orcs, pend, rng


def _tokens(orcs, pend, rng, k, accept_lens, vocab):
    toks = np.zeros((len(orcs), k + 1), np.int32)
    for r, o in enumerate(orcs):
        m = accept_lens[r % len(accept_lens)]
        cont = _greedy_cont(o, pend[r], m + 1)
        toks[r, 0] = pend[r]
        toks[r, 1:] = rng.integers(0, vocab, k)
        toks[r, 1:1 + m] = cont[:m]
        if m < k:
            toks[r, 1 + m] = (cont[m] + 1) % vocab  # first rejected draft
    return toks


@pytest.mark.parametrize("model", ["dense", "moe"])
def test_batched_verify_matches_per_request_oracle(dev, model):
    """Three requests at different positions verify k+1 rows each in one
    step with different accepted lengths; logits, decisions, commits and
    positions match per-request oracles over three consecutive steps."""
    cfg, eng, orcs, pend, rng = _setup(dev, Mdl.TINY if model == "dense" else Mdl.TINY_MOE, 3)
    k = 4
    for step, lens in enumerate([(0, 2, 4), (4, 1, 3), (2, 0, 1)]):
        toks = _tokens(orcs, pend, rng, k, lens, cfg.vocab)
        res = _step(eng, orcs, toks, what=f"step {step}")
        pend = [int(res[r, 1]) for r in range(3)]
    eng.close()
    for o in orcs:
        o.close()


def test_forced_acceptance_lengths(dev):
    """Prescribed acceptance lengths (benchmark configurations 3 and 4) commit
    exactly that prefix; the next token is the greedy choice at that row."""
    cfg, eng, orcs, pend, rng = _setup(dev, Mdl.TINY, 4)
    k = 6
    for forced in ([0, 3, 6, 2], [6, 0, 1, 9]):
        toks = np.concatenate([np.array(pend, np.int32)[:, None],
                               rng.integers(0, cfg.vocab, (4, k)).astype(np.int32)], axis=1)
        res = _step(eng, orcs, toks, forced=np.array(forced, np.int32), what=f"forced {forced}")
        pend = [int(res[r, 1]) for r in range(4)]
    eng.close()
    for o in orcs:
        o.close()


def test_fork_shares_prefix_blocks(dev):
    """memory/prefix.go sharing: requests 1 and 2 fork request 0 after a
    37-token prefix (two full 16-token blocks shared, the partial block
    copied), continue with their own suffixes, and verify in one batch."""
    cfg = replace(Mdl.TINY, batch=3, max_rows=16, kv_blocks=3 * 16 - 4)
    w = Mdl.make_weights(cfg, seed=3)
    eng = Mdl.Engine(dev, cfg, w)
    rng = np.random.default_rng(8)
    prefix = rng.integers(0, cfg.vocab, 37).astype(np.int32)
    eng.prefill_request(0, prefix)
    orcs = []
    for r in range(3):
        o = O.Q35(cfg, w)
        o.forward(prefix)
        orcs.append(o)
    eng.fork(0, 1)
    eng.fork(0, 2)
    assert [eng.request_position(r) for r in range(3)] == [37, 37, 37]
    pend = []
    for r in range(3):
        suffix = rng.integers(0, cfg.vocab, 5 + 9 * r).astype(np.int32)
        eng.prefill_request(r, suffix[:-1])
        orcs[r].forward(suffix[:-1])
        pend.append(int(suffix[-1]))
    for step, lens in enumerate([(1, 3, 0), (2, 2, 4)]):
        toks = _tokens(orcs, pend, rng, 4, lens, cfg.vocab)
        res = _step(eng, orcs, toks, what=f"fork step {step}")
        pend = [int(res[r, 1]) for r in range(3)]
    # a reset request returns its blocks; a new prompt reuses them
    eng.reset_request(1)
    p2 = rng.integers(0, cfg.vocab, 30).astype(np.int32)
    eng.prefill_request(1, p2[:-1])
    o = O.Q35(cfg, w)
    o.forward(p2[:-1])
    orcs[1].close()
    orcs[1] = o
    pend[1] = int(p2[-1])
    toks = _tokens(orcs, pend, rng, 4, (0, 1, 2), cfg.vocab)
    _step(eng, orcs, toks, what="after reset")
    eng.close()
    for o in orcs:
        o.close()


def test_long_draft_seventeen_rows(dev):
    """k = 16 drafts (configuration 4): 17 verify rows per request, two
    requests; the recurrent scan and commit take more than 16 rows."""
    cfg, eng, orcs, pend, rng = _setup(dev, Mdl.TINY, 2, max_rows=17)
    k = 16
    for step, lens in enumerate([(16, 5), (3, 11)]):
        toks = _tokens(orcs, pend, rng, k, lens, cfg.vocab)
        res = _step(eng, orcs, toks, what=f"k16 step {step}")
        pend = [int(res[r, 1]) for r in range(2)]
    eng.close()
    for o in orcs:
        o.close()


@pytest.mark.parametrize("shared_ffn", [256, 512])
def test_moe_single_request_prefill_and_verify(dev, shared_ffn):
    """A shared expert as wide as the routed ones runs inside the grouped
    GEMMs (expert index n_experts); a wider one as its own GEMMs. Both
    against the oracle."""
    cfg = replace(Mdl.TINY_MOE, shared_ffn=shared_ffn)
    w = Mdl.make_weights(cfg, seed=9)
    eng = Mdl.Engine(dev, cfg, w)
    orc = O.Q35(cfg, w)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, 29).astype(np.int32)
    _close(eng.prefill(prompt), orc.forward(prompt), "moe prefill")
    rows = np.array([3, 1, 4, 1, 5], np.int32)
    eng.verify(rows)
    _close(eng.logits(5), _all_rows(orc, rows), "moe verify")
    for li in range(cfg.n_layers):  # every layer's routing of the step: rows x used selections
        cnt = eng.moe_counts(li)
        assert cnt.sum() == len(rows) * cfg.n_experts_used and 0 <= cnt.min() and cnt.max() <= len(rows), (li, cnt)
    eng.close()
    orc.close()
