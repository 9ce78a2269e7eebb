"""GPU verify engine (yuuka_q35_*) against the CPU reference decoder (oracle
restatement of model/qwen35 + engine/speculative.go) on the same seeded
weights. Logit tolerance: |gpu - cpu| <= 1e-2 * (|cpu| + rms(row)) per
element, the north-star bar; greedy tokens must be identical (a mismatch is
only tolerated at a logged near-tie of the top two logits)."""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from oracle import oracle as O
from yuuka_amd import model as Mdl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny():
    cfg = Mdl.TINY
    w = Mdl.make_weights(cfg, seed=7)
    return cfg, w


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


def test_prefill_logits_match_oracle(dev, tiny):
    cfg, w = tiny
    eng = Mdl.Engine(dev, cfg, w)
    orc = O.Q35(cfg, w)
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, 37).astype(np.int32)
    got = eng.prefill(prompt)
    want = orc.forward(prompt)
    _close(got, want, "prefill")
    assert eng.position == orc.position == 37
    eng.close()
    orc.close()


@pytest.mark.parametrize("kv", [Mdl.F16, Mdl.F32])
def test_verify_rows_match_prefill_logits(dev, tiny, kv):
    cfg, w = tiny
    cfg = replace(cfg, kv_dtype=kv)
    eng = Mdl.Engine(dev, cfg, w)
    orc = O.Q35(cfg, w, kv_format=1 if kv == Mdl.F16 else 0)
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, cfg.vocab, 20).astype(np.int32)
    eng.prefill(prompt[:-1])
    orc.forward(prompt[:-1])
    rows = np.concatenate([prompt[-1:], rng.integers(0, cfg.vocab, 4)]).astype(np.int32)
    res = eng.verify(rows)
    got = eng.logits(5)
    want = orc.forward(rows, all_logits=True)
    _close(got, want, "verify")
    a, nxt, am = O.accept_greedy(got, rows[1:])
    assert (res[0], res[1]) == (a, nxt)
    a_ref, nxt_ref, _ = O.accept_greedy(want, rows[1:])
    if (a, nxt) != (a_ref, nxt_ref):
        assert _top2_gap(want[min(a, a_ref)]) < 1e-2
    eng.close()
    orc.close()


@pytest.mark.parametrize("cpw", [1, 2, 3])
@pytest.mark.parametrize("k", [4, 16])
def test_verify_over_chunk_groups_matches_oracle(dev, tiny, monkeypatch, cpw, k):
    """A 200-token context spans four 64-key chunks: one verify-attention
    workgroup walks `cpw` of them with a running softmax (cpw = 1: one chunk
    per workgroup), then the groups are merged. Logits of k + 1 verify rows
    against the oracle."""
    monkeypatch.setenv("YUUKA_ATTN_CPW", str(cpw))
    cfg, w = tiny
    cfg = replace(cfg, max_rows=max(cfg.max_rows, k + 1))
    eng = Mdl.Engine(dev, cfg, w)
    orc = O.Q35(cfg, w, kv_format=1)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, cfg.vocab, 200).astype(np.int32)
    eng.prefill(prompt[:-1])
    orc.forward(prompt[:-1])
    rows = np.concatenate([prompt[-1:], rng.integers(0, cfg.vocab, k)]).astype(np.int32)
    eng.verify(rows)
    got = eng.logits(k + 1)
    want = orc.forward(rows, all_logits=True)
    _close(got, want, f"verify cpw={cpw} k={k}")
    eng.close()
    orc.close()


def test_partial_acceptance_commits_exact_prefix(dev, tiny):
    """Drafts chosen so that exactly two are accepted: the device commit must
    leave the state the oracle has after the accepted prefix, and the next
    step's logits must agree."""
    cfg, w = tiny
    eng = Mdl.Engine(dev, cfg, w)
    orc = O.Q35(cfg, w)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, cfg.vocab, 12).astype(np.int32)
    eng.prefill(prompt[:-1])
    orc.forward(prompt[:-1])
    # true greedy continuation from the oracle (on a snapshot)
    snap, pos = orc.snapshot()
    seq = [int(prompt[-1])]
    for _ in range(3):
        lg = orc.forward([seq[-1]])
        seq.append(O.argmax(lg))
    orc.restore(snap, pos)
    drafts = [seq[1], seq[2], (seq[3] + 1) % cfg.vocab, 5]
    res = eng.verify(np.array([prompt[-1]] + drafts, np.int32))
    assert res[0] == 2 and res[1] == seq[3]
    orc.forward([prompt[-1], seq[1], seq[2]])
    assert eng.position == orc.position
    gs, gp = eng.snapshot()
    cs, cp = orc.snapshot()
    assert gp == cp
    g32, c32 = gs.view(np.float32), cs.view(np.float32)
    assert np.max(np.abs(g32 - c32)) <= 1e-3 * (np.max(np.abs(c32)) + 1e-6)
    # next step continues from the committed state
    nxt = [res[1], 1, 2, 3, 4]
    eng.verify(np.array(nxt, np.int32))
    _close(eng.logits(5), orc.forward(nxt, all_logits=True), "after commit")
    eng.close()
    orc.close()


def test_snapshot_restore_roundtrip(dev, tiny):
    cfg, w = tiny
    eng = Mdl.Engine(dev, cfg, w)
    prompt = np.arange(1, 30, dtype=np.int32)
    eng.prefill(prompt)
    snap, pos = eng.snapshot()
    a = eng.verify(np.array([7, 8, 9], np.int32))
    la = eng.logits(3)
    eng.restore(snap, pos)
    b = eng.verify(np.array([7, 8, 9], np.int32))
    assert np.array_equal(a, b)
    assert np.array_equal(la, eng.logits(3))
    eng.close()


def test_speculative_generate_equals_greedy(dev, tiny):
    """engine/speculative_test.go:180-215 TestSpeculativeMatchesGreedy on the
    device engine: speculative output equals plain greedy decoding."""
    cfg, w = tiny
    eng = Mdl.Engine(dev, cfg, w)
    orc = O.Q35(cfg, w)
    prompt = [5, 6, 7, 5, 6, 7, 5, 6, 9, 5, 6, 7]
    toks, stats = eng.generate(prompt, 40, max_draft=4, min_match=2)
    ref, _, _ = O.generate_greedy_speculative(orc, prompt, 40, 4, 2)
    if toks != ref:
        # only acceptable at a near-tie: find the first difference
        i = next(j for j in range(min(len(toks), len(ref))) if toks[j] != ref[j])
        orc.reset()
        lg = orc.forward(prompt + ref[:i])
        assert _top2_gap(lg) < 1e-2, (i, toks[i], ref[i])
    assert stats.output_tokens == 40 and stats.steps <= 40
    eng.close()
    orc.close()


def test_stochastic_generate_is_deterministic(dev, tiny):
    cfg, w = tiny
    eng = Mdl.Engine(dev, cfg, w)
    acc = Mdl.accept_struct(mode=1, temperature=0.8, seed=11)
    prompt = [3, 4, 5, 3, 4, 5, 3, 4]
    a, _ = eng.generate(prompt, 24, accept=acc)
    b, _ = eng.generate(prompt, 24, accept=acc)
    assert a == b and len(a) == 24
    c, _ = eng.generate(prompt, 24, accept=Mdl.accept_struct(mode=1, temperature=0.8, seed=12))
    assert len(c) == 24
    eng.close()


def test_eager_plan_execution_equals_graph_replay(dev, tiny, monkeypatch):
    """YUUKA_Q35_EAGER=1 (profiling) runs the same plans op by op instead
    of replaying captured graphs: the logits and results are bit-identical."""
    cfg, w = tiny
    out = []
    for eager in ("0", "1"):
        monkeypatch.setenv("YUUKA_Q35_EAGER", eager)
        eng = Mdl.Engine(dev, cfg, w)
        eng.prefill(np.arange(3, 40, dtype=np.int32))
        res = eng.verify(np.array([4, 5, 6, 7, 8], np.int32))
        out.append((res.copy(), eng.logits(5)))
        eng.close()
    assert np.array_equal(out[0][0], out[1][0])
    assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))



@pytest.mark.parametrize("which", ["dense", "moe"])
def test_engine_from_gguf_equals_engine_from_weights(dev, tiny, tmp_path, which):
    """A model written to GGUF and loaded back (yuuka_amd.gguf: the reader,
    LoadConfig and Load of model/qwen35) gives the engine the same bytes:
    prefill, verify result and verify logits bit-identical to the engine
    built from the in-memory weights."""
    from yuuka_amd import gguf as G
    if which == "dense":
        cfg, w = tiny
    else:
        cfg = Mdl.TINY_MOE
        w = Mdl.make_weights(cfg, seed=11)
    path = str(tmp_path / f"{which}.gguf")
    G.write_q35(path, cfg, w)
    session = dict(capacity=cfg.capacity, block_size=cfg.block_size, kv_dtype=cfg.kv_dtype,
                   max_rows=cfg.max_rows, batch=cfg.batch, kv_blocks=cfg.kv_blocks)
    out = []
    with G.Reader(path) as r:
        cfg2 = G.load_config(r, **session)
        assert cfg2.n_experts == cfg.n_experts and cfg2.vocab == cfg.vocab
        w2 = G.load_weights(r, cfg2)
        for c, ws in ((cfg, w), (cfg2, w2)):
            eng = Mdl.Engine(dev, c, ws)
            first = eng.prefill(np.arange(5, 30, dtype=np.int32) % c.vocab)
            res = eng.verify(np.array([9, 10, 11, 12, 13], np.int32))
            out.append((first, res.copy(), eng.logits(5)))
            eng.close()
        del w2
    for a, b in zip(out[0], out[1]):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


@pytest.mark.parametrize("width", [3, 5])
@pytest.mark.parametrize("k", [4, 16])
def test_other_conv_widths_match_oracle(dev, width, k):
    """GDN causal conv of width 3 or 5 (the models use 4; other widths take
    the kernels' generic conv path): prefill, k + 1 verify rows and the
    committed state after a partial accept against the oracle."""
    cfg = replace(Mdl.TINY, conv_kernel=width, max_rows=max(Mdl.TINY.max_rows, k + 1))
    w = Mdl.make_weights(cfg, seed=11)
    eng = Mdl.Engine(dev, cfg, w)
    orc = O.Q35(cfg, w, kv_format=1)
    rng = np.random.default_rng(width * 100 + k)
    prompt = rng.integers(0, cfg.vocab, 30).astype(np.int32)
    _close(eng.prefill(prompt[:-1]), orc.forward(prompt[:-1]), f"prefill width={width}")
    rows = np.concatenate([prompt[-1:], rng.integers(0, cfg.vocab, k)]).astype(np.int32)
    snap, pos = orc.snapshot()
    res = eng.verify(rows)
    want = orc.forward(rows, all_logits=True)
    _close(eng.logits(k + 1), want, f"verify width={width} k={k}")
    # the device accepted res[0] drafts: the oracle replays the same prefix
    orc.restore(snap, pos)
    orc.forward(rows[: res[0] + 1])
    gs, gp = eng.snapshot()
    cs, cp = orc.snapshot()
    assert gp == cp
    g32, c32 = gs.view(np.float32), cs.view(np.float32)
    assert np.max(np.abs(g32 - c32)) <= 1e-3 * (np.max(np.abs(c32)) + 1e-6)
    eng.close()
    orc.close()
