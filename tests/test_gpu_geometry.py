"""The verify engine at the BASELINE configurations' own shapes, against the
CPU reference decoder (oracle restatement of model/qwen35 +
engine/speculative.go), at reduced depth so that the oracle finishes in
seconds, plus size-independent properties at full depth:

* config 2 shapes: hidden 2560, FFN 9216, 16 Q / 4 KV heads of 256, GDN rank
  16 (conv_dim 6144), V = 151936 through the LM head, 4 layers (3 GDN + 1
  attention), 64-token prompt, k = 4, greedy;
* config 3 shapes: 16 requests x 9 rows forked from a shared prefix,
  stochastic T = 0.7 / top-p 0.9, then prescribed accept lengths;
* config 4 shapes: hidden 4096, FFN 12288, 4 requests x 17 rows, the grouped
  (multi-chunk) attention workgroups;
* config 5 shapes: hidden 2048, 256 experts top-8 + shared expert 512,
  8 requests x 5 rows, stochastic T = 0.8;
* full depth (32 layers, 512-token prompt): verify rows equal prefill rows,
  a partial accept's commit equals a fresh run, repeated runs are
  bit-identical; config 4's 16k context agrees between chunk groupings.

Logit bar (north star): |gpu - cpu| <= 1e-2 * (|cpu| + rms(row)) per
element. Greedy decisions must equal the oracle's except at a near-tie of
the top two logits (< 1e-2); stochastic decisions are checked with the
oracle's Philox draws on the device's own logits and must be identical.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from oracle import oracle as O
from yuuka_amd import model as Mdl

pytestmark = pytest.mark.gpu


def _close(got, want, what="", tol=1e-2):
    want = np.atleast_2d(want)
    got = np.atleast_2d(got)
    for r in range(want.shape[0]):
        rms = float(np.sqrt(np.mean(want[r].astype(np.float64) ** 2)))
        err = np.abs(got[r].astype(np.float64) - want[r])
        assert np.all(err <= tol * (np.abs(want[r]) + rms)), (what, r, float(err.max()), rms)


def _top2_gap(row):
    s = np.sort(row)
    return float(s[-1] - s[-2])


def _all_rows(o, rows):
    snap, pos = o.snapshot()
    want = o.forward(rows, all_logits=True)
    o.restore(snap, pos)
    return want


def _greedy_cont(o, pending, n):
    snap, pos = o.snapshot()
    seq = [int(pending)]
    for _ in range(n):
        seq.append(O.argmax(o.forward([seq[-1]])))
    o.restore(snap, pos)
    return seq[1:]


def _check_greedy(got, want, drafts, res, what):
    a, nxt, _ = O.accept_greedy(got, drafts)
    assert (int(res[0]), int(res[1])) == (a, nxt), what
    a_ref, nxt_ref, _ = O.accept_greedy(want, drafts)
    if (a, nxt) != (a_ref, nxt_ref):
        assert _top2_gap(want[min(a, a_ref)]) < 1e-2, (what, a, a_ref)
    return a


# ---------------------------------------------------------------- config 2

@pytest.fixture(scope="module")
def cfg2(dev):
    cfg = replace(Mdl.QWEN35_4B_LIKE, n_layers=4, capacity=256)
    w = Mdl.make_weights(cfg, seed=21)
    eng = Mdl.Engine(dev, cfg, w)
    orc = O.Q35(cfg, w)
    yield cfg, w, eng, orc
    eng.close()
    orc.close()


def test_config2_shapes_verify_and_commit(cfg2):
    """4B-like widths, 4 layers: prefill, a verify step with two accepted
    drafts, the device commit (recurrent state against the oracle's), and
    the next step's logits."""
    cfg, w, eng, orc = cfg2
    eng.reset()
    orc.reset()
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg.vocab, 64).astype(np.int32)
    _close(eng.prefill(prompt[:-1]), orc.forward(prompt[:-1]), "prefill")
    cont = _greedy_cont(orc, prompt[-1], 3)
    rows = np.array([prompt[-1], cont[0], cont[1], (cont[2] + 1) % cfg.vocab, 17], np.int32)
    res = eng.verify(rows)
    got = eng.logits(5)
    want = _all_rows(orc, rows)
    _close(got, want, "verify")
    a = _check_greedy(got, want, rows[1:], res, "verify")
    orc.forward(rows[:a + 1])
    assert eng.position == orc.position
    gs, gp = eng.snapshot()
    cs, cp = orc.snapshot()
    assert gp == cp
    g32, c32 = gs.view(np.float32), cs.view(np.float32)
    assert np.max(np.abs(g32 - c32)) <= 1e-3 * (np.max(np.abs(c32)) + 1e-6)
    nxt = np.array([res[1], 3, 1, 4, 1], np.int32)
    eng.verify(nxt)
    _close(eng.logits(5), _all_rows(orc, nxt), "after commit")


# ---------------------------------------------------------------- config 3

def _batched_check(eng, checked, toks, res, got, want, accept, step, forced=None, what=""):
    n = toks.shape[0]
    for r in range(n):
        drafts = toks[r, 1:]
        if forced is not None:
            assert int(res[r, 0]) == min(int(forced[r]), toks.shape[1] - 1), (what, r)
        elif accept.mode == 0:
            if r in want:
                _check_greedy(got[r], want[r], drafts, res[r], f"{what} request {r}")
            else:
                a, nxt, _ = O.accept_greedy(got[r], drafts)
                assert (int(res[r, 0]), int(res[r, 1])) == (a, nxt), (what, r)
        else:
            a, nxt, _, _ = O.accept_stochastic(got[r], drafts, accept.temperature, accept.seed, step, r,
                                               accept.top_k, accept.top_p)
            assert (int(res[r, 0]), int(res[r, 1])) == (a, nxt), (what, r)
    for r, o in checked.items():
        o.forward(toks[r, :int(res[r, 0]) + 1])
        assert eng.request_position(r) == o.position, (what, r)


def _batched_setup(dev, base, batch, rows, prefix_len, suffix_lens, checked_ids, seed, share_experts=False):
    cfg = replace(base, n_layers=4, batch=batch, max_rows=rows,
                  capacity=prefix_len + max(suffix_lens) + 4 * rows + 16)
    w = Mdl.make_weights(cfg, seed=seed, share_experts=share_experts)
    eng = Mdl.Engine(dev, cfg, w)
    rng = np.random.default_rng(seed)
    prefix = rng.integers(0, cfg.vocab, prefix_len).astype(np.int32)
    eng.prefill_request(0, prefix)
    for r in range(1, batch):
        eng.fork(0, r)
    checked, pend = {}, []
    for r in range(batch):
        suffix = rng.integers(0, cfg.vocab, suffix_lens[r % len(suffix_lens)]).astype(np.int32)
        if suffix.size > 1:
            eng.prefill_request(r, suffix[:-1])
        pend.append(int(suffix[-1]))
        if r in checked_ids:
            o = O.Q35(cfg, w)
            hist = np.concatenate([prefix, suffix[:-1]])
            o.forward(hist)
            checked[r] = o
    return cfg, w, eng, checked, pend, rng


def _run_batched(eng, cfg, checked, pend, rng, rows, accept, steps, forced_steps=()):
    batch = len(pend)
    for step in range(steps):
        toks = np.concatenate([np.array(pend, np.int32)[:, None],
                               rng.integers(0, cfg.vocab, (batch, rows - 1)).astype(np.int32)], axis=1)
        for r, o in checked.items():  # some drafts the model agrees with
            m = (r + step) % rows
            cont = _greedy_cont(o, pend[r], min(m, 3))
            toks[r, 1:1 + len(cont)] = cont
        want = {r: _all_rows(o, toks[r]) for r, o in checked.items()}
        forced = forced_steps[step] if step < len(forced_steps) else None
        res = eng.step_batch(toks, 0, accept=accept, forced=forced)
        got = eng.logits(batch * rows).reshape(batch, rows, -1)
        for r in checked:
            _close(got[r], want[r], f"step {step} request {r}")
        _batched_check(eng, checked, toks, res, got, want, accept, step, forced, f"step {step}")
        pend = [int(res[r, 1]) for r in range(batch)]
    return pend


def test_config3_shapes_sixteen_forked_requests(dev):
    """16 requests x 9 rows at 4B widths, forked from one 32-token prefix
    (shared KV blocks), stochastic T = 0.7 / top-p 0.9 with each request's
    own Philox stream, then prescribed accept lengths (config 3's forced
    partial acceptance). Four requests are checked against the oracle;
    every request's decisions against the oracle's acceptance rule."""
    cfg, w, eng, checked, pend, rng = _batched_setup(dev, Mdl.QWEN35_4B_LIKE, 16, 9, 32, (1, 2, 4, 5, 3),
                                                      (0, 5, 10, 15), seed=31)
    acc = Mdl.accept_struct(mode=1, temperature=0.7, seed=77, top_p=0.9)
    forced = [None, np.array([(3 * r) % 9 for r in range(16)], np.int32)]
    _run_batched(eng, cfg, checked, pend, rng, 9, acc, 2, forced_steps=forced)
    eng.close()
    for o in checked.values():
        o.close()


# ---------------------------------------------------------------- config 4

def test_config4_shapes_grouped_attention(dev, monkeypatch):
    """9B-like widths (hidden 4096, FFN 12288), 4 requests x 17 rows with
    contexts of ~100-170 tokens; the attention workgroups walk groups of
    two 64-key chunks with a running softmax (the long-context kernel)."""
    monkeypatch.setenv("YUUKA_ATTN_CPW", "2")
    cfg, w, eng, checked, pend, rng = _batched_setup(dev, Mdl.QWEN35_9B_LIKE, 4, 17, 96, (3, 40, 70, 9),
                                                      (0, 2), seed=41)
    _run_batched(eng, cfg, checked, pend, rng, 17, Mdl.accept_struct(), 2)
    eng.close()
    for o in checked.values():
        o.close()


# ---------------------------------------------------------------- config 5

def test_config5_shapes_moe_batch(dev):
    """MoE-like widths (hidden 2048, 256 experts top-8 + shared expert of
    512), 8 requests x 5 rows, stochastic T = 0.8."""
    cfg, w, eng, checked, pend, rng = _batched_setup(dev, Mdl.QWEN35_MOE_LIKE, 8, 5, 16, (2, 5, 9, 1),
                                                      tuple(range(8)), seed=51, share_experts=True)
    acc = Mdl.accept_struct(mode=1, temperature=0.8, seed=5)
    _run_batched(eng, cfg, checked, pend, rng, 5, acc, 2)
    eng.close()
    for o in checked.values():
        o.close()


# ------------------------------------------------------- full depth, no oracle

@pytest.fixture(scope="module")
def full4b(dev):
    cfg = replace(Mdl.QWEN35_4B_LIKE, capacity=640)
    w = Mdl.make_weights(cfg, seed=61)
    eng = Mdl.Engine(dev, cfg, w)
    yield cfg, eng
    eng.close()


def test_full_depth_verify_rows_equal_prefill_rows(full4b):
    """32 layers, 512-token prompt: verify row i's logits equal the logits a
    fresh prefill of the same tokens ends with (different kernels: the
    chunked prefill GEMM and attention against the verify step's)."""
    cfg, eng = full4b
    rng = np.random.default_rng(62)
    prompt = rng.integers(0, cfg.vocab, 512).astype(np.int32)
    rows = rng.integers(0, cfg.vocab, 5).astype(np.int32)
    eng.reset()
    eng.prefill(prompt)
    snap, pos = eng.snapshot()
    eng.verify(rows)
    got = eng.logits(5)
    for i in range(5):
        eng.reset()
        want = eng.prefill(np.concatenate([prompt, rows[:i + 1]]))
        _close(got[i], want, f"row {i}")
    # repeated verify from the same state is bit-identical
    eng.reset()
    eng.prefill(prompt)
    eng.verify(rows)
    assert np.array_equal(eng.logits(5), got)


def test_full_depth_partial_commit_equals_fresh_run(full4b):
    """A verify step that accepts exactly two drafts leaves the state a
    fresh prefill of the same tokens leaves, and the next verify step agrees."""
    cfg, eng = full4b
    rng = np.random.default_rng(63)
    prompt = rng.integers(0, cfg.vocab, 512).astype(np.int32)
    eng.reset()
    eng.prefill(prompt[:-1])
    # the device's own greedy choices as drafts: two accepted, then a miss
    seq = [int(prompt[-1])]
    snap, pos = eng.snapshot()
    for _ in range(3):
        lg = eng.prefill(np.array([seq[-1]], np.int32))
        seq.append(int(np.argmax(lg)))
    eng.restore(snap, pos)
    rows = np.array([seq[0], seq[1], seq[2], (seq[3] + 1) % cfg.vocab, 9], np.int32)
    res = eng.verify(rows)
    assert int(res[0]) == 2 and int(res[1]) == seq[3]
    s_verify, p_verify = eng.snapshot()
    nxt = np.array([res[1], 5, 6, 7, 8], np.int32)
    eng.verify(nxt)
    l_verify = eng.logits(5)
    eng.reset()
    eng.prefill(np.concatenate([prompt, rows[1:3]]))
    s_fresh, p_fresh = eng.snapshot()
    assert p_verify == p_fresh
    a, b = s_verify.view(np.float32), s_fresh.view(np.float32)
    assert np.max(np.abs(a - b)) <= 2e-3 * (np.max(np.abs(b)) + 1e-6)
    eng.verify(nxt)
    _close(eng.logits(5), l_verify, "next step")


def test_config4_16k_context_chunk_groupings_agree(dev, monkeypatch):
    """9B-like attention at 16k context, 4 requests x 17 rows (2 layers: one
    GDN, one attention): one chunk per workgroup (cpw 1) and the automatic
    long-context grouping give the same logits; repeated runs are
    bit-identical."""
    cfg = replace(Mdl.QWEN35_9B_LIKE, n_layers=2, full_interval=2, batch=4, max_rows=17,
                  capacity=16384 + 64)
    w = Mdl.make_weights(cfg, seed=71)
    rng = np.random.default_rng(72)
    prompts = [rng.integers(0, cfg.vocab, 16384 - 37 * r).astype(np.int32) for r in range(4)]
    toks = rng.integers(0, cfg.vocab, (4, 17)).astype(np.int32)
    out = {}
    for cpw in ("1", "auto", "auto2"):
        if cpw == "1":
            monkeypatch.setenv("YUUKA_ATTN_CPW", "1")
        else:
            monkeypatch.delenv("YUUKA_ATTN_CPW", raising=False)
        dev_eng = Mdl.Engine(dev, cfg, w)
        for r in range(4):
            dev_eng.prefill_request(r, prompts[r])
        dev_eng.step_batch(toks, 0, accept=Mdl.accept_struct(), forced=np.zeros(4, np.int32))
        out[cpw] = dev_eng.logits(4 * 17)
        dev_eng.close()
    assert np.array_equal(out["auto"], out["auto2"])
    _close(out["auto"], out["1"], "cpw auto vs 1", tol=1e-4)


def test_config3_rows_long_context_grouped_attention(dev, monkeypatch):
    """Config 3's attention geometry at real context lengths: 16 Q / 4 KV
    heads of 256, 9 verify rows per request (36 MFMA rows per KV head, the
    three-tile grouped kernel attn_verify_mfma_group_kernel<3, true>), three
    requests at ~450-700 tokens of context, the key chunks walked in groups
    of 3 and of 5 per workgroup with the running softmax, and the one-chunk
    kernel; each against the oracle decoder on every request (observed
    1-2e-3 of the row rms for all three), and the groupings against each
    other. Narrow non-attention widths (hidden 256,
    one attention layer, 1024-token vocabulary) keep the oracle's prefill
    short; the attention shapes are config 3's."""
    cfg = replace(Mdl.QWEN35_4B_LIKE, hidden=256, ffn=512, n_layers=1, full_interval=1, vocab=1024, batch=3,
                  max_rows=9, capacity=768)
    w = Mdl.make_weights(cfg, seed=81)
    rng = np.random.default_rng(82)
    prompts = [rng.integers(0, cfg.vocab, n).astype(np.int32) for n in (700, 451, 598)]
    toks = rng.integers(0, cfg.vocab, (3, 9)).astype(np.int32)
    want = []
    for r in range(3):
        o = O.Q35(replace(cfg, batch=1), w)
        o.forward(prompts[r][:-1])
        toks[r, 0] = prompts[r][-1]
        want.append(o.forward(toks[r], all_logits=True))
        o.close()
    out = {}
    for cpw in ("3", "5", "1"):
        monkeypatch.setenv("YUUKA_ATTN_CPW", cpw)
        eng = Mdl.Engine(dev, cfg, w)
        for r in range(3):
            eng.prefill_request(r, prompts[r][:-1])
        eng.step_batch(toks, 0, accept=Mdl.accept_struct(), forced=np.zeros(3, np.int32))
        got = eng.logits(3 * 9).reshape(3, 9, -1)
        eng.close()
        for r in range(3):
            _close(got[r], want[r], f"cpw {cpw} request {r}")
        out[cpw] = got
    # the groupings agree up to float32 reassociation, which the narrow
    # model's int16 activation quantization turns into ~1e-3 of the logits'
    # rms (the same spread all three show against the oracle)
    _close(out["3"], out["1"], "cpw 3 vs 1", tol=5e-3)
    _close(out["5"], out["1"], "cpw 5 vs 1", tol=5e-3)


def test_many_rows_long_context_grouped_attention_two_row_blocks(dev, monkeypatch):
    """25 verify rows per request at 16 Q / 4 KV heads: 100 MFMA rows per KV
    head, more than the six-tile grouped kernel
    (attn_verify_mfma_group_kernel<6, true>) holds, so it walks the key
    chunks twice, for a block of 24 rows (every tile in use) and a block of
    one row (one tile of six in use). Two requests at ~400-500 tokens, chunk
    groups of 3 and the one-chunk kernel, each against the oracle decoder."""
    cfg = replace(Mdl.QWEN35_4B_LIKE, hidden=256, ffn=512, n_layers=1, full_interval=1, vocab=1024, batch=2,
                  max_rows=25, capacity=640)
    w = Mdl.make_weights(cfg, seed=91)
    rng = np.random.default_rng(92)
    prompts = [rng.integers(0, cfg.vocab, n).astype(np.int32) for n in (517, 388)]
    toks = rng.integers(0, cfg.vocab, (2, 25)).astype(np.int32)
    want = []
    for r in range(2):
        o = O.Q35(replace(cfg, batch=1), w)
        o.forward(prompts[r][:-1])
        toks[r, 0] = prompts[r][-1]
        want.append(o.forward(toks[r], all_logits=True))
        o.close()
    for cpw in ("3", "1"):
        monkeypatch.setenv("YUUKA_ATTN_CPW", cpw)
        eng = Mdl.Engine(dev, cfg, w)
        for r in range(2):
            eng.prefill_request(r, prompts[r][:-1])
        eng.step_batch(toks, 0, accept=Mdl.accept_struct(), forced=np.zeros(2, np.int32))
        got = eng.logits(2 * 25).reshape(2, 25, -1)
        eng.close()
        for r in range(2):
            _close(got[r], want[r], f"cpw {cpw} request {r}")
