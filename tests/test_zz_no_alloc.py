"""yuuka_verify_accept_noalloc (the acceptance entry point that allocates
nothing: its partials live in a fixed per-GPU device array) against
yuuka_verify_accept on the same inputs, through the C ABI: greedy at
configuration 1's shape, stochastic top-p at configuration 3's 16 x 9 rows,
two calls in a row with the second smaller, and the size limit."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from yuuka_amd import hip

pytestmark = pytest.mark.gpu

V = 151936


def _noalloc(stream, logits, drafts, result, params):
    hip.check(hip.lib().yuuka_verify_accept_noalloc(stream.ptr, logits.ptr, 0, hip._p(drafts), 0, result.ptr, 0,
                                                    C.byref(params), None), "verify_accept_noalloc")


def _case(dev, stream, rng, batch, k, params):
    logits = rng.normal(0, 3, (batch * (k + 1), V)).astype(np.float32)
    drafts = rng.integers(0, V, (batch, k)).astype(np.int32)
    # some drafts the target agrees with, so acceptance runs past row 0
    for b in range(batch):
        m = b % (k + 1)
        drafts[b, :m] = logits[b * (k + 1):b * (k + 1) + m].argmax(axis=1)
    lb, db = dev.upload(logits), dev.upload(drafts)
    want, got = dev.alloc(batch * 16), dev.alloc(batch * 16)
    hip.verify_accept(stream, lb, db, want, params)
    _noalloc(stream, lb, db, got, params)
    stream.sync()
    return want.read(np.int32), got.read(np.int32)


def test_noalloc_accept_matches_allocating_entry_point(dev, stream):
    rng = np.random.default_rng(90)
    big = hip.accept_params(hip.ACCEPT_STOCHASTIC, 16, 8, V, temperature=0.7, top_p=0.9, seed=5, step=3)
    assert hip.lib().yuuka_noalloc_accept_bytes(C.byref(big)) <= 8 << 20
    small = hip.accept_params(hip.ACCEPT_GREEDY, 1, 4, V)
    # two calls in a row, the second with a smaller input; then the other order
    for params, batch, k in ((big, 16, 8), (small, 1, 4), (small, 1, 4), (big, 16, 8)):
        want, got = _case(dev, stream, rng, batch, k, params)
        assert np.array_equal(want, got), (batch, k, want, got)


def test_noalloc_accept_rejects_beyond_its_scratch(dev, stream):
    batch, vocab = 8192, 16
    params = hip.accept_params(hip.ACCEPT_GREEDY, batch, 0, vocab)
    assert hip.lib().yuuka_noalloc_accept_bytes(C.byref(params)) > 8 << 20
    lb = dev.upload(np.zeros((batch, vocab), np.float32))
    res = dev.upload(np.full(batch * 4, -7, np.int32))
    with pytest.raises(hip.HipError) as e:
        _noalloc(stream, lb, None, res, params)
    assert "exceed the fixed scratch" in str(e.value)
    stream.sync()
    assert np.all(res.read(np.int32) == -7)
