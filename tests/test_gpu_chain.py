"""Chained streaming GEMMs (k_fchain.hip): a layer's out-projection, FFN
gate/up, FFN down and the next in-projection (or the LM head) run as one
persistent launch whose stages wait on device-scope counters. The chained
plan must give bit-identical verify logits and results to the same plan
with every projection launched on its own (the default), step after
step with different inputs (a stage that read stale activations from
another XCD's cache would differ), at the config-2 widths; and the
reference decoder still agrees within the north-star bar."""
from __future__ import annotations

import os
from dataclasses import replace

import numpy as np
import pytest

from oracle import oracle as O
from yuuka_amd import model as Mdl

pytestmark = pytest.mark.gpu


class _Chained:
    """Runs engine calls with chaining switched on (YUUKA_STREAM_CHAIN=1,
    read when a plan is executed or captured)."""

    def __enter__(self):
        os.environ["YUUKA_STREAM_CHAIN"] = "1"

    def __exit__(self, *a):
        os.environ.pop("YUUKA_STREAM_CHAIN", None)


def test_chained_equals_plain_config2_widths(dev):
    # 3 GDN + 1 attention layer: chains (GDN out, gate/up, down, GDN in),
    # (GDN out, gate/up, down, attention in), (attention o, gate/up, down,
    # LM head)
    cfg = replace(Mdl.QWEN35_4B_LIKE, n_layers=4, capacity=256)
    w = Mdl.make_weights(cfg, seed=33)
    os.environ.pop("YUUKA_STREAM_CHAIN", None)
    plain = Mdl.Engine(dev, cfg, w)
    with _Chained():
        chained = Mdl.Engine(dev, cfg, w)
    orc = O.Q35(cfg, w)
    try:
        rng = np.random.default_rng(8)
        prompt = rng.integers(0, cfg.vocab, 40).astype(np.int32)
        plain.prefill(prompt)
        with _Chained():
            chained.prefill(prompt)
        orc.forward(prompt)
        for step in range(4):
            rows = rng.integers(0, cfg.vocab, 5).astype(np.int32)
            print(f"chain step {step} rows {rows.tolist()}", flush=True)
            rp = plain.verify(rows)
            gp = plain.logits(5)
            with _Chained():
                rc = chained.verify(rows)
                gc = chained.logits(5)
            assert np.array_equal(gc.view(np.uint32), gp.view(np.uint32)), (step, float(np.abs(gc - gp).max()))
            assert tuple(rc[:2]) == tuple(rp[:2]), step
            if step == 0:
                snap, pos = orc.snapshot()
                want = orc.forward(rows, all_logits=True)
                orc.restore(snap, pos)
                for r in range(5):
                    rms = float(np.sqrt(np.mean(want[r].astype(np.float64) ** 2)))
                    assert np.all(np.abs(gc[r] - want[r]) <= 1e-2 * (np.abs(want[r]) + rms)), r
            orc.forward(rows[: int(rc[0]) + 1])
    finally:
        chained.close()
        plain.close()
        orc.close()
