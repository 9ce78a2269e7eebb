"""Verify attention with a NaN score: the reference's attention kernels
compute expf(score - max) (kernels/hip/attention), so a key whose score is
NaN makes the softmax weights, and with them the query heads that attend to
it, NaN; every other head stays finite. The op (ATTN_VERIFY, the MFMA
kernel: F16 pool, 16 Q / 4 KV heads of 256, 64 rotated dimensions) must do
the same rather than give the NaN key a zero weight."""
from __future__ import annotations

import numpy as np
import pytest

from yuuka_amd import hip

pytestmark = pytest.mark.gpu


def test_nan_key_propagates_to_its_query_heads(dev, stream):
    heads, kvh, hd, rot, bs = 16, 4, 256, 64, 16
    kv_dim, rows, pos, cap = kvh * hd, 1, 64, 128
    rng = np.random.default_rng(3)
    q = rng.normal(0, 1, (rows, heads * 2 * hd)).astype(np.float32)
    k = rng.normal(0, 1, (rows, kv_dim)).astype(np.float32)
    v = rng.normal(0, 1, (rows, kv_dim)).astype(np.float32)
    blocks = cap // bs
    kpool = rng.normal(0, 1, (blocks * bs, kv_dim)).astype(np.float16)
    vpool = rng.normal(0, 1, (blocks * bs, kv_dim)).astype(np.float16)
    kpool[10, 2 * hd:3 * hd] = np.float16(np.nan)  # cached key 10 of KV head 2
    qb, kb, vb = dev.upload(q), dev.upload(k), dev.upload(v)
    kpb, vpb = dev.upload(kpool.view(np.uint16)), dev.upload(vpool.view(np.uint16))
    table = dev.upload(np.arange(blocks, dtype=np.int32))
    qn, kn = dev.upload(np.ones(hd, np.float32)), dev.upload(np.ones(hd, np.float32))
    rope = dev.alloc(rows * (rot // 2) * 8)
    out = dev.alloc(rows * heads * hd * 4)
    p = hip.Plan(dev)
    p.add(hip.OP["ROPE_TABLE"], [rope], n=[rows, rot, 0], f=[1.0e7])
    p.add(hip.OP["ATTN_VERIFY"], [qb, kb, vb, kpb, vpb, out, table, qn, kn, rope],
          n=[kvh, heads, hd, kv_dim, rows, 0], u=[bs, cap, 1, rot], f=[1.0 / 16.0, 1e-6])
    p.execute(stream, 0, pos, True)
    stream.sync()
    o = out.read(np.float32, rows * heads * hd).reshape(rows, heads, hd)
    group = heads // kvh
    for h in range(heads):
        if h // group == 2:
            assert np.all(np.isnan(o[0, h])), h
        else:
            assert np.all(np.isfinite(o[0, h])), h
    p.destroy()
