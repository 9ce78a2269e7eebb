"""GPU parity of the fused verify GEMM (plan op GEMM_FUSED) against the oracle
restatement of tensor/quant.go MatMul on the same seeded inputs, with the
fused RMSNorm prologue (forward.go:460-470) and the residual / SwiGLU
epilogues. Tolerance: the 16-bit activation quantization error budget
relative to the output rms, plus the north-star 1e-2 relative bar."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from yuuka_amd import hip, synth

pytestmark = pytest.mark.gpu


def _check(got, want, budget=5e-4):
    want = want.astype(np.float64)
    rms = float(np.sqrt(np.mean(want ** 2))) + 1e-30
    err = np.abs(got.astype(np.float64) - want)
    assert float(err.max()) <= budget * rms, (float(err.max()), rms)
    assert np.all(err <= 1e-2 * (np.abs(want) + rms))


# Launches of more than 8 rows take the many-row kernel. Its MFMA operands
# are FP16, as in the reference's own many-row GEMM
# (kernels/hip/gemm/wmma_gemm.hip load_a_tile / load_b_tile): the activations
# round to FP16 (at most 2^-12 relative per element) and the Q6_K scale x
# quant products above 2048 to even integers, with FP32 accumulation. The
# largest error over a launch's outputs is then about 1e-3 of their rms
# (SwiGLU products about twice that); MANY_BUDGET bounds it, and the
# per-element 1e-2 bound of the verify logits is checked as everywhere.
MANY_BUDGET = 3e-3


def _run(dev, stream, x, segs, k, rows, epilogue=hip.EPI_STORE, norm=None, eps=1e-6, residuals=None):
    """segs: [(dtype, w_bytes_array, n_out)] -> list of outputs."""
    plan = hip.Plan(dev)
    xb = dev.upload(x.astype(np.float32))
    nb = dev.upload(norm.astype(np.float32)) if norm is not None else None
    outs, spec = [], []
    for i, (dt, w, n) in enumerate(segs):
        ob = dev.alloc(rows * n * 4)
        rb = None
        if residuals is not None:
            ob.write(residuals[i].astype(np.float32))
            rb = ob   # in-place residual: out = W y + out
        outs.append(ob)
        spec.append((dev.upload(w), dt, n, ob, rb))
    hip.gemm_fused_op(plan, xb, k, rows, spec, epilogue, nb, eps)
    plan.execute(stream)
    stream.sync()
    res = [o.read(np.float32).reshape(rows, n) for o, (_, _, n) in zip(outs, segs)]
    plan.destroy()
    return res


def _want(dt, w, n, k, y):
    return O.matmul(dt, w, y, n, k)


CASES = [
    # (segments [(dtype, n)], K, rows, norm)
    ([(O.Q4_K, 9216)], 2560, 5, False),             # configuration-1 shape
    ([(O.Q4_K, 6144), (O.Q4_K, 2048), (O.Q4_K, 16), (O.Q4_K, 16)], 2560, 5, True),  # GDN projections
    ([(O.Q4_K, 8192), (O.Q4_K, 1024), (O.Q6_K, 1024)], 2560, 5, True),              # attention q/k/v
    ([(O.Q4_K, 2560)], 9216, 5, False),             # down projection
    ([(O.Q4_K, 2560)], 2048, 5, False),             # GDN out projection
    ([(O.Q6_K, 3000)], 2560, 5, True),              # LM head shape (fewer rows)
    ([(O.Q4_K, 100)], 256, 1, False),
    ([(O.Q4_K, 333)], 1024, 8, True),
    ([(O.Q4_K, 300), (O.Q6_K, 77)], 1536, 12, False),
    ([(O.Q4_K, 64)], 9216, 16, False),              # K split into LDS chunks
    ([(O.Q6_K, 130)], 2560, 16, True),
]


@pytest.mark.parametrize("segs,k,rows,norm", CASES)
def test_fused_gemm_matches_oracle(dev, stream, segs, k, rows, norm):
    rng = np.random.default_rng(k * 7 + rows + len(segs))
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    g = rng.normal(1, 0.1, k).astype(np.float32) if norm else None
    ws = [synth.quant_matrix(rng, dt, n, k) for dt, n in segs]
    got = _run(dev, stream, x, [(dt, w, n) for (dt, n), w in zip(segs, ws)], k, rows, norm=g)
    y = O.rmsnorm_rows(x, g, 1e-6) if norm else x
    for (dt, n), w, gv in zip(segs, ws, got):
        _check(gv, _want(dt, w, n, k, y), budget=MANY_BUDGET if rows > 8 else 5e-4)


def test_fused_gemm_residual_epilogue(dev, stream):
    rng = np.random.default_rng(11)
    k, n, rows = 9216, 2560, 5
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    w = synth.quant_matrix(rng, O.Q4_K, n, k)
    res = rng.normal(0, 3, (rows, n)).astype(np.float32)
    got = _run(dev, stream, x, [(O.Q4_K, w, n)], k, rows, hip.EPI_RESIDUAL, residuals=[res])[0]
    prod = _want(O.Q4_K, w, n, k, x)
    _check(got - res, prod)


def test_fused_gemm_swiglu_epilogue(dev, stream):
    rng = np.random.default_rng(12)
    k, n, rows = 2560, 1000, 5
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    g = rng.normal(1, 0.1, k).astype(np.float32)
    wg = synth.quant_matrix(rng, O.Q4_K, n, k)
    wu = synth.quant_matrix(rng, O.Q4_K, n, k)
    got = _run(dev, stream, x, [(O.Q4_K, wg, n), (O.Q4_K, wu, n)], k, rows, hip.EPI_SWIGLU, norm=g)[0]
    y = O.rmsnorm_rows(x, g, 1e-6)
    want = O.silu_mul(_want(O.Q4_K, wg, n, k, y), _want(O.Q4_K, wu, n, k, y))
    _check(got, want, budget=1e-3)


def test_fused_gemm_repeatable_and_outliers(dev, stream):
    """Bitwise repeatable; a row of zeros stays zero; a 1e4 outlier in one
    super-block only costs that super-block's resolution."""
    rng = np.random.default_rng(13)
    k, n, rows = 2560, 700, 4
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    x[1] = 0.0
    x[2, 5] = 1e4
    w = synth.quant_matrix(rng, O.Q4_K, n, k)
    a = _run(dev, stream, x, [(O.Q4_K, w, n)], k, rows)[0]
    b = _run(dev, stream, x, [(O.Q4_K, w, n)], k, rows)[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert not np.any(a[1])
    want = _want(O.Q4_K, w, n, k, x)
    for r in (0, 2, 3):
        _check(a[r:r + 1], want[r:r + 1], budget=2e-3)


def test_fused_gemm_rejects_bad_ops(dev):
    plan = hip.Plan(dev)
    xb = dev.alloc(5 * 2560 * 4)
    wb = dev.alloc(synth.BLOCK_BYTES[O.Q4_K] * 10 * 64)
    ob = dev.alloc(5 * 64 * 4)
    with pytest.raises(hip.HipError):   # K not a multiple of 256
        hip.gemm_fused_op(plan, xb, 2500, 5, [(wb, O.Q4_K, 64, ob, None)])
    with pytest.raises(hip.HipError):   # 513 rows
        hip.gemm_fused_op(plan, xb, 2560, 513, [(wb, O.Q4_K, 64, ob, None)])
    with pytest.raises(hip.HipError):   # weight buffer too small for 65 rows
        hip.gemm_fused_op(plan, xb, 2560, 5, [(wb, O.Q4_K, 65, ob, None)])
    with pytest.raises(hip.HipError):   # Q8_0 weights
        hip.gemm_fused_op(plan, xb, 2560, 5, [(wb, O.Q8_0, 64, ob, None)])
    with pytest.raises(hip.HipError):   # residual epilogue without residual
        hip.gemm_fused_op(plan, xb, 2560, 5, [(wb, O.Q4_K, 64, ob, None)], hip.EPI_RESIDUAL)
    plan.destroy()


def _gated_head_norm(x, z, w, eps):
    """recurrent.go:39-50 per 128-element head: x * (scale * w) * silu(z),
    scale = 1/sqrt(mean(x^2) + eps) with a float64 sum (oracle silu)."""
    rows, k = x.shape
    out = np.empty_like(x)
    for r in range(rows):
        for h in range(k // 128):
            seg = x[r, h * 128:(h + 1) * 128]
            mean = np.float32(np.sum(seg.astype(np.float64) ** 2) / 128.0)
            scale = np.float32(1.0 / np.sqrt(np.float64(mean + np.float32(eps))))
            y = seg * (scale * w).astype(np.float32)
            out[r, h * 128:(h + 1) * 128] = y * O.silu_mul(z[r, h * 128:(h + 1) * 128], np.ones(128, np.float32))
    return out.astype(np.float32)


def test_fused_gemm_gated_head_norm_prologue(dev, stream):
    """Gated DeltaNet output projection: the prologue applies the per-head
    gated RMSNorm (gate = SiLU(z) supplied by its producer) before the GEMM."""
    rng = np.random.default_rng(21)
    k, n, rows, eps = 2048, 700, 5, 1e-6
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    z = rng.normal(0, 1, (rows, k)).astype(np.float32)
    w = rng.normal(1, 0.1, 128).astype(np.float32)
    gate = O.silu_mul(z, np.ones_like(z))
    wq = synth.quant_matrix(rng, O.Q4_K, n, k)
    plan = hip.Plan(dev)
    xb, gb, wb = dev.upload(x), dev.upload(gate), dev.upload(w)
    ob, wqb = dev.alloc(rows * n * 4), dev.upload(wq)
    bufs = [None] * 16
    bufs[0], bufs[2], bufs[6], bufs[14], bufs[15] = xb, wqb, ob, gb, wb
    plan.add(hip.OP["GEMM_FUSED"], bufs, n=[k, rows, n, 0, 0, 0], u=[O.Q4_K, 0], f=[eps])
    plan.execute(stream)
    stream.sync()
    got = ob.read(np.float32).reshape(rows, n)
    plan.destroy()
    y = _gated_head_norm(x, z, w, eps)
    _check(got, _want(O.Q4_K, wq, n, k, y))


def test_fused_gemm_silu_store(dev, stream):
    rng = np.random.default_rng(22)
    k, n, rows = 2560, 300, 5
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    wq = synth.quant_matrix(rng, O.Q4_K, n, k)
    plan = hip.Plan(dev)
    xb, wqb, ob = dev.upload(x), dev.upload(wq), dev.alloc(rows * n * 4)
    bufs = [None] * 14
    bufs[0], bufs[2], bufs[6] = xb, wqb, ob
    plan.add(hip.OP["GEMM_FUSED"], bufs, n=[k, rows, n, 0, 0, 0], u=[O.Q4_K, 0, 1], f=[1e-6])
    plan.execute(stream)
    stream.sync()
    got = ob.read(np.float32).reshape(rows, n)
    plan.destroy()
    prod = _want(O.Q4_K, wq, n, k, x)
    _check(got, O.silu_mul(prod, np.ones_like(prod)), budget=1e-3)


# Many rows (batched requests): one launch reads every weight once per 64 rows.
MANY = [
    ([(O.Q4_K, 1000)], 2560, 9, True),
    ([(O.Q4_K, 8192), (O.Q4_K, 1024), (O.Q6_K, 1024)], 2560, 40, True),   # attention q/k/v, 8 requests x 5
    ([(O.Q6_K, 3001)], 2560, 64, True),                                   # LM head shape
    ([(O.Q4_K, 2560)], 9216, 65, False),                                  # FFN down, two row blocks
    ([(O.Q4_K, 700), (O.Q4_K, 130), (O.Q4_K, 16), (O.Q4_K, 16)], 4096, 144, True),  # 16 requests x 9
    ([(O.Q6_K, 520)], 12288, 17, False),
]


@pytest.mark.parametrize("segs,k,rows,norm", MANY)
def test_fused_gemm_many_rows(dev, stream, segs, k, rows, norm):
    rng = np.random.default_rng(k * 3 + rows + len(segs))
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    g = rng.normal(1, 0.1, k).astype(np.float32) if norm else None
    ws = [synth.quant_matrix(rng, dt, n, k) for dt, n in segs]
    got = _run(dev, stream, x, [(dt, w, n) for (dt, n), w in zip(segs, ws)], k, rows, norm=g)
    y = O.rmsnorm_rows(x, g, 1e-6) if norm else x
    for (dt, n), w, gv in zip(segs, ws, got):
        _check(gv, _want(dt, w, n, k, y), budget=MANY_BUDGET)


def test_fused_gemm_many_rows_epilogues(dev, stream):
    """SwiGLU, residual, output maps and the gated head norm at 37 rows."""
    rng = np.random.default_rng(31)
    k, n, rows = 2048, 520, 37
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    g = rng.normal(1, 0.1, k).astype(np.float32)
    wg = synth.quant_matrix(rng, O.Q4_K, n, k)
    wu = synth.quant_matrix(rng, O.Q4_K, n, k)
    y = O.rmsnorm_rows(x, g, 1e-6)
    got = _run(dev, stream, x, [(O.Q4_K, wg, n), (O.Q4_K, wu, n)], k, rows, hip.EPI_SWIGLU, norm=g)[0]
    _check(got, O.silu_mul(_want(O.Q4_K, wg, n, k, y), _want(O.Q4_K, wu, n, k, y)), budget=2 * MANY_BUDGET)
    res = rng.normal(0, 3, (rows, n)).astype(np.float32)
    got = _run(dev, stream, x, [(O.Q4_K, wg, n)], k, rows, hip.EPI_RESIDUAL, residuals=[res])[0]
    _check(got - res, _want(O.Q4_K, wg, n, k, x), budget=MANY_BUDGET)
    # gated head norm prologue + SiLU output map
    z = rng.normal(0, 1, (rows, k)).astype(np.float32)
    w = rng.normal(1, 0.1, 128).astype(np.float32)
    gate = O.silu_mul(z, np.ones_like(z))
    plan = hip.Plan(dev)
    xb, gb, wb = dev.upload(x), dev.upload(gate), dev.upload(w)
    ob, wqb = dev.alloc(rows * n * 4), dev.upload(wg)
    bufs = [None] * 16
    bufs[0], bufs[2], bufs[6], bufs[14], bufs[15] = xb, wqb, ob, gb, wb
    plan.add(hip.OP["GEMM_FUSED"], bufs, n=[k, rows, n, 0, 0, 0], u=[O.Q4_K, 0, 1], f=[1e-6])
    plan.execute(stream)
    stream.sync()
    got = ob.read(np.float32).reshape(rows, n)
    plan.destroy()
    prod = _want(O.Q4_K, wg, n, k, _gated_head_norm(x, z, w, 1e-6))
    _check(got, O.silu_mul(prod, np.ones_like(prod)), budget=2 * MANY_BUDGET)


@pytest.mark.parametrize("k_a", [9216, 2048])
def test_many_rows_pair_reduce_and_prologue_in_one_launch(dev, stream, k_a):
    """A split-K residual GEMM followed by a GEMM that normalises its output
    (the FFN down -> next in-projection and out-projection -> FFN gate/up
    pairs of a batched step) runs with the split reduction and the second
    prologue in one kernel. Executed that way (plan.execute) and op by op
    (execute_profiled, which pairs nothing), every output is bit-identical,
    and both match the oracle. With k_a = 2048 the second GEMM's quantized
    rows do not fit before the first one's partial sums, so its workspace
    moves behind them (a leading K = 9216 launch makes the plan's workspace
    large enough, as the down projection does in the engine's plans)."""
    rng = np.random.default_rng(77 + k_a)
    rows, h, f = 144, 2560, 1536
    x_a = rng.normal(0, 1, (rows, k_a)).astype(np.float32)
    res0 = rng.normal(0, 2, (rows, h)).astype(np.float32)
    g = rng.normal(1, 0.1, h).astype(np.float32)
    w_a = synth.quant_matrix(rng, O.Q4_K, h, k_a)
    w_g = synth.quant_matrix(rng, O.Q4_K, f, h)
    w_u = synth.quant_matrix(rng, O.Q6_K, f, h)
    x_big = rng.normal(0, 1, (rows, 9216)).astype(np.float32)
    w_big = synth.quant_matrix(rng, O.Q4_K, 512, 9216)
    plan = hip.Plan(dev)
    xa, xb, gb = dev.upload(x_a), dev.upload(x_big), dev.upload(g)
    hbuf = dev.alloc(rows * h * 4)
    ob, og, ou = dev.alloc(rows * 512 * 4), dev.alloc(rows * f * 4), dev.alloc(rows * f * 4)
    wa, wg, wu, wbig = dev.upload(w_a), dev.upload(w_g), dev.upload(w_u), dev.upload(w_big)
    hip.gemm_fused_op(plan, xb, 9216, rows, [(wbig, O.Q4_K, 512, ob, None)])  # sizes the workspace
    hip.gemm_fused_op(plan, xa, k_a, rows, [(wa, O.Q4_K, h, hbuf, hbuf)], hip.EPI_RESIDUAL)
    hip.gemm_fused_op(plan, hbuf, h, rows, [(wg, O.Q4_K, f, og, None), (wu, O.Q6_K, f, ou, None)], norm=gb)
    outs = []
    for run in (plan.execute, plan.execute_profiled):
        hbuf.write(res0)
        run(stream)
        stream.sync()
        outs.append([b.read(np.float32).copy() for b in (hbuf, og, ou)])
    plan.destroy()
    for a, b in zip(*outs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    hh = outs[0][0].reshape(rows, h)
    _check(hh - res0, _want(O.Q4_K, w_a, h, k_a, x_a), budget=MANY_BUDGET)
    y = O.rmsnorm_rows(hh, g, 1e-6)
    _check(outs[0][1].reshape(rows, f), _want(O.Q4_K, w_g, f, h, y), budget=MANY_BUDGET)
    _check(outs[0][2].reshape(rows, f), _want(O.Q6_K, w_u, f, h, y), budget=MANY_BUDGET)


def test_many_rows_reduce_and_rmsnorm_in_one_launch(dev, stream):
    """A split-K residual GEMM whose output the next RMSNORM_BATCH normalises
    (out-projection -> the MoE FFN's norm) runs with the split reduction and
    the RMSNorm in one kernel. Executed that way (plan.execute) and op by op
    (execute_profiled, which pairs nothing), both outputs are bit-identical,
    and they match the oracle. A narrow output (8 workgroups of channels)
    over a deep K makes the launch split K."""
    rng = np.random.default_rng(91)
    rows, h, k = 40, 1024, 8192
    x = rng.normal(0, 1, (rows, k)).astype(np.float32)
    res0 = rng.normal(0, 2, (rows, h)).astype(np.float32)
    g = rng.normal(1, 0.1, h).astype(np.float32)
    w = synth.quant_matrix(rng, O.Q4_K, h, k)
    plan = hip.Plan(dev)
    xb, gb, wb = dev.upload(x), dev.upload(g), dev.upload(w)
    hbuf, yb = dev.alloc(rows * h * 4), dev.alloc(rows * h * 4)
    hip.gemm_fused_op(plan, xb, k, rows, [(wb, O.Q4_K, h, hbuf, hbuf)], hip.EPI_RESIDUAL)
    plan.add(hip.OP["RMSNORM_BATCH"], [hbuf, gb, yb], n=[h, rows, h, h], f=[1e-6])
    outs = []
    for run in (plan.execute, plan.execute_profiled):
        hbuf.write(res0)
        run(stream)
        stream.sync()
        outs.append([b.read(np.float32).copy() for b in (hbuf, yb)])
    plan.destroy()
    for a, b in zip(*outs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    hh = outs[0][0].reshape(rows, h)
    _check(hh - res0, _want(O.Q4_K, w, h, k, x), budget=MANY_BUDGET)
    # the float64 sum of squares is added in a different order from the
    # oracle's sequential one: at most a last-bit difference of the scale
    np.testing.assert_allclose(outs[0][1].reshape(rows, h), O.rmsnorm_rows(hh, g, 1e-6), rtol=1e-6, atol=0)


def test_many_rows_swiglu_pair_reduce_and_prologue_in_one_launch(dev, stream):
    """A split-K SwiGLU GEMM (FFN gate/up) followed by the GEMM that reads its
    output (FFN down): the split reduction with SiLU(gate) * up and the down
    prologue run as one kernel. Executed that way (plan.execute) and op by op
    (execute_profiled), every output is bit-identical, and both match the
    oracle. 68 rows (one block of five row tiles) split the gate/up launch."""
    rng = np.random.default_rng(93)
    rows, h, f = 68, 2048, 4096
    x = rng.normal(0, 1, (rows, h)).astype(np.float32)
    res0 = rng.normal(0, 2, (rows, h)).astype(np.float32)
    g = rng.normal(1, 0.1, h).astype(np.float32)
    w_g, w_u = synth.quant_matrix(rng, O.Q4_K, f, h), synth.quant_matrix(rng, O.Q4_K, f, h)
    w_d = synth.quant_matrix(rng, O.Q4_K, h, f)
    plan = hip.Plan(dev)
    xb, gb = dev.upload(x), dev.upload(g)
    wg, wu, wd = dev.upload(w_g), dev.upload(w_u), dev.upload(w_d)
    hb, ob = dev.alloc(rows * f * 4), dev.alloc(rows * h * 4)
    hip.gemm_fused_op(plan, xb, h, rows, [(wg, O.Q4_K, f, hb, None), (wu, O.Q4_K, f, None, None)], hip.EPI_SWIGLU,
                      norm=gb)
    hip.gemm_fused_op(plan, hb, f, rows, [(wd, O.Q4_K, h, ob, ob)], hip.EPI_RESIDUAL)
    outs = []
    for run in (plan.execute, plan.execute_profiled):
        ob.write(res0)
        run(stream)
        stream.sync()
        outs.append([b.read(np.float32).copy() for b in (hb, ob)])
    plan.destroy()
    for a, b in zip(*outs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    y = O.rmsnorm_rows(x, g, 1e-6)
    hh = outs[0][0].reshape(rows, f)
    want_h = O.silu_mul(_want(O.Q4_K, w_g, f, h, y), _want(O.Q4_K, w_u, f, h, y))
    _check(hh, want_h, budget=MANY_BUDGET * 4)
    _check(outs[0][1].reshape(rows, h) - res0, _want(O.Q4_K, w_d, h, f, hh), budget=MANY_BUDGET)
