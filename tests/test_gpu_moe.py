"""GPU parity of the MoE plan ops against the oracle restatement of
forward.go:320-439 (forwardMoEFFN, selectExperts) and tensor/quant.go MatMul:
the reference's v10 ops MOE_ROUTE / MOE_GATE_UP / MOE_DOWN / MOE_REDUCE_ADD
(layouts yuuka_hip.h:457-470) and the extension ops MOE_ROUTER /
MOE_COMBINE. Expert routing and bins are exact; expert GEMMs are held to
the 16-bit activation quantization budget of the verify GEMM."""
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


def _route(dev, stream, logits, used):
    rows, E = logits.shape
    cap = rows * used
    lb = dev.upload(logits.astype(np.float32))
    ids, w, cnt = dev.alloc(cap * 4), dev.alloc(cap * 4), dev.alloc(E * 4)
    ar, asl, aw = dev.alloc(E * cap * 4), dev.alloc(E * cap * 4), dev.alloc(E * cap * 4)
    cnt.write(np.full(E, -7, np.int32))  # every count must be written by the op
    plan = hip.Plan(dev)
    plan.add(hip.OP["MOE_ROUTE"], [lb, ids, w, cnt, ar, asl, aw], n=[rows, E, used])
    plan.execute(stream)
    stream.sync()
    plan.destroy()
    out = dict(ids=ids.read(np.int32).reshape(rows, used), w=w.read(np.float32).reshape(rows, used),
               counts=cnt.read(np.int32), arows=ar.read(np.int32).reshape(E, cap),
               aslots=asl.read(np.int32).reshape(E, cap), aw=aw.read(np.float32).reshape(E, cap))
    return out, (ids, w, cnt, ar, asl, aw)


def _bins(ids, used, E):
    rows = ids.shape[0]
    bins = [[] for _ in range(E)]
    for r in range(rows):
        for s in range(used):
            bins[ids[r, s]].append((r, s))
    return bins


# Up to 16 rows route and bin in one workgroup; more rows take the per-row
# and per-expert launches.
@pytest.mark.parametrize("rows,E,used", [(5, 256, 8), (40, 256, 8), (3, 16, 4), (7, 8, 8), (16, 1024, 16),
                                         (64, 512, 8), (33, 1024, 16), (200, 64, 4)])
def test_route_matches_select_experts(dev, stream, rows, E, used):
    rng = np.random.default_rng(rows * 1000 + E)
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    logits[0, 3] = logits[0, E - 1] = logits[0].max() + 0.5   # tie between the two largest
    if rows > 1:
        logits[1, :] = 0.25                               # every expert equal
    if rows > 2:
        logits[2, 5] = np.nan                             # NaN never wins later in the scan
        logits[2, 0] = np.nan                             # ...but keeps slot 0 when it starts it
    got, _ = _route(dev, stream, logits, used)
    for r in range(rows):
        ids, w = O.select_experts(logits[r], used)
        assert got["ids"][r].tolist() == ids.tolist(), r
        np.testing.assert_allclose(got["w"][r], w, rtol=2e-7, atol=0)
    bins = _bins(got["ids"], used, E)
    for e in range(E):
        assert got["counts"][e] == len(bins[e])
        for a, (r, s) in enumerate(bins[e]):
            assert (got["arows"][e, a], got["aslots"][e, a]) == (r, s)
            assert got["aw"][e, a].tobytes() == got["w"][r, s].tobytes()


def _quantized(x):
    """The kernel's activation rounding: per 256-element block, q = rint(x *
    (32639 / max|x|)) in float32, scale max|x| / 32639. Comparing against the
    oracle on these values pins the kernel's integer arithmetic tightly;
    comparing against the unrounded values bounds the quantization error."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, 256)
    m = np.abs(x).max(axis=1, keepdims=True)
    with np.errstate(divide="ignore"):
        inv = np.where(m > 0, np.float32(32639) / m, 0).astype(np.float32)
        sc = np.where(m > 0, m / np.float32(32639), 0).astype(np.float32)
    q = np.rint((x * inv).astype(np.float32))
    return (q.astype(np.float64) * sc).astype(np.float32).reshape(-1)


def _experts(rng, E, n, k):
    return synth.quant_matrix(rng, O.Q4_K, E * n, k, model_scale=True)


def _expert_rows(w, e, n, k):
    rb = O.row_bytes(O.Q4_K, k)
    return w[e * n * rb:(e + 1) * n * rb]


@pytest.mark.parametrize("rows,E,used,H,F", [(5, 64, 8, 2048, 512), (12, 8, 4, 512, 256), (40, 32, 8, 1024, 256)])
def test_grouped_gate_up_down_reduce(dev, stream, rows, E, used, H, F):
    """MOE_GATE_UP (plain and SwiGLU), MOE_DOWN and MOE_REDUCE_ADD over the
    bins of MOE_ROUTE, each against the oracle on the same inputs. The last
    case puts more than eight rows on some experts (several chunks)."""
    rng = np.random.default_rng(rows + E + H)
    logits = rng.normal(0, 1, (rows, E)).astype(np.float32)
    if E <= 8:
        logits[:, 0] += 3.0  # every row picks expert 0
    route, (ids_b, w_b, cnt, ar, asl, aw) = _route(dev, stream, logits, used)
    gate_w, up_w, down_w = _experts(rng, E, F, H), _experts(rng, E, F, H), _experts(rng, E, H, F)
    norm = rng.normal(0, 1, (rows, H)).astype(np.float32)
    gb, ub, db = dev.upload(gate_w), dev.upload(up_w), dev.upload(down_w)
    nb = dev.upload(norm)
    go, uo, act = dev.alloc(rows * used * F * 4), dev.alloc(rows * used * F * 4), dev.alloc(rows * used * F * 4)
    plan = hip.Plan(dev)
    plan.add(hip.OP["MOE_GATE_UP"], [nb, gb, ub, cnt, ar, asl, go, uo], n=[H, F, rows, E, used], u=[O.Q4_K])
    plan.add(hip.OP["MOE_GATE_UP"], [nb, gb, ub, cnt, ar, asl, act, None], n=[H, F, rows, E, used], u=[O.Q4_K],
             flags=hip.FLAG_MOE_SWIGLU)
    plan.execute(stream)
    stream.sync()
    plan.destroy()
    g = go.read(np.float32).reshape(rows, used, F)
    u = uo.read(np.float32).reshape(rows, used, F)
    a = act.read(np.float32).reshape(rows, used, F)
    ids = route["ids"]
    for r in range(rows):
        for s in range(used):
            e = int(ids[r, s])
            _check(g[r, s], O.matmul(O.Q4_K, _expert_rows(gate_w, e, F, H), norm[r], F, H)[0])
            _check(u[r, s], O.matmul(O.Q4_K, _expert_rows(up_w, e, F, H), norm[r], F, H)[0])
            _check(g[r, s], O.matmul(O.Q4_K, _expert_rows(gate_w, e, F, H), _quantized(norm[r]), F, H)[0], 2e-5)
            np.testing.assert_array_equal(a[r, s], O.silu_mul(g[r, s], u[r, s]))

    # down projection of the SwiGLU activations, then the weighted reduce
    eo = dev.alloc(rows * used * H * 4)
    x0 = rng.normal(0, 1, (rows, H)).astype(np.float32)
    xb = dev.upload(x0)
    plan = hip.Plan(dev)
    plan.add(hip.OP["MOE_DOWN"], [act, db, cnt, ar, asl, eo], n=[F, H, rows, E, used], u=[O.Q4_K])
    plan.add(hip.OP["MOE_REDUCE_ADD"], [xb, eo, w_b], n=[H, rows, used])
    plan.execute(stream)
    stream.sync()
    plan.destroy()
    out = eo.read(np.float32).reshape(rows, used, H)
    for r in range(rows):
        for s in range(used):
            e = int(ids[r, s])
            # SwiGLU outputs are heavy-tailed (a product of two projections): the
            # per-super-block 16-bit scale leaves up to ~1e-3 of the output rms.
            _check(out[r, s], O.matmul(O.Q4_K, _expert_rows(down_w, e, H, F), a[r, s], H, F)[0], 2e-3)
            _check(out[r, s], O.matmul(O.Q4_K, _expert_rows(down_w, e, H, F), _quantized(a[r, s]), H, F)[0], 2e-5)
    # reduce: float32 operations in slot order (forward.go:356-359, 388)
    want = x0.copy()
    w = route["w"]
    for r in range(rows):
        t = np.zeros(H, np.float32)
        for s in range(used):
            t = (t + (np.float32(w[r, s]) * out[r, s]).astype(np.float32)).astype(np.float32)
        want[r] = (want[r] + t).astype(np.float32)
    np.testing.assert_array_equal(xb.read(np.float32).reshape(rows, H), want)

    # the same ops on packed copies of the experts (yuuka_moe_pack_q4k,
    # FLAG_MOE_PACKED): every output bit-identical
    def packed(w, nrows, ncols):
        dst = dev.alloc(len(w))
        hip.moe_pack_q4k(stream, dst, dev.upload(w), nrows, ncols)
        return dst
    gp, up_, dp = packed(gate_w, E * F, H), packed(up_w, E * F, H), packed(down_w, E * H, F)
    go2, uo2, act2, eo2 = (dev.alloc(rows * used * F * 4), dev.alloc(rows * used * F * 4),
                           dev.alloc(rows * used * F * 4), dev.alloc(rows * used * H * 4))
    plan = hip.Plan(dev)
    plan.add(hip.OP["MOE_GATE_UP"], [nb, gp, up_, cnt, ar, asl, go2, uo2], n=[H, F, rows, E, used], u=[O.Q4_K],
             flags=hip.FLAG_MOE_PACKED)
    plan.add(hip.OP["MOE_GATE_UP"], [nb, gp, up_, cnt, ar, asl, act2, None], n=[H, F, rows, E, used], u=[O.Q4_K],
             flags=hip.FLAG_MOE_SWIGLU | hip.FLAG_MOE_PACKED)
    plan.add(hip.OP["MOE_DOWN"], [act2, dp, cnt, ar, asl, eo2], n=[F, H, rows, E, used], u=[O.Q4_K],
             flags=hip.FLAG_MOE_PACKED)
    plan.execute(stream)
    stream.sync()
    plan.destroy()
    np.testing.assert_array_equal(go2.read(np.float32).reshape(rows, used, F), g)
    np.testing.assert_array_equal(uo2.read(np.float32).reshape(rows, used, F), u)
    np.testing.assert_array_equal(act2.read(np.float32).reshape(rows, used, F), a)
    np.testing.assert_array_equal(eo2.read(np.float32).reshape(rows, used, H), out)


def test_router_and_combine_extension_ops(dev, stream):
    rng = np.random.default_rng(3)
    rows, E, H, used = 6, 64, 512, 4
    y = rng.normal(0, 1, (rows, H)).astype(np.float32)
    wr = rng.normal(0, 0.05, (E, H)).astype(np.float32)
    sv = rng.normal(0, 0.05, H).astype(np.float32)
    yb, wb, svb = dev.upload(y), dev.upload(wr), dev.upload(sv)
    lb, sg = dev.alloc(rows * E * 4), dev.alloc(rows * 4)
    plan = hip.Plan(dev)
    plan.add(hip.OP["MOE_ROUTER"], [yb, wb, lb, svb, sg], n=[H, E, rows])
    plan.execute(stream)
    stream.sync()
    plan.destroy()
    want = O.matmul(O.F32, wr.view(np.uint8).reshape(-1), y, E, H)
    np.testing.assert_allclose(lb.read(np.float32).reshape(rows, E), want, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(sg.read(np.float32), y @ sv, rtol=1e-5, atol=1e-5)

    eo = rng.normal(0, 1, (rows, used, H)).astype(np.float32)
    w = rng.uniform(0, 1, (rows, used)).astype(np.float32)
    so = rng.normal(0, 1, (rows, H)).astype(np.float32)
    g = rng.normal(0, 1, rows).astype(np.float32)
    x0 = rng.normal(0, 1, (rows, H)).astype(np.float32)
    xb, eob, wb2, sob, gb = dev.upload(x0), dev.upload(eo), dev.upload(w), dev.upload(so), dev.upload(g)
    plan = hip.Plan(dev)
    plan.add(hip.OP["MOE_COMBINE"], [xb, eob, wb2, sob, gb], n=[H, rows, used])
    plan.execute(stream)
    stream.sync()
    plan.destroy()
    want = x0.copy()
    for r in range(rows):
        t = np.zeros(H, np.float32)
        for s in range(used):
            t = (t + (w[r, s] * eo[r, s]).astype(np.float32)).astype(np.float32)
        sgm = np.float32(O.lib().orc_sigmoid(float(g[r])))
        t = (t + (sgm * so[r]).astype(np.float32)).astype(np.float32)
        want[r] = (want[r] + t).astype(np.float32)
    np.testing.assert_array_equal(xb.read(np.float32).reshape(rows, H), want)


def test_moe_pack_rejects_bad_arguments(dev, stream):
    """Row counts off the 16-row tile, columns off the super-block, buffers
    too small or overlapping are refused before any launch."""
    b = dev.alloc(64 * 1024 * 144 // 256 * 4)
    c = dev.alloc(64 * 1024 * 144 // 256 * 4)
    for rows, n_in, dst, src in [(15, 256, c, b), (16, 200, c, b), (4096, 1024, c, b), (16, 256, b, b)]:
        with pytest.raises(hip.HipError):
            hip.moe_pack_q4k(stream, dst, src, rows, n_in)
    hip.moe_pack_q4k(stream, c, b, 64, 1024)
    stream.sync()


def test_moe_ops_reject_bad_arguments(dev):
    plan = hip.Plan(dev)
    b = dev.alloc(1 << 16)
    with pytest.raises(hip.HipError):
        plan.add(hip.OP["MOE_ROUTE"], [b] * 7, n=[4, 8, 9])          # used > experts
    with pytest.raises(hip.Unsupported):
        plan.add(hip.OP["MOE_GATE_UP"], [b] * 8, n=[256, 16, 1, 1, 1], u=[O.Q6_K])
    with pytest.raises(hip.Unsupported):  # more rows than one grouped GEMM takes
        plan.add(hip.OP["MOE_GATE_UP"], [b] * 8, n=[256, 16, 513, 8, 2], u=[O.Q4_K])
    with pytest.raises(hip.HipError):
        plan.add(hip.OP["MOE_REDUCE_ADD"], [b, b, b], n=[1 << 20, 64, 8])  # overflow of the buffers
    plan.destroy()


def test_router_normal_logits(dev, stream):
    """ROUTER_NORMAL (router logits N(0,1)): the draws
    have mean 0 and variance 1, are the same for the same (seed, step, layer)
    and change with the step counter and the layer; the route op then picks
    distinct experts as uniform routing does (about E (1 - (1 - used/E)^rows)
    of them)."""
    rows, E, used = 40, 256, 8
    lb = dev.alloc(rows * E * 4)
    step = dev.upload(np.array([7], np.uint64))
    outs = []
    for layer, st in ((3, 7), (3, 7), (3, 8), (4, 7)):
        step.write(np.array([st], np.uint64))
        p = hip.Plan(dev)
        p.add(hip.OP["ROUTER_NORMAL"], [lb, step], n=[rows, E, 99, layer])
        p.execute(stream)
        stream.sync()
        outs.append(lb.read(np.float32, rows * E).reshape(rows, E))
        p.destroy()
    a = outs[0].astype(np.float64)
    assert abs(a.mean()) < 0.05 and abs(a.var() - 1.0) < 0.08, (a.mean(), a.var())
    assert np.all(np.isfinite(a))
    assert np.array_equal(outs[0], outs[1])
    assert not np.array_equal(outs[0], outs[2]) and not np.array_equal(outs[0], outs[3])
    # tail mass of a standard normal: P(|z| > 2) ~ 0.0455
    assert abs(np.mean(np.abs(a) > 2.0) - 0.0455) < 0.01
    ids = dev.alloc(rows * used * 4)
    w = dev.alloc(rows * used * 4)
    cnt, ar, asl, aw = dev.alloc(E * 4), dev.alloc(E * rows * used * 4), dev.alloc(E * rows * used * 4), \
        dev.alloc(E * rows * used * 4)
    p = hip.Plan(dev)
    p.add(hip.OP["MOE_ROUTE"], [lb, ids, w, cnt, ar, asl, aw], n=[rows, E, used])
    p.execute(stream)
    stream.sync()
    distinct = int((cnt.read(np.int32, E) > 0).sum())
    expect = E * (1 - (1 - used / E) ** rows)
    assert abs(distinct - expect) < 20, (distinct, expect)
    p.destroy()
