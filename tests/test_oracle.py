"""Pins the C restatement (oracle/) against the reference's own known-answer
tests and against what the mathematics fixes. CPU only.

Reference tests restated here (paths in the reference tree):
  tensor/quant_test.go:14-35   TestFloat16RoundTrip
  tensor/quant_test.go:101-172 TestDequantizeQ4K / Q5K / Q6K
  tensor/quant_test.go:252-342 TestMatMulMatchesDequantizedDot
  engine/speculative_test.go:139-151 TestLookupDraft
  engine/sampling_test.go:8-36, 93-98 greedy / top-k=1 / single-token sampler
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def put_half(buf: np.ndarray, off: int, v: float) -> None:
    h = O.f32_to_f16(v)
    buf[off] = h & 0xFF
    buf[off + 1] = h >> 8


# ----------------------------------------------------------------- fp16

def test_float16_round_trip_reference_values():
    # tensor/quant_test.go:14-35
    for v in [0, 1, -1, 0.5, 65504, 6.103515625e-05, 5.960464477539063e-08, math.inf, -math.inf]:
        got = O.f16_to_f32(O.f32_to_f16(v))
        if math.isinf(v):
            assert math.isinf(got) and math.copysign(1, got) == math.copysign(1, v)
        elif v == 0:
            assert got == 0 and math.copysign(1, got) == math.copysign(1, v)
        else:
            assert abs(got - v) <= abs(v) * 0.001


def test_f16_to_f32_exhaustive_against_ieee():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ieee = bits.view(np.float16).astype(np.float32)
    ours = np.array([O.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ieee)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ieee[~nan].view(np.uint32))


def test_f32_to_f16_round_trips_every_finite_half():
    for h in range(0, 65536, 7):
        e = (h >> 10) & 0x1F
        if e == 0x1F:
            continue
        assert O.f32_to_f16(O.f16_to_f32(h)) == h


# -------------------------------------------------------------- dequant

def test_dequantize_q4k_reference_kat():
    # tensor/quant_test.go:101-128
    src = np.zeros(144, np.uint8)
    put_half(src, 0, 1)
    put_half(src, 2, 0)
    src[4:8] = 1
    src[12:16] = 1
    src[16:144] = 0x01
    dst = O.dequantize(O.Q4_K, src, 1, 256)[0]
    want = np.array([1.0 if i % 64 < 32 else 0.0 for i in range(256)], np.float32)
    assert np.array_equal(dst, want)


def test_dequantize_q5k_reference_kat():
    # tensor/quant_test.go:130-154
    src = np.zeros(176, np.uint8)
    put_half(src, 0, 1)
    put_half(src, 2, 0)
    src[4:8] = 1
    src[12:16] = 1
    src[16] = 0x55
    dst = O.dequantize(O.Q5_K, src, 1, 256)[0]
    for i in (0, 64, 128, 192):
        assert dst[i] == 16
    assert dst[1] == 0


def test_dequantize_q6k_reference_kat():
    # tensor/quant_test.go:156-172
    src = np.zeros(210, np.uint8)
    src[0] = 0x0F
    src[128] = 0x02
    src[192] = 1
    put_half(src, 208, 1)
    dst = O.dequantize(O.Q6_K, src, 1, 256)[0]
    assert dst[0] == 15 and dst[1] == -32


def pack_q4k_scales(sc, mn):
    """GGML 12-byte packing of eight 6-bit scales and mins (the inverse of
    getScaleMinK4, written from the format: the first four pairs sit in the
    low 6 bits of bytes 0-3 / 4-7; the last four keep their low nibbles in
    bytes 8-11 and their top two bits in the high bits of bytes 0-7)."""
    q = [0] * 12
    for j in range(4):
        q[j] = sc[j] & 63
        q[j + 4] = mn[j] & 63
    for j in range(4, 8):
        q[j + 4] = (sc[j] & 0x0F) | ((mn[j] & 0x0F) << 4)
        q[j - 4] |= (sc[j] >> 4) << 6
        q[j] |= (mn[j] >> 4) << 6
    return q


def test_q4k_scale_packing_and_nibble_order_sweep():
    rng = np.random.default_rng(7)
    for trial in range(64):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        d = np.float32(rng.uniform(0.001, 0.1))
        dm = np.float32(rng.uniform(0.001, 0.1))
        d = np.float32(np.float16(d))
        dm = np.float32(np.float16(dm))
        blk = np.zeros(144, np.uint8)
        blk[0:2] = np.array([d], np.float16).view(np.uint8)
        blk[2:4] = np.array([dm], np.float16).view(np.uint8)
        blk[4:16] = pack_q4k_scales(sc, mn)
        # element e: group j=e//64, low nibble for e%64 < 32 (sub-block 2j), else high.
        for e in range(256):
            j, l = e // 64, e % 64
            byte = 16 + 32 * j + (l % 32)
            if l < 32:
                blk[byte] = (blk[byte] & 0xF0) | q[e]
            else:
                blk[byte] = (blk[byte] & 0x0F) | (q[e] << 4)
        got = O.dequantize(O.Q4_K, blk, 1, 256)[0]
        want = np.empty(256, np.float32)
        for e in range(256):
            s = e // 32
            d1 = np.float32(d * np.float32(sc[s]))
            m1 = np.float32(dm * np.float32(mn[s]))
            want[e] = np.float32(np.float32(d1 * np.float32(q[e])) - m1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), trial


def test_q6k_element_order_sweep():
    """Element e of a Q6_K block: half n=e//128, quarter t=(e%128)//32, l=e%32;
    low/high nibble of ql[64n + 32(t&1) + l] for t<2 / t>=2, bits 2t..2t+1 of
    qh[32n+l], scale sc[8n + 2t + l//16]."""
    rng = np.random.default_rng(11)
    q6 = rng.integers(0, 64, 256)
    sc = rng.integers(-128, 128, 16).astype(np.int8)
    blk = np.zeros(210, np.uint8)
    for e in range(256):
        n, t, l = e // 128, (e % 128) // 32, e % 32
        qi = 64 * n + 32 * (t & 1) + l
        if t < 2:
            blk[qi] |= q6[e] & 0x0F
        else:
            blk[qi] |= (q6[e] & 0x0F) << 4
        blk[128 + 32 * n + l] |= (q6[e] >> 4) << (2 * t)
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = np.array([0.5], np.float16).view(np.uint8)
    got = O.dequantize(O.Q6_K, blk, 1, 256)[0]
    for e in range(256):
        n, t, l = e // 128, (e % 128) // 32, e % 32
        s = sc[8 * n + 2 * t + l // 16]
        want = np.float32(np.float32(np.float32(0.5) * np.float32(s)) * np.float32(q6[e] - 32))
        assert got[e] == want, e


# --------------------------------------------------------------- matmul

def _matmul_fixture(dtype, rows=3, cols=256):
    """Byte pattern of tensor/quant_test.go:252-342."""
    eb, bb = O.BLOCK[dtype]
    rb = cols // eb * bb
    data = np.zeros(rows * rb, np.uint8)
    for r in range(rows):
        row = data[r * rb:(r + 1) * rb]
        row[:] = [(r * 37 + i * 11) % 255 for i in range(rb)]
        if dtype == O.F32:
            row[:] = np.array([(i % 7) - 3 for i in range(cols)], np.float32).view(np.uint8)
        elif dtype == O.F16:
            row[:] = np.array([(i % 5) - 2 for i in range(cols)], np.float16).view(np.uint8)
        elif dtype == O.Q8_0:
            for i in range(cols // 32):
                put_half(row, i * 34, 0.03125)
        elif dtype in (O.Q4_K, O.Q5_K):
            for i in range(0, rb, bb):
                put_half(row, i, 0.25)
                put_half(row, i + 2, 0.125)
        elif dtype == O.Q6_K:
            for i in range(0, rb, bb):
                put_half(row, i + 208, 0.25)
    return data


@pytest.mark.parametrize("dtype", [O.F32, O.F16, O.Q8_0, O.Q4_K, O.Q5_K, O.Q6_K])
def test_matmul_matches_dequantized_dot(dtype):
    rows, cols = 3, 256
    data = _matmul_fixture(dtype, rows, cols)
    x = np.array([(i % 9) - 4 for i in range(cols)], np.float32)
    dec = O.dequantize(dtype, data, rows, cols)
    want = np.zeros(rows, np.float32)
    for r in range(rows):
        s = np.float32(0)
        for i in range(cols):
            s = np.float32(s + np.float32(dec[r, i] * x[i]))
        want[r] = s
    got = O.matmul(dtype, data, x, rows, cols)[0]
    assert np.max(np.abs(got - want)) <= 1e-5


def test_matmul_worker_split_is_rowwise_independent():
    rng = np.random.default_rng(3)
    from yuuka_amd import synth
    w = synth.quant_matrix(rng, O.Q4_K, 37, 512)
    x = rng.normal(size=(2, 512)).astype(np.float32)
    a = O.matmul(O.Q4_K, w, x, 37, 512, workers=1)
    b = O.matmul(O.Q4_K, w, x, 37, 512, workers=5)
    assert np.array_equal(a, b)


# ---------------------------------------------------------- draft / argmax

def test_lookup_draft_reference_vectors():
    # engine/speculative_test.go:139-151
    assert O.lookup_draft([1, 2, 3, 4, 1, 2, 3], 4, 2) == [4, 1, 2, 3]
    assert O.lookup_draft([1, 2, 3], 4, 2) == []
    assert O.lookup_draft([5, 5, 5, 5], 3, 2) == [5]


def test_argmax_first_maximum_and_nan_rules():
    assert O.argmax(np.array([0.5, 2.0, 1.0])) == 1
    assert O.argmax(np.array([1.0, 3.0, 3.0, 2.0])) == 1
    assert O.argmax(np.array([np.nan, 5.0, 7.0])) == 0
    assert O.argmax(np.array([1.0, np.nan, 0.5])) == 0
    assert O.argmax(np.array([-np.inf, -np.inf])) == 0
    rng = np.random.default_rng(5)
    for _ in range(50):
        v = rng.integers(-3, 4, 40).astype(np.float32)
        assert O.argmax(v) == int(np.argmax(v))  # numpy also returns the first maximum


# --------------------------------------------------------------- philox

def test_philox_random123_known_answers():
    # Published known-answer vectors of Philox4x32-10 (Random123 kat_vectors).
    assert O.philox([0, 0, 0, 0], [0, 0]) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert O.philox([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert O.philox([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0]) == \
        [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def test_philox_matches_rocrand_engine():
    for case in json.loads((GOLDEN / "philox_rocrand.json").read_text()):
        assert O.philox(case["ctr"], case["key"]) == case["out"]


def test_draw_counter_layout_and_range():
    u = O.draw(0, 0, 0, 0, 0)
    o = O.philox([0, 0, 0, 0], [0, 0])
    assert u == ((o[0] << 32 | o[1]) >> 11) / 2.0 ** 53
    us = [O.draw(7, s, r, q, p) for s in range(4) for r in range(4) for q in range(2) for p in range(2)]
    assert len(set(us)) == len(us) and all(0.0 <= x < 1.0 for x in us)


# -------------------------------------------------------------- sampler

def test_sampler_greedy_and_topk1():
    # engine/sampling_test.go:8-36: greedy and top-k=1 pick index 1
    for t, k in ((0.0, 0), (1.0, 1)):
        kept, w, total, best = O.target_weights(np.array([0.5, 2.0, 1.0], np.float32), t, k)
        assert best == 1 and w[1] / total == 1.0


def test_sampler_single_token():
    # ExampleSampler (sampling_test.go:93-98): V=1 -> token 0 with p = 1
    kept, w, total, best = O.target_weights(np.array([1.0], np.float32), 1.0)
    assert kept == 1 and w[0] / total == 1.0


def test_sampler_weights_are_tempered_softmax():
    rng = np.random.default_rng(2)
    logits = rng.normal(0, 3, 1000).astype(np.float32)
    logits[17] = -np.inf
    logits[23] = np.nan
    kept, w, total, best = O.target_weights(logits, 0.8)
    ok = np.isfinite(logits)
    z = logits[ok].astype(np.float64) / 0.8
    p = np.exp(z - z.max())
    p /= p.sum()
    assert kept == ok.sum()
    # the reference subtracts the maximum in float32 (sampling.go:96), which
    # moves each weight by at most a few float32 ulps of (logit - max) / T
    assert np.allclose((w / total)[ok], p, rtol=2e-6, atol=1e-15)
    assert w[17] == 0 and w[23] == 0
    assert best == int(np.nanargmax(np.where(ok, logits, -np.inf)))


def test_sampler_top_p_smallest_prefix():
    logits = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float64)).astype(np.float32)
    kept, w, total, _ = O.target_weights(logits, 1.0, 0, 0.7)
    assert kept == 2 and w[2] == 0 and w[3] == 0
    kept, w, total, _ = O.target_weights(logits, 1.0, 0, 0.5)
    assert kept == 1
    kept, w, total, _ = O.target_weights(logits, 1.0, 3, 1.0)
    assert kept == 3 and w[3] == 0


def test_sampler_top_p_zero_is_off_and_ties_keep_lowest_ids():
    """NewSampler maps top-p 0 to 1 (sampling.go:46-48); equal logits are
    ordered by id (sampling.go:84-89), so a cut inside a tie keeps the lowest
    ids, and -0 ties with +0."""
    logits = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float64)).astype(np.float32)
    kept, w, _, _ = O.target_weights(logits, 1.0, 0, 0.0)
    assert kept == 4 and (w > 0).all()
    flat = np.zeros(10, np.float32)
    flat[[1, 4, 6]] = -0.0
    kept, w, _, _ = O.target_weights(flat, 1.0, 3, 1.0)
    assert kept == 3 and np.flatnonzero(w).tolist() == [0, 1, 2]
    kept, w, _, _ = O.target_weights(flat, 1.0, 0, 0.25)  # 3 of 10 equal weights reach 0.25
    assert kept == 3 and np.flatnonzero(w).tolist() == [0, 1, 2]


# ------------------------------------------------------------ acceptance

def test_accept_greedy_onehot_reduces_to_string_compare():
    V = 16
    rows = np.zeros((4, V), np.float32)
    target = [3, 4, 5, 9]
    for i, t in enumerate(target):
        rows[i, t] = 1
    assert O.accept_greedy(rows, [3, 4, 5])[:2] == (3, 9)
    assert O.accept_greedy(rows, [3, 7, 5])[:2] == (1, 4)
    assert O.accept_greedy(rows, [1, 4, 5])[:2] == (0, 3)
    assert O.accept_greedy(rows[:1], [])[:2] == (0, 3)


def test_accept_stochastic_emits_the_target_marginal():
    """Speculative sampling with a one-hot draft must emit the first token with
    probability p exactly: P(x) = p(d)[x=d] + (1-p(d)) * p(x)/(1-p(d)) [x!=d]."""
    V = 6
    logits = np.array([[1.0, 0.2, -0.5, 0.7, 0.0, -1.0], [0.0] * 6], np.float32)
    _, w, total, _ = O.target_weights(logits[0], 0.8)
    p = w / total
    counts = np.zeros(V)
    n = 20000
    for step in range(n):
        a, nxt, _, _ = O.accept_stochastic(logits, [3], 0.8, seed=1, step=step, request=0)
        counts[3 if a == 1 else nxt] += 1
    expected = p * n
    chi2 = float(np.sum((counts - expected) ** 2 / expected))
    assert chi2 < 30.0, (counts, expected)  # 5 dof; p(chi2 > 30) ~ 1.5e-5


def test_accept_stochastic_greedy_temperature_is_greedy():
    rng = np.random.default_rng(4)
    logits = rng.normal(0, 3, (5, 100)).astype(np.float32)
    drafts = [int(np.argmax(logits[0])), int(np.argmax(logits[1])), 3, 4]
    g = O.accept_greedy(logits, drafts)[:2]
    s = O.accept_stochastic(logits, drafts, 0.0, 0, 0, 0)[:2]
    assert g == s


# --------------------------------------------------------------- model pieces

def test_gdn_scan_identities():
    ss, groups, rank = 8, 2, 2
    conv_dim = 2 * groups * ss + rank * ss
    rng = np.random.default_rng(9)
    state = rng.normal(size=(rank, ss, ss)).astype(np.float32)
    conv = rng.normal(size=(1, conv_dim)).astype(np.float32)
    out = np.zeros((1, rank, ss), np.float32)
    # decay 1 (alpha 0) and beta 0 leave the state unchanged; out = S^T q
    s0 = state.copy()
    O.lib().orc_gdn_scan(O._ptr(state), O._ptr(conv), O._ptr(np.zeros(rank, np.float32)),
                         O._ptr(np.zeros(rank, np.float32)), O._ptr(out), 1, groups, rank, ss, conv_dim)
    assert np.array_equal(state, s0)
    for h in range(rank):
        q = conv[0, (h % groups) * ss:(h % groups + 1) * ss]
        assert np.allclose(out[0, h], s0[h].T @ q, rtol=1e-5, atol=1e-5)
    # from S = 0, one token: S = beta k v^T, o = beta (k.q) v
    state = np.zeros((rank, ss, ss), np.float32)
    beta = np.array([0.5, 0.25], np.float32)
    O.lib().orc_gdn_scan(O._ptr(state), O._ptr(conv), O._ptr(np.zeros(rank, np.float32)),
                         O._ptr(beta), O._ptr(out), 1, groups, rank, ss, conv_dim)
    key_dim = groups * ss
    for h in range(rank):
        g = h % groups
        q = conv[0, g * ss:(g + 1) * ss]
        k = conv[0, key_dim + g * ss:key_dim + (g + 1) * ss]
        v = conv[0, 2 * key_dim + h * ss:2 * key_dim + (h + 1) * ss]
        assert np.allclose(state[h], beta[h] * np.outer(k, v), rtol=1e-5, atol=1e-6)
        assert np.allclose(out[0, h], beta[h] * np.dot(k, q) * v, rtol=1e-4, atol=1e-5)


def test_rmsnorm_and_rope_closed_forms():
    rng = np.random.default_rng(1)
    x = rng.normal(size=64).astype(np.float32)
    w = rng.normal(size=64).astype(np.float32)
    dst = np.zeros(64, np.float32)
    O.lib().orc_rmsnorm(O._ptr(dst), O._ptr(x), O._ptr(w), 64, 1e-6)
    want = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * w
    assert np.allclose(dst, want, rtol=1e-5)
    v = rng.normal(size=(2, 16)).astype(np.float32)
    v0 = v.copy()
    O.lib().orc_rope(O._ptr(v), 2, 16, 16, 8, 0, 10000.0)
    assert np.array_equal(v, v0)  # position 0 is the identity
    O.lib().orc_rope(O._ptr(v), 2, 16, 16, 8, 37, 10000.0)
    assert np.allclose(np.linalg.norm(v[:, :8], axis=1), np.linalg.norm(v0[:, :8], axis=1), rtol=1e-5)
    assert np.array_equal(v[:, 8:], v0[:, 8:])  # beyond rot_dim untouched
    assert abs(O.lib().orc_softplus(0.0) - math.log(2)) < 1e-7
    assert O.lib().orc_softplus(25.0) == 25.0


# ------------------------------------------------------------ MoE routing

def test_select_experts_against_sorting():
    """forward.go:393-439: the repeated strict-greater scan equals a stable
    sort by descending logit (lower index first on ties); the weights are the
    softmax over the selected logits."""
    rng = np.random.default_rng(4)
    for trial in range(50):
        E, used = int(rng.integers(1, 40)), 0
        used = int(rng.integers(1, E + 1))
        logits = rng.integers(-3, 4, E).astype(np.float32) if trial % 2 else rng.normal(0, 1, E).astype(np.float32)
        ids, w = O.select_experts(logits, used)
        order = np.lexsort((np.arange(E), -logits.astype(np.float64)))[:used]
        assert ids.tolist() == order.tolist()
        sel = logits[order].astype(np.float64)
        p = np.exp(sel - sel.max())
        np.testing.assert_allclose(w, p / p.sum(), rtol=1e-6)
        assert abs(float(w.sum()) - 1.0) < 1e-5


def test_select_experts_nan_and_more_slots_than_experts():
    logits = np.array([np.nan, 1.0, 2.0, np.nan], np.float32)
    ids, _ = O.select_experts(logits, 2)
    assert ids.tolist() == [0, 2]          # a NaN first candidate is never replaced
    ids, _ = O.select_experts(np.array([1.0, 3.0], np.float32), 2)
    assert ids.tolist() == [1, 0]
