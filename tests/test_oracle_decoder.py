"""Closed-form pins of the oracle decoder's layer wiring (CPU only).

The oracle's orc_q35_forward restates model/qwen35/forward.go:116-389. Its
pieces (dequant, matmul, rmsnorm, rope, sigmoid/silu/softplus, the GDN scan,
selectExperts) are pinned in test_oracle.py; these tests pin how the layers
put them together. Each model is built from integer weight matrices packed
exactly as Q4_K (synth.q4k_from_int: identity, permutation and sign maps), so
every projection is known in closed form and a wrong head map, gate half,
softmax scale, conv tap order, residual or FFN wiring changes the result:

* attention (forward.go:157-226): a single key gives out_h = v_{h/group} *
  sigmoid(gate_h); zero keys give the mean of the values; two keys with the
  rotated dimensions zeroed give softmax([q.k0, q.k1] / sqrt(head_dim));
  the GQA map kvh = h / group is checked with distinct per-KV-head values;
* recurrent (forward.go:228-293): conv taps e_last pass the projection
  through SiLU; a tap on the oldest slot delays by kernel-1 tokens; the
  delta rule's first two tokens in closed form (S0 = 0);
* FFN (forward.go:295-315) and MoE (forward.go:320-389): zero weights make
  the layer the identity residual; one expert with a zero shared expert is
  the dense FFN bit for bit; two of four experts combine with the softmax
  of the selected router logits plus sigmoid(shared_gate . y) * shared(y);
* output head: logits = output . rmsnorm(x) * output_norm.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
from yuuka_amd import model as Mdl
from yuuka_amd import synth

EPS = 1e-6


def qmat(wint, d=1.0):
    wint = np.asarray(wint)
    return dict(data=synth.q4k_from_int(wint, d), rows=wint.shape[0], cols=wint.shape[1], dtype=Mdl.Q4_K)


def zmat(rows, cols):
    return qmat(np.zeros((rows, cols), np.int64), 0.0)


def f32mat(a):
    a = np.ascontiguousarray(a, np.float32)
    return dict(data=a.view(np.uint8).ravel(), rows=a.shape[0], cols=a.shape[1], dtype=Mdl.F32)


def eye(rows, cols, sign=1):
    m = np.zeros((rows, cols), np.int64)
    for i in range(min(rows, cols)):
        m[i, i] = sign
    return m


def rms(x, w):
    return O.rmsnorm_rows(np.atleast_2d(x).astype(np.float32), np.asarray(w, np.float32), EPS)[0].astype(np.float64)


def sig(x):
    return 1.0 / (1.0 + np.exp(-x))


def silu(x):
    return x * sig(x)


def softplus(x):
    return np.log1p(np.exp(x))


def dense(m):
    return O.dequantize(m["dtype"], m["data"], m["rows"], m["cols"]).astype(np.float64) \
        if m["dtype"] != Mdl.F32 else m["data"].view(np.float32).reshape(m["rows"], m["cols"]).astype(np.float64)


def rope(vec, heads, stride, rot, pos, base):
    v = np.ascontiguousarray(vec, np.float32).copy()
    O.lib().orc_rope(v.ctypes.data_as(C.c_void_p), heads, stride, 0, rot, pos, base)
    return v.astype(np.float64)


def close(got, want, tol=2e-5):
    scale = max(1.0, float(np.max(np.abs(want))))
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    assert err <= tol * scale, (err, scale)


def base_cfg(**kw):
    c = dict(n_layers=1, hidden=256, ffn=256, heads=4, kv_heads=2, head_dim=64, rope_dim=16, vocab=8,
             groups=2, rank=4, state_size=128, full_interval=1, capacity=64, block_size=16)
    c.update(kw)
    return Mdl.Q35Config(**c)


def emb_rows(rng, cfg):
    e = rng.integers(-8, 8, (cfg.vocab, cfg.hidden))
    return e, qmat(e, 0.25)


def run(cfg, w, tokens, kv_format=0):
    orc = O.Q35(cfg, w, kv_format=kv_format, workers=1)
    try:
        return orc.forward_residual(tokens).astype(np.float64)
    finally:
        orc.close()


def ffn_zero(cfg):
    return dict(ffn_gate=zmat(cfg.ffn, cfg.hidden), ffn_up=zmat(cfg.ffn, cfg.hidden),
                ffn_down=zmat(cfg.hidden, cfg.ffn), post_norm=np.ones(cfg.hidden, np.float32))


def model(cfg, emb, layers, rng):
    return dict(embedding=emb, output=qmat(rng.integers(-8, 8, (cfg.vocab, cfg.hidden)), 0.125),
                output_norm=(1 + rng.normal(0, 0.1, cfg.hidden)).astype(np.float32), layers=layers)


# ------------------------------------------------------------- attention

def attn_layer(cfg, rng, wk=None, zero_rot=False):
    """q rows of head h = unit rows picking y[h*hd + d]; gate rows = -unit
    rows of the same slice; k rows of KV head j pick y[j*hd + d] (or wk);
    v rows of KV head j pick y[128 + j*hd + d] with sign (-1)^j; o = I."""
    H, hd, nh, nkv = cfg.hidden, cfg.head_dim, cfg.heads, cfg.kv_heads
    wq = np.zeros((nh * 2 * hd, H), np.int64)
    for h in range(nh):
        for d in range(hd):
            if not (zero_rot and d < cfg.rope_dim):
                wq[h * 2 * hd + d, (h * hd + d) % H] = 1
            wq[h * 2 * hd + hd + d, (h * hd + d) % H] = -1
    if wk is None:
        wk = np.zeros((nkv * hd, H), np.int64)
        for j in range(nkv):
            for d in range(hd):
                if not (zero_rot and d < cfg.rope_dim):
                    wk[j * hd + d, (j * hd + d + 7) % H] = 1
    wv = np.zeros((nkv * hd, H), np.int64)
    for j in range(nkv):
        for d in range(hd):
            wv[j * hd + d, (128 + j * hd + d) % H] = (-1) ** j
    L = dict(attn_norm=(1 + rng.normal(0, 0.2, H)).astype(np.float32), q=qmat(wq), k=qmat(wk), v=qmat(wv),
             o=qmat(eye(H, nh * hd)), q_norm=(1 + rng.normal(0, 0.2, hd)).astype(np.float32),
             k_norm=(1 + rng.normal(0, 0.2, hd)).astype(np.float32))
    L.update(ffn_zero(cfg))
    return L


def attn_expected(cfg, L, xs):
    """Closed form of one attention layer over the rows xs (positions 0..)."""
    hd, nh, nkv = cfg.head_dim, cfg.heads, cfg.kv_heads
    group = nh // nkv
    Wq, Wk, Wv, Wo = dense(L["q"]), dense(L["k"]), dense(L["v"]), dense(L["o"])
    Ks, Vs, out_rows = [], [], []
    for p, x in enumerate(xs):
        y = rms(x, L["attn_norm"])
        qf, k, v = Wq @ y, Wk @ y, Wv @ y
        qf = qf.astype(np.float32).astype(np.float64)
        for h in range(nh):
            qf[h * 2 * hd:h * 2 * hd + hd] = rms(qf[h * 2 * hd:h * 2 * hd + hd], L["q_norm"])
        for j in range(nkv):
            k[j * hd:(j + 1) * hd] = rms(k[j * hd:(j + 1) * hd], L["k_norm"])
        qf = rope(qf, nh, 2 * hd, cfg.rope_dim, p, cfg.rope_base)
        k = rope(k, nkv, hd, cfg.rope_dim, p, cfg.rope_base)
        Ks.append(k)
        Vs.append(v)
        att = np.zeros(nh * hd)
        for h in range(nh):
            j = h // group
            q = qf[h * 2 * hd:h * 2 * hd + hd]
            s = np.array([q @ K[j * hd:(j + 1) * hd] for K in Ks]) / np.sqrt(hd)
            wgt = np.exp(s - s.max())
            wgt /= wgt.sum()
            o = sum(wgt[i] * Vs[i][j * hd:(j + 1) * hd] for i in range(len(Ks)))
            att[h * hd:(h + 1) * hd] = o * sig(qf[h * 2 * hd + hd:h * 2 * hd + 2 * hd])
        out_rows.append(x + Wo @ att)
    return np.array(out_rows)


def test_attention_single_key_is_gated_value():
    """One token: softmax over one key is 1, so head h outputs
    v_{h/group} * sigmoid(gate_h) whatever q and k are."""
    rng = np.random.default_rng(1)
    cfg = base_cfg()
    e, emb = emb_rows(rng, cfg)
    L = attn_layer(cfg, rng)
    got = run(cfg, model(cfg, emb, [L], rng), [3])
    x = 0.25 * e[3].astype(np.float64)
    y = rms(x, L["attn_norm"])
    hd = cfg.head_dim
    want = x.copy()
    for h in range(cfg.heads):
        j = h // (cfg.heads // cfg.kv_heads)
        v = (-1) ** j * y[128 + j * hd:128 + (j + 1) * hd]
        gate = -y[h * hd:(h + 1) * hd]
        want[h * hd:(h + 1) * hd] += v * sig(gate)
    close(got[0], want)
    # the GQA map h / group, not h % kv_heads: heads 1 and 2 differ in KV head
    assert not np.allclose(want[64:128] - x[64:128], 0)


def test_attention_zero_keys_average_values():
    """Zero key projections: every score is 0, the softmax is uniform and
    each row outputs the running mean of the values (causal)."""
    rng = np.random.default_rng(2)
    cfg = base_cfg()
    e, emb = emb_rows(rng, cfg)
    L = attn_layer(cfg, rng, wk=np.zeros((cfg.kv_heads * cfg.head_dim, cfg.hidden), np.int64))
    toks = [1, 5, 2, 7, 0]
    got = run(cfg, model(cfg, emb, [L], rng), toks)
    hd, g = cfg.head_dim, cfg.heads // cfg.kv_heads
    vals = []
    for p, t in enumerate(toks):
        x = 0.25 * e[t].astype(np.float64)
        y = rms(x, L["attn_norm"])
        vals.append(y)
        want = x.copy()
        for h in range(cfg.heads):
            j = h // g
            v = np.mean([(-1) ** j * yy[128 + j * hd:128 + (j + 1) * hd] for yy in vals], axis=0)
            want[h * hd:(h + 1) * hd] += v * sig(-y[h * hd:(h + 1) * hd])
        close(got[p], want)


def test_attention_two_keys_softmax_scale():
    """Rotated dimensions zeroed in q and k: two keys give
    softmax([q.k0, q.k1] / sqrt(head_dim)) exactly, at any position."""
    rng = np.random.default_rng(3)
    cfg = base_cfg()
    e, emb = emb_rows(rng, cfg)
    L = attn_layer(cfg, rng, zero_rot=True)
    toks = [4, 6]
    got = run(cfg, model(cfg, emb, [L], rng), toks)
    hd, g = cfg.head_dim, cfg.heads // cfg.kv_heads
    Wq, Wk = dense(L["q"]), dense(L["k"])
    xs = [0.25 * e[t].astype(np.float64) for t in toks]
    ys = [rms(x, L["attn_norm"]) for x in xs]
    want = xs[1].copy()
    for h in range(cfg.heads):
        j = h // g
        q = rms((Wq @ ys[1])[h * 2 * hd:h * 2 * hd + hd], L["q_norm"])
        ks = [rms((Wk @ y)[j * hd:(j + 1) * hd], L["k_norm"]) for y in ys]
        s = np.array([q @ k for k in ks]) / 8.0
        p1 = 1.0 / (1.0 + np.exp(s[0] - s[1]))
        vs = [(-1) ** j * y[128 + j * hd:128 + (j + 1) * hd] for y in ys]
        want[h * hd:(h + 1) * hd] += ((1 - p1) * vs[0] + p1 * vs[1]) * sig(-ys[1][h * hd:(h + 1) * hd])
    close(got[1], want)


@pytest.mark.parametrize("kv_format,tol", [(0, 2e-5), (1, 2e-3)])
def test_attention_general_with_rope(kv_format, tol):
    """Rotated keys over six positions (pinned rope at each position), F32
    and F16 KV rows."""
    rng = np.random.default_rng(4)
    cfg = base_cfg()
    e, emb = emb_rows(rng, cfg)
    L = attn_layer(cfg, rng)
    toks = [2, 3, 2, 6, 1, 3]
    got = run(cfg, model(cfg, emb, [L], rng), toks, kv_format=kv_format)
    want = attn_expected(cfg, L, [0.25 * e[t].astype(np.float64) for t in toks])
    close(got, want, tol)


# ------------------------------------------------------------- recurrent

def rec_layer(cfg, rng, taps=None):
    H, ss, G, R = cfg.hidden, cfg.state_size, cfg.groups, cfg.rank
    kd, inner = G * ss, R * ss
    cd = 2 * kd + inner
    wqkv = np.zeros((cd, H), np.int64)
    for i in range(kd):
        wqkv[i, i % H] = 1                       # q: y
        wqkv[kd + i, (H - 1 - i) % H] = 1        # k: y reversed
    for h in range(R):
        for j in range(ss):
            wqkv[2 * kd + h * ss + j, (h * 64 + j) % H] = (-1) ** h
    wz = np.zeros((inner, H), np.int64)
    for i in range(inner):
        wz[i, (3 * i + 1) % H] = 1
    if taps is None:
        taps = rng.normal(0, 0.5, (cd, cfg.conv_kernel))
    L = dict(attn_norm=(1 + rng.normal(0, 0.2, H)).astype(np.float32), qkv=qmat(wqkv), gate=qmat(wz),
             beta=qmat(rng.integers(-2, 3, (R, H)), 0.25), alpha=qmat(rng.integers(-2, 3, (R, H)), 0.25),
             out=qmat(rng.integers(-3, 4, (H, inner)), 0.125),
             conv=np.ascontiguousarray(taps, np.float32).ravel(),
             dt=rng.normal(0, 0.5, R).astype(np.float32), a=(-rng.uniform(0.2, 2.0, R)).astype(np.float32),
             ssm_norm=(1 + rng.normal(0, 0.2, ss)).astype(np.float32))
    L.update(ffn_zero(cfg))
    return L


def rec_expected(cfg, L, xs):
    """Closed form of one Gated DeltaNet layer over rows xs from zero state:
    conv over the last kernel inputs (taps oldest first, current last), SiLU,
    per-group L2 norms (q also / sqrt(state)), delta rule per head with key
    group h % groups, gated RMSNorm, out projection, residual."""
    ss, G, R, Kc = cfg.state_size, cfg.groups, cfg.rank, cfg.conv_kernel
    kd = G * ss
    Wqkv, Wz, Wb, Wa, Wout = (dense(L[n]) for n in ("qkv", "gate", "beta", "alpha", "out"))
    taps = L["conv"].astype(np.float64).reshape(-1, Kc)
    hist = [np.zeros(Wqkv.shape[0]) for _ in range(Kc - 1)]
    S = np.zeros((R, ss, ss))
    rows = []
    for x in xs:
        y = rms(x, L["attn_norm"])
        qkv, z = Wqkv @ y, Wz @ y
        beta = sig(Wb @ y)
        alpha = softplus(Wa @ y + L["dt"]) * L["a"]
        window = hist + [qkv]
        cv = silu(sum(taps[:, t] * window[t] for t in range(Kc)))
        hist = window[1:]
        q, k = cv[:kd].copy(), cv[kd:2 * kd].copy()
        for g in range(G):
            sl = slice(g * ss, (g + 1) * ss)
            q[sl] = q[sl] / np.sqrt(np.sum(q[sl] ** 2) + EPS) / np.sqrt(ss)
            k[sl] = k[sl] / np.sqrt(np.sum(k[sl] ** 2) + EPS)
        o = np.zeros(R * ss)
        for h in range(R):
            g = h % G
            qh, kh, vh = q[g * ss:(g + 1) * ss], k[g * ss:(g + 1) * ss], cv[2 * kd + h * ss:2 * kd + (h + 1) * ss]
            S[h] *= np.exp(alpha[h])
            d = (vh - S[h].T @ kh) * beta[h]
            S[h] += np.outer(kh, d)
            oh = S[h].T @ qh
            oh = rms(oh, L["ssm_norm"]) * silu(z[h * ss:(h + 1) * ss])
            o[h * ss:(h + 1) * ss] = oh
        rows.append(x + Wout @ o)
    return np.array(rows)


def rec_cfg():
    return base_cfg(full_interval=1000)   # layer 0 recurrent (config.go:280-282)


@pytest.mark.parametrize("taps", ["last", "oldest", "random"])
def test_recurrent_layer_closed_form(taps):
    rng = np.random.default_rng(5)
    cfg = rec_cfg()
    cd = 2 * cfg.groups * cfg.state_size + cfg.inner
    t = None
    if taps == "last":
        t = np.zeros((cd, cfg.conv_kernel))
        t[:, -1] = 1.0
    elif taps == "oldest":
        t = np.zeros((cd, cfg.conv_kernel))
        t[:, 0] = 1.0
        t[:, -1] = 0.5
    e, emb = emb_rows(rng, cfg)
    L = rec_layer(cfg, rng, t)
    toks = [1, 4, 4, 0, 6, 2]
    got = run(cfg, model(cfg, emb, [L], rng), toks)
    want = rec_expected(cfg, L, [0.25 * e[t_].astype(np.float64) for t_ in toks])
    close(got, want, 1e-4)


def test_recurrent_first_token_is_rank_one():
    """From zero state, token 0: S = k (v beta)^T, so o = c v with
    c = beta (k.q) for the normalized k and q of the head's key group; the
    out projection sees rmsnorm(c v) * silu(z) per head."""
    rng = np.random.default_rng(6)
    cfg = rec_cfg()
    cd = 2 * cfg.groups * cfg.state_size + cfg.inner
    t = np.zeros((cd, cfg.conv_kernel))
    t[:, -1] = 1.0
    e, emb = emb_rows(rng, cfg)
    L = rec_layer(cfg, rng, t)
    got = run(cfg, model(cfg, emb, [L], rng), [5])
    x = 0.25 * e[5].astype(np.float64)
    y = rms(x, L["attn_norm"])
    cv = silu(dense(L["qkv"]) @ y)
    z = dense(L["gate"]) @ y
    ss, G, kd = cfg.state_size, cfg.groups, cfg.groups * cfg.state_size
    o = np.zeros(cfg.inner)
    for h in range(cfg.rank):
        g = h % G
        q, k = cv[g * ss:(g + 1) * ss], cv[kd + g * ss:kd + (g + 1) * ss]
        q = q / np.sqrt(q @ q + EPS) / np.sqrt(ss)
        k = k / np.sqrt(k @ k + EPS)
        c = sig(dense(L["beta"])[h] @ y) * (k @ q)
        v = cv[2 * kd + h * ss:2 * kd + (h + 1) * ss]
        o[h * ss:(h + 1) * ss] = rms(c * v, L["ssm_norm"]) * silu(z[h * ss:(h + 1) * ss])
    close(got[0], x + dense(L["out"]) @ o, 1e-4)


# ------------------------------------------------------------ FFN and MoE

def test_zero_layer_is_identity_residual():
    """Every projection zero: attention and FFN add exactly 0."""
    rng = np.random.default_rng(7)
    cfg = base_cfg()
    e, emb = emb_rows(rng, cfg)
    H, hd = cfg.hidden, cfg.head_dim
    L = dict(attn_norm=np.ones(H, np.float32), q=zmat(cfg.heads * 2 * hd, H), k=zmat(cfg.kv_heads * hd, H),
             v=zmat(cfg.kv_heads * hd, H), o=zmat(H, cfg.heads * hd), q_norm=np.ones(hd, np.float32),
             k_norm=np.ones(hd, np.float32))
    L.update(ffn_zero(cfg))
    got = run(cfg, model(cfg, emb, [L], rng), [1, 2, 3])
    assert np.array_equal(got, 0.25 * e[[1, 2, 3]].astype(np.float64))


def dense_ffn_layer(cfg, rng):
    H, F = cfg.hidden, cfg.ffn
    L = attn_layer(cfg, rng)
    L.update(ffn_gate=qmat(rng.integers(-3, 4, (F, H)), 0.25), ffn_up=qmat(rng.integers(-3, 4, (F, H)), 0.25),
             ffn_down=qmat(rng.integers(-3, 4, (H, F)), 0.125), post_norm=(1 + rng.normal(0, 0.2, H)).astype(np.float32))
    return L


def test_dense_ffn_closed_form():
    """x + down(silu(gate y) * up y), y = rmsnorm(x) * post_norm, on top of
    the attention closed form."""
    rng = np.random.default_rng(8)
    cfg = base_cfg()
    e, emb = emb_rows(rng, cfg)
    L = dense_ffn_layer(cfg, rng)
    got = run(cfg, model(cfg, emb, [L], rng), [2])
    x = attn_expected(cfg, L, [0.25 * e[2].astype(np.float64)])[0]
    y = rms(x, L["post_norm"])
    want = x + dense(L["ffn_down"]) @ (silu(dense(L["ffn_gate"]) @ y) * (dense(L["ffn_up"]) @ y))
    close(got[0], want, 1e-4)


def moe_from_dense(cfg, L, rng, experts, used):
    """The dense layer's FFN as expert 0 of `experts`, other experts random,
    router f32 rows, zero shared expert and shared gate."""
    H, F = cfg.hidden, cfg.ffn
    M = {k: v for k, v in L.items() if not k.startswith("ffn_")}

    def stack(name, rows, cols):
        mats = [dense(L[name]) / 0.25 if name != "ffn_down" else dense(L[name]) / 0.125]
        mats += [rng.integers(-3, 4, (rows, cols)) for _ in range(experts - 1)]
        return np.concatenate([np.rint(m).astype(np.int64) for m in mats], axis=0)

    M.update(gate_exps=qmat(stack("ffn_gate", F, H), 0.25), up_exps=qmat(stack("ffn_up", F, H), 0.25),
             down_exps=qmat(stack("ffn_down", H, F), 0.125),
             router=f32mat(rng.normal(0, 1, (experts, H))), shared_gate_vec=np.zeros(H, np.float32),
             shared_gate=zmat(F, H), shared_up=zmat(F, H), shared_down=zmat(H, F))
    return M


def test_single_expert_moe_equals_dense_ffn():
    """One expert, top-1, zero shared expert: weight exp(0)/1 = 1 and the
    shared term sigmoid(0) * 0 = 0, so the residual equals the dense FFN
    model's bit for bit."""
    rng = np.random.default_rng(9)
    cfg = base_cfg()
    e, emb = emb_rows(rng, cfg)
    L = dense_ffn_layer(cfg, rng)
    toks = [3, 1, 6]
    w_dense = model(cfg, emb, [L], np.random.default_rng(0))
    w_moe = model(cfg, emb, [moe_from_dense(cfg, L, rng, 1, 1)], np.random.default_rng(0))
    mcfg = base_cfg(ffn=0, n_experts=1, n_experts_used=1, expert_ffn=cfg.ffn, shared_ffn=cfg.ffn)
    assert np.array_equal(run(mcfg, w_moe, toks), run(cfg, w_dense, toks))


def test_moe_two_of_four_experts_closed_form():
    """Top-2 of 4 experts by router logit (ties to the lower index), weights
    softmax over the two selected logits, plus sigmoid(shared_gate . y) times
    the shared expert."""
    rng = np.random.default_rng(10)
    cfg = base_cfg()
    H, F, E = cfg.hidden, cfg.ffn, 4
    e, emb = emb_rows(rng, cfg)
    L = dense_ffn_layer(cfg, rng)
    M = moe_from_dense(cfg, L, rng, E, 2)
    M.update(shared_gate_vec=rng.normal(0, 0.1, H).astype(np.float32),
             shared_gate=qmat(rng.integers(-3, 4, (F, H)), 0.25), shared_up=qmat(rng.integers(-3, 4, (F, H)), 0.25),
             shared_down=qmat(rng.integers(-3, 4, (H, F)), 0.125))
    mcfg = base_cfg(ffn=0, n_experts=E, n_experts_used=2, expert_ffn=F, shared_ffn=F)
    got = run(mcfg, model(mcfg, emb, [M], rng), [4])
    x = attn_expected(cfg, L, [0.25 * e[4].astype(np.float64)])[0]
    y = rms(x, M["post_norm"])
    logits = (dense(M["router"]) @ y)
    order = sorted(range(E), key=lambda i: (-logits[i], i))[:2]
    wsel = np.exp(logits[order] - logits[order].max())
    wsel /= wsel.sum()
    G, U, D = dense(M["gate_exps"]), dense(M["up_exps"]), dense(M["down_exps"])
    acc = np.zeros(H)
    for w_, i in zip(wsel, order):
        acc += w_ * (D[i * H:(i + 1) * H] @ (silu(G[i * F:(i + 1) * F] @ y) * (U[i * F:(i + 1) * F] @ y)))
    sh = dense(M["shared_down"]) @ (silu(dense(M["shared_gate"]) @ y) * (dense(M["shared_up"]) @ y))
    acc += sig(M["shared_gate_vec"].astype(np.float64) @ y) * sh
    close(got[0], x + acc, 1e-4)


# ------------------------------------------------- layer order and head

def test_two_layers_compose_in_order_and_head():
    """A recurrent layer then an attention layer (full_interval 2) equals the
    two closed forms composed in that order; the logits are
    output . (rmsnorm(x) * output_norm)."""
    rng = np.random.default_rng(11)
    cfg = base_cfg(n_layers=2, full_interval=2)
    e, emb = emb_rows(rng, cfg)
    R = rec_layer(cfg, rng)
    A = attn_layer(cfg, rng)
    w = model(cfg, emb, [R, A], rng)
    toks = [1, 2, 7]
    got = run(cfg, w, toks)
    xs = [0.25 * e[t].astype(np.float64) for t in toks]
    want = attn_expected(cfg, A, list(rec_expected(cfg, R, xs)))
    close(got, want, 1e-4)
    orc = O.Q35(cfg, w, kv_format=0, workers=1)
    logits, hid = orc.forward_hidden(toks)
    orc.close()
    close(hid, np.array([rms(r, w["output_norm"]) for r in want]), 1e-4)
    close(logits, hid.astype(np.float64) @ dense(w["output"]).T, 1e-4)
