"""The v10 verify plan exactly as the unchanged Go engine submits it, through
the C ABI, against the CPU reference decoder.

GoSession below restates engine/gpu/plan.go:569-682 buildPrefillPlan in its
prefillAllLogits form (the plan Session.PrefillLogits runs,
engine/gpu/session.go:246-303) with the op layouts of backend/hip/hip.go:
EMBEDDING_BATCH, then per layer RMSNORM_BATCH -> projections (LM_HEAD /
GEMV_BATCH / GEMM as hip.SelectPrefillPath picks them,
backend/hip/dispatch.go:49-123) -> RMSNORM_HEADS_BATCH -> ROPE_BATCH ->
KV_WRITE_BATCH_PAGED -> ATTENTION_PREFILL_PAGED, or RECURRENT_CHUNK with the
state updated in place; the FFN as GEMM_SWIGLU or LM_HEAD pair + SILU_MUL,
down projection and ADD; RMSNORM_BATCH + LM_HEAD over every row. No op
carries an extension flag. The prompt is prefilled with the same plan form
in chunks of at most 16 rows, as speculative verification would call it.
Same logit bar as the engine tests: |gpu - cpu| <= 1e-2 (|cpu| + rms(row)).
"""
from __future__ import annotations

import math
from dataclasses import replace

import numpy as np
import pytest

from oracle import oracle as O
from yuuka_amd import hip
from yuuka_amd import model as Mdl

pytestmark = pytest.mark.gpu

OP = dict(SILU_MUL=9, ADD=10, GEMM=16, GEMV_BATCH=17, RMSNORM_BATCH=18, RMSNORM_HEADS_BATCH=19, ROPE_BATCH=20,
          RECURRENT_CHUNK=23, EMBEDDING_BATCH=24, KV_WRITE_BATCH_PAGED=28, ATTENTION_PREFILL_PAGED=29,
          GEMM_SWIGLU=34, LM_HEAD=37)
MAX_LM_HEAD_ROWS = 16
LM_HEAD_MIN_OUTPUTS = 1024


def select_path(dtype, rows, n_in, n_out):
    """backend/hip/dispatch.go:49-123 for the K-quant weights of the model
    (F16 weights are not used): 'stream' (LM_HEAD), 'gemv' (GEMV_BATCH) or
    'wmma' (GEMM)."""
    if rows <= 0:
        return "gemv"
    if 0 < rows <= MAX_LM_HEAD_ROWS and n_in % 256 == 0 and n_out >= LM_HEAD_MIN_OUTPUTS:
        return "stream"
    if n_in % 256 == 0 and n_out >= 64 and rows >= 128:
        return "mmq"
    if rows < 4 or (n_in > n_out and rows < 8):
        return "gemv"
    return "wmma"


def _close(got, want, what=""):
    want = np.atleast_2d(want)
    got = np.atleast_2d(got)
    for r in range(want.shape[0]):
        rms = float(np.sqrt(np.mean(want[r].astype(np.float64) ** 2)))
        err = np.abs(got[r].astype(np.float64) - want[r])
        assert np.all(err <= 1e-2 * (np.abs(want[r]) + rms)), (what, r, float(err.max()), rms)


class GoSession:
    """Device weights, the m.prefill activation buffers and one session's KV
    pool, block table and recurrent state, as engine/gpu allocates them."""

    def __init__(self, dev, cfg, w):
        self.dev, self.cfg, self.w = dev, cfg, w
        self.stream = hip.Stream(dev)
        up = dev.upload
        self.wd = dict(embedding=up(w["embedding"]["data"]), output=up(w["output"]["data"]),
                       output_norm=up(w["output_norm"]), layers=[])
        for L in w["layers"]:
            self.wd["layers"].append({k: up(v["data"] if isinstance(v, dict) else v) for k, v in L.items()})
        c, R = cfg, MAX_LM_HEAD_ROWS
        self.conv_dim = 2 * c.groups * c.state_size + c.inner
        f = lambda n: dev.alloc(max(4, n * 4))  # noqa: E731
        self.x, self.norm, self.tmp = f(R * c.hidden), f(R * c.hidden), f(R * c.hidden)
        self.q, self.k, self.v = f(R * c.heads * c.head_dim * 2), f(R * c.kv_heads * c.head_dim), \
            f(R * c.kv_heads * c.head_dim)
        self.attn = f(R * c.heads * c.head_dim)
        self.qkv, self.z, self.conv = f(R * self.conv_dim), f(R * c.inner), f(R * self.conv_dim)
        self.alpha, self.beta, self.gdn = f(R * c.rank), f(R * c.rank), f(R * c.inner)
        self.ffn_gate, self.ffn_up = f(R * c.ffn), f(R * c.ffn)
        self.tokens = f(R)
        self.logits = f(R * c.vocab)
        blocks = (c.capacity + c.block_size - 1) // c.block_size
        self.table = up(np.arange(blocks, dtype=np.int32))
        kvb = blocks * c.block_size * c.kv_heads * c.head_dim * 2  # F16 rows
        self.pool_k, self.pool_v, self.conv_state, self.rec_state = {}, {}, {}, {}
        for i in range(c.n_layers):
            if c.is_recurrent(i):
                self.conv_state[i] = up(np.zeros((c.conv_kernel - 1) * self.conv_dim, np.float32))
                self.rec_state[i] = up(np.zeros(c.rank * c.state_size * c.state_size, np.float32))
            else:
                self.pool_k[i], self.pool_v[i] = up(np.zeros(kvb, np.uint8)), up(np.zeros(kvb, np.uint8))
        self.position = 0
        self.plans = {}

    # hip.go Add* layouts -------------------------------------------------
    @staticmethod
    def matmul(plan, path, w, dtype, x, out, n_in, n_out, rows):
        code = {"stream": OP["LM_HEAD"], "gemv": OP["GEMV_BATCH"], "wmma": OP["GEMM"]}[path]
        plan.add(code, [w, x, out], n=[n_in, n_out, rows], u=[dtype])

    def rmsnorm_batch(self, plan, src, weight, dst, rows, cols):
        plan.add(OP["RMSNORM_BATCH"], [src, weight, dst], n=[cols, rows, cols, cols], f=[self.cfg.eps])

    def build(self, rows):
        """engine/gpu/plan.go:569-682 with outputMode = prefillAllLogits."""
        c, W = self.cfg, self.wd
        p = hip.Plan(self.dev)
        H, hd = c.hidden, c.head_dim
        emb = self.w["embedding"]
        row_bytes = O.row_bytes(emb["dtype"], H)
        p.add(OP["EMBEDDING_BATCH"], [W["embedding"], self.x, self.tokens], n=[H, rows, row_bytes, c.vocab],
              u=[emb["dtype"]])
        for i in range(c.n_layers):
            Lw, Ld = self.w["layers"][i], W["layers"][i]
            self.rmsnorm_batch(p, self.x, Ld["attn_norm"], self.norm, rows, H)

            def proj(name, out, n_out, n_in=H, x=self.norm):
                dt = Lw[name]["dtype"]
                self.matmul(p, select_path(dt, rows, n_in, n_out), Ld[name], dt, x, out, n_in, n_out, rows)

            if c.is_recurrent(i):  # plan.go:848-913
                proj("qkv", self.qkv, self.conv_dim)
                proj("gate", self.z, c.inner)
                proj("beta", self.beta, c.rank)
                proj("alpha", self.alpha, c.rank)
                bufs = [self.conv_state[i], self.rec_state[i], self.qkv, self.z, self.alpha, self.beta, Ld["conv"],
                        Ld["dt"], Ld["a"], Ld["ssm_norm"], self.gdn, self.conv]
                p.add(OP["RECURRENT_CHUNK"], bufs, n=[rows, c.groups, c.rank, c.state_size, self.conv_dim, c.inner],
                      u=[c.conv_kernel], f=[c.eps, 1.0 / math.sqrt(c.state_size)])
                proj("out", self.tmp, H, n_in=c.inner, x=self.gdn)
                p.add(OP["ADD"], [self.x, self.tmp], n=[rows * H])
            else:  # plan.go:684-846
                kv_dim, q_dim = c.kv_heads * hd, c.heads * hd * 2
                proj("q", self.q, q_dim)
                proj("k", self.k, kv_dim)
                proj("v", self.v, kv_dim)
                p.add(OP["RMSNORM_HEADS_BATCH"], [self.k, Ld["k_norm"], self.k], n=[hd, c.kv_heads, hd, rows],
                      f=[c.eps])
                p.add(OP["ROPE_BATCH"], [self.k], n=[c.kv_heads, hd, hd, c.rope_dim, rows, kv_dim], u=[0],
                      f=[c.rope_base])
                p.add(OP["KV_WRITE_BATCH_PAGED"], [self.k, self.v, self.pool_k[i], self.pool_v[i], self.table],
                      n=[kv_dim, rows], u=[c.block_size, c.capacity, Mdl.F16])
                p.add(OP["RMSNORM_HEADS_BATCH"], [self.q, Ld["q_norm"], self.q], n=[hd, c.heads, 2 * hd, rows],
                      f=[c.eps])
                p.add(OP["ROPE_BATCH"], [self.q], n=[c.heads, 2 * hd, hd, c.rope_dim, rows, q_dim], u=[0],
                      f=[c.rope_base])
                p.add(OP["ATTENTION_PREFILL_PAGED"],
                      [self.q, self.pool_k[i], self.pool_v[i], self.attn, self.table],
                      n=[c.kv_heads, c.heads, hd, kv_dim, rows, 0], u=[c.block_size, c.capacity, Mdl.F16, 0],
                      f=[1.0 / math.sqrt(hd)])
                proj("o", self.tmp, H, n_in=c.heads * hd, x=self.attn)
                p.add(OP["ADD"], [self.x, self.tmp], n=[rows * H])
            # plan.go:915-987 addPrefillFFN
            self.rmsnorm_batch(p, self.x, Ld["post_norm"], self.norm, rows, H)
            gdt, udt = Lw["ffn_gate"]["dtype"], Lw["ffn_up"]["dtype"]
            gate_path = select_path(gdt, rows, H, c.ffn)
            if gdt == udt and gate_path == "wmma":
                p.add(OP["GEMM_SWIGLU"], [Ld["ffn_gate"], Ld["ffn_up"], self.norm, self.ffn_gate],
                      n=[H, c.ffn, rows], u=[gdt])
            else:
                proj("ffn_gate", self.ffn_gate, c.ffn)
                proj("ffn_up", self.ffn_up, c.ffn)
                p.add(OP["SILU_MUL"], [self.ffn_gate, self.ffn_up, self.ffn_gate], n=[rows * c.ffn])
            proj("ffn_down", self.tmp, H, n_in=c.ffn, x=self.ffn_gate)
            p.add(OP["ADD"], [self.x, self.tmp], n=[rows * H])
        p.mark_tail()
        self.rmsnorm_batch(p, self.x, W["output_norm"], self.norm, rows, H)
        out = self.w["output"]
        assert select_path(out["dtype"], rows, H, c.vocab) == "stream"
        p.add(OP["LM_HEAD"], [W["output"], self.norm, self.logits], n=[H, c.vocab, rows], u=[out["dtype"]])
        return p

    def prefill_logits(self, tokens):
        """engine/gpu/session.go:246-303."""
        t = np.ascontiguousarray(tokens, np.int32)
        rows = t.size
        assert 0 < rows <= MAX_LM_HEAD_ROWS
        if rows not in self.plans:
            self.plans[rows] = self.build(rows)
        self.tokens.write(t)
        self.plans[rows].execute(self.stream, 0, self.position, True)
        self.stream.sync()
        self.position += rows
        return self.logits.read(np.float32, rows * self.cfg.vocab).reshape(rows, self.cfg.vocab)

    def close(self):
        for p in self.plans.values():
            p.destroy()
        self.stream.destroy()


@pytest.mark.parametrize("shape", ["tiny", "config2"])
def test_go_shaped_v10_plan_matches_oracle(dev, shape):
    if shape == "tiny":
        cfg = Mdl.TINY
    else:
        cfg = replace(Mdl.QWEN35_4B_LIKE, n_layers=4, capacity=256)
    w = Mdl.make_weights(cfg, seed=13)
    s = GoSession(dev, cfg, w)
    orc = O.Q35(cfg, w)
    rng = np.random.default_rng(14)
    prompt = rng.integers(0, cfg.vocab, 37).astype(np.int32)
    # prompt in chunks of 16, 16, 5 rows (rows >= 8 take GEMM / GEMM_SWIGLU
    # for the narrow projections, rows < 8 GEMV_BATCH)
    for a in range(0, prompt.size, 16):
        got = s.prefill_logits(prompt[a:a + 16])
        want = orc.forward(prompt[a:a + 16], all_logits=True)
        _close(got, want, f"{shape} prompt chunk at {a}")
    # verify rows: 1 pending token + 4 drafts, then 16 rows
    for rows in (5, 16, 2):
        toks = rng.integers(0, cfg.vocab, rows).astype(np.int32)
        got = s.prefill_logits(toks)
        want = orc.forward(toks, all_logits=True)
        _close(got, want, f"{shape} verify {rows} rows")
    s.close()
    orc.close()


# ------------------------------------------------------------ decode plan

DOP = dict(GEMV=1, RMSNORM=2, L2NORM=3, GATED_RMSNORM=4, ROPE=5, CONV1D=7, GDN=8, SILU_MUL=9, ADD=10, SCALE=12,
           EMBEDDING=13, RMSNORM_HEADS=15, KV_WRITE_PAGED=26, ATTENTION_PAGED=27, QUANT_Q8_1=36, LM_HEAD=37,
           GEMV_Q8_1=38, RECURRENT_TOKEN=39, CONV_L2NORM=40, GEMV_RESIDUAL=41, GEMV_PAIR=42)
PAIR_WRITE_BOTH, PAIR_SWIGLU = 0, 1


def decode_path(n_in, n_out):
    """backend/hip/dispatch.go:199-207 SelectDecodeGemvPath without the int8
    option: the streaming LM_HEAD kernel from 1024 outputs (SelectLMHeadPath
    at one row, :96-123), else the per-row GEMV."""
    return "stream" if n_in % 256 == 0 and n_out >= LM_HEAD_MIN_OUTPUTS else "gemv"


class GoDecode:
    """engine/gpu/plan.go:238-307 buildDecodePlan (with addRecurrent,
    addFullAttention and addFFN, :309-527) over a GoSession's weights, KV pool
    and recurrent state, with the op layouts of backend/hip/hip.go. legacy
    selects the separate CONV1D / L2NORM / GDN / GATED_RMSNORM operators
    (Options.LegacyDeltaNet) instead of CONV_L2NORM + RECURRENT_TOKEN."""

    def __init__(self, s: GoSession, legacy: bool = False):
        self.s, self.legacy = s, legacy
        c, dev = s.cfg, s.dev
        f = lambda n: dev.alloc(max(4, n * 4))  # noqa: E731
        self.x, self.norm, self.tmp = f(c.hidden), f(c.hidden), f(c.hidden)
        self.q, self.k, self.v = f(c.heads * c.head_dim * 2), f(c.kv_heads * c.head_dim), f(c.kv_heads * c.head_dim)
        self.attn = f(c.heads * c.head_dim)
        self.scores = f(c.heads * c.capacity * 4)
        self.qkv, self.z, self.conv = f(s.conv_dim), f(c.inner), f(s.conv_dim)
        self.alpha, self.beta, self.gdn, self.gdn_norm = f(c.rank), f(c.rank), f(c.inner), f(c.inner)
        self.ffn_gate, self.ffn_up = f(c.ffn), f(c.ffn)
        self.logits = f(c.vocab)
        self.plan = self.build()

    def matmul(self, p, w, dt, x, out, n_in, n_out):  # plan.go:54-77
        code = DOP["LM_HEAD"] if decode_path(n_in, n_out) == "stream" else DOP["GEMV"]
        n = [n_in, n_out, 1] if code == DOP["LM_HEAD"] else [n_in, n_out]
        p.add(code, [w, x, out], n=n, u=[dt])

    def matmul_residual(self, p, w, dt, x, out, n_in, n_out):  # plan.go:84-94
        if decode_path(n_in, n_out) == "stream":
            p.add(DOP["GEMV_RESIDUAL"], [w, x, out, out], n=[n_in, n_out, 1], u=[dt])
            return
        self.matmul(p, w, dt, x, self.tmp, n_in, n_out)
        p.add(DOP["ADD"], [out, self.tmp], n=[n_out])

    def matmul_pair(self, p, wa, dta, wb, dtb, x, out_a, out_b, n_in, na, nb, epilogue):  # plan.go:103-141
        streaming = decode_path(n_in, na) == "stream" and decode_path(n_in, nb) == "stream"
        narrow = epilogue == PAIR_WRITE_BOTH and na == nb and n_in % 512 == 0 and dta == dtb
        if dta == dtb and (streaming or narrow) and (epilogue != PAIR_SWIGLU or na == nb):
            second = None if epilogue == PAIR_SWIGLU else out_b
            p.add(DOP["GEMV_PAIR"], [wa, wb, x, out_a, second], n=[n_in, na, nb], u=[dta, dtb, epilogue])
            return
        self.matmul(p, wa, dta, x, out_a, n_in, na)
        self.matmul(p, wb, dtb, x, out_b, n_in, nb)
        if epilogue == PAIR_SWIGLU:
            p.add(DOP["SILU_MUL"], [out_a, out_b, out_a], n=[na])

    def build(self):
        s, c = self.s, self.s.cfg
        W = s.wd
        p = hip.Plan(s.dev)
        H, hd = c.hidden, c.head_dim
        emb = s.w["embedding"]
        p.add(DOP["EMBEDDING"], [W["embedding"], self.x], n=[H, O.row_bytes(emb["dtype"], H)], u=[emb["dtype"]])
        for i in range(c.n_layers):
            Lw, Ld = s.w["layers"][i], W["layers"][i]
            dt = lambda name: Lw[name]["dtype"]  # noqa: E731
            p.add(DOP["RMSNORM"], [self.x, Ld["attn_norm"], self.norm], n=[H], f=[c.eps])
            if c.is_recurrent(i):  # plan.go:403-527
                key_dim, inner, rank = c.groups * c.state_size, c.inner, c.rank
                self.matmul(p, Ld["qkv"], dt("qkv"), self.norm, self.qkv, H, s.conv_dim)
                self.matmul(p, Ld["gate"], dt("gate"), self.norm, self.z, H, inner)
                self.matmul_pair(p, Ld["beta"], dt("beta"), Ld["alpha"], dt("alpha"), self.norm, self.beta,
                                 self.alpha, H, rank, rank, PAIR_WRITE_BOTH)
                q_scale = 1.0 / math.sqrt(c.state_size)
                qkv_offs = [0, key_dim * 4, 2 * key_dim * 4]
                fused = (c.state_size == 128 and s.conv_dim % 256 == 0 and (2 * key_dim) % 256 == 0
                         and key_dim % 128 == 0)
                if fused and not self.legacy:
                    p.add(DOP["CONV_L2NORM"], [s.conv_state[i], Ld["conv"], self.qkv, self.conv],
                          n=[s.conv_dim, c.conv_kernel, 2 * key_dim, key_dim, c.state_size], f=[c.eps, q_scale])
                    p.add(DOP["RECURRENT_TOKEN"],
                          [s.rec_state[i], self.conv, self.conv, self.conv, self.alpha, self.beta, Ld["dt"], Ld["a"],
                           self.gdn_norm, Ld["ssm_norm"], self.z],
                          offs=[0] + qkv_offs, n=[c.groups, rank, c.state_size], f=[c.eps])
                else:
                    p.add(DOP["CONV1D"], [s.conv_state[i], Ld["conv"], self.qkv, self.conv],
                          n=[s.conv_dim, c.conv_kernel])
                    p.add(DOP["L2NORM"], [self.conv, None, self.conv], n=[c.groups, c.state_size, c.state_size],
                          f=[c.eps, q_scale])
                    p.add(DOP["L2NORM"], [self.conv, None, self.conv], offs=[key_dim * 4, 0, key_dim * 4],
                          n=[c.groups, c.state_size, c.state_size], f=[c.eps, 1.0])
                    p.add(DOP["GDN"],
                          [s.rec_state[i], self.conv, self.conv, self.conv, self.alpha, self.beta, Ld["dt"], Ld["a"],
                           self.gdn],
                          offs=[0] + qkv_offs, n=[c.groups, rank, c.state_size])
                    p.add(DOP["GATED_RMSNORM"], [self.gdn, Ld["ssm_norm"], self.z, self.gdn_norm],
                          n=[c.state_size, rank, c.state_size], f=[c.eps])
                self.matmul_residual(p, Ld["out"], dt("out"), self.gdn_norm, self.x, inner, H)
            else:  # plan.go:309-390
                kv_dim, q_dim = c.kv_heads * hd, c.heads * hd * 2
                self.matmul(p, Ld["q"], dt("q"), self.norm, self.q, H, q_dim)
                self.matmul(p, Ld["k"], dt("k"), self.norm, self.k, H, kv_dim)
                self.matmul(p, Ld["v"], dt("v"), self.norm, self.v, H, kv_dim)
                p.add(DOP["RMSNORM_HEADS"], [self.q, Ld["q_norm"], self.q], n=[hd, c.heads, 2 * hd], f=[c.eps])
                p.add(DOP["RMSNORM_HEADS"], [self.k, Ld["k_norm"], self.k], n=[hd, c.kv_heads, hd], f=[c.eps])
                p.add(DOP["ROPE"], [self.q], n=[c.heads, 2 * hd, hd, c.rope_dim], f=[c.rope_base])
                p.add(DOP["ROPE"], [self.k], n=[c.kv_heads, hd, hd, c.rope_dim], f=[c.rope_base])
                p.add(DOP["KV_WRITE_PAGED"], [self.k, self.v, s.pool_k[i], s.pool_v[i], s.table], n=[kv_dim],
                      u=[c.block_size, c.capacity, Mdl.F16])
                p.add(DOP["ATTENTION_PAGED"],
                      [self.q, s.pool_k[i], s.pool_v[i], self.attn, self.scores, s.table],
                      n=[c.kv_heads, c.heads, hd, kv_dim, c.capacity], u=[c.block_size, c.capacity, Mdl.F16, 0],
                      f=[1.0 / math.sqrt(hd)])
                self.matmul_residual(p, Ld["o"], dt("o"), self.attn, self.x, c.heads * hd, H)
            # plan.go:529-561 addFFN
            p.add(DOP["RMSNORM"], [self.x, Ld["post_norm"], self.norm], n=[H], f=[c.eps])
            self.matmul_pair(p, Ld["ffn_gate"], dt("ffn_gate"), Ld["ffn_up"], dt("ffn_up"), self.norm,
                             self.ffn_gate, self.ffn_up, H, c.ffn, c.ffn, PAIR_SWIGLU)
            self.matmul_residual(p, Ld["ffn_down"], dt("ffn_down"), self.ffn_gate, self.x, c.ffn, H)
        p.mark_tail()
        p.add(DOP["RMSNORM"], [self.x, W["output_norm"], self.norm], n=[H], f=[c.eps])
        out = s.w["output"]
        self.matmul(p, W["output"], out["dtype"], self.norm, self.logits, H, c.vocab)
        return p

    def step(self, token, graph=None, dyn=None):
        """session.go Step: one token at the session position."""
        s = self.s
        if graph is None:
            self.plan.execute(s.stream, int(token), s.position, True)
        else:
            hip.check(hip.lib().yuuka_dynamic_set(s.stream.ptr, dyn.ptr, int(token), s.position), "dynamic_set")
            graph.replay(s.stream)
        s.stream.sync()
        s.position += 1
        return self.logits.read(np.float32, s.cfg.vocab)


@pytest.mark.parametrize("shape,legacy", [("tiny", False), ("tiny", True), ("config2", False)])
def test_go_shaped_decode_plan_matches_oracle(dev, shape, legacy):
    """NewSession's single-token plan (session.go:129) submitted unchanged:
    a prompt prefilled with the v10 prefill plan, then tokens decoded one at a
    time, directly and from a captured graph that reads {token, position}
    from the dynamic buffer, each against the CPU reference decoder."""
    cfg = Mdl.TINY if shape == "tiny" else replace(Mdl.QWEN35_4B_LIKE, n_layers=4, capacity=256)
    w = Mdl.make_weights(cfg, seed=17)
    s = GoSession(dev, cfg, w)
    d = GoDecode(s, legacy=legacy)
    orc = O.Q35(cfg, w)
    rng = np.random.default_rng(18)
    prompt = rng.integers(0, cfg.vocab, 21).astype(np.int32)
    for a in range(0, prompt.size, 16):
        s.prefill_logits(prompt[a:a + 16])
        orc.forward(prompt[a:a + 16])
    tok = int(rng.integers(0, cfg.vocab))
    for t in range(4):
        print(f"decode {shape} legacy={legacy} token {t} at {s.position}", flush=True)
        got = d.step(tok)
        want = orc.forward([tok])
        _close(got, want, f"{shape} decode step {t}")
        tok = int(np.argmax(want))
    dyn = dev.alloc(8)
    g = hip.Graph(d.plan, s.stream, dyn)
    for t in range(3):
        got = d.step(tok, g, dyn)
        want = orc.forward([tok])
        _close(got, want, f"{shape} graph decode step {t}")
        tok = int(np.argmax(want))
    g.destroy()
    d.plan.destroy()
    s.close()
    orc.close()


def test_q8_1_quantize_and_int8_decode_matvec(dev, stream):
    """QUANT_Q8_1 against the reference quantizer's contract
    (kernels/hip/gemm/mmq_gemm.hip:442-487: per 32 values d = amax / 127,
    q = clamp(rint(v / d)), {d, d * sum(q)}) bit for bit, SILU_MUL_QUANT_Q8_1
    on SiLU(gate) * up, and GEMV_Q8_1 (digits from QUANT_Q8_1, and the fused
    form on the FP32 row) against the oracle matmul of the dequantized row
    q * d."""
    rng = np.random.default_rng(19)
    K, N = 2560, 1536
    x = rng.normal(0, 1, K).astype(np.float32)
    x[:32] = 0.0  # an all-zero block: d = 0, digits 0
    w = Mdl.synth.quant_matrix(rng, Mdl.Q4_K, N, K, model_scale=True)
    xb, wb = dev.upload(x), dev.upload(w)
    qs, ds, out, out2 = dev.alloc(K), dev.alloc(K // 4), dev.alloc(N * 4), dev.alloc(N * 4)
    p = hip.Plan(dev)
    p.add(DOP["QUANT_Q8_1"], [xb, qs, ds], n=[K, 1])
    p.add(DOP["GEMV_Q8_1"], [wb, qs, ds, out], n=[K, N], u=[Mdl.Q4_K, 0])
    p.add(DOP["GEMV_Q8_1"], [wb, xb, None, out2], n=[K, N], u=[Mdl.Q4_K, 1])
    p.execute(stream)
    stream.sync()
    blk = x.reshape(-1, 32)
    amax = np.abs(blk).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    inv = np.where(amax > 0, np.float32(127) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    q = np.clip(np.rint(blk * inv[:, None]), -127, 127).astype(np.int8)
    got_q = qs.read(np.int8, K).reshape(-1, 32)
    got_d = ds.read(np.float32, K // 16).reshape(-1, 2)
    assert np.array_equal(got_q, q)
    assert np.array_equal(got_d[:, 0], d)
    assert np.array_equal(got_d[:, 1], (d * q.astype(np.int32).sum(axis=1).astype(np.float32)).astype(np.float32))
    xq = (q.astype(np.float32) * d[:, None]).reshape(1, K)
    want = O.matmul(Mdl.Q4_K, w, xq, N, K)[0]
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    for got in (out.read(np.float32, N), out2.read(np.float32, N)):
        assert np.max(np.abs(got - want)) <= 5e-4 * rms
    # SwiGLU form
    up = rng.normal(0, 1, K).astype(np.float32)
    ub = dev.upload(up)
    p2 = hip.Plan(dev)
    p2.add(43, [xb, ub, qs, ds], n=[K, 1])
    p2.execute(stream)
    stream.sync()
    h = O.silu_mul(x, up)
    hb = h.reshape(-1, 32)
    amax = np.abs(hb).max(axis=1)
    inv = np.where(amax > 0, np.float32(127) / np.where(amax > 0, amax, 1), 0).astype(np.float32)
    q = np.clip(np.rint(hb * inv[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(qs.read(np.int8, K).reshape(-1, 32), q)
    p.destroy()
    p2.destroy()
