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
