"""ctypes wrapper of liboracle.so — the C restatement of the reference CPU
path (yuuka_oracle.c, qwen35_ref.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline. The
product library never loads it.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "liboracle.so"

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 8, 12, 13, 14
BLOCK = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(L):
    vp, u64, i64, u32, i32, dbl = C.c_void_p, C.c_uint64, C.c_int64, C.c_uint32, C.c_int32, C.c_double
    sig = {
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
        "orc_row_bytes": (u64, [u32, u64]),
        "orc_dequantize_row": (C.c_int, [vp, u64, u32, vp, u64]),
        "orc_matmul": (C.c_int, [vp, vp, C.c_int, vp, i64, i64, u32, C.c_int]),
        "orc_argmax": (i32, [vp, i64]),
        "orc_lookup_draft": (C.c_int, [vp, C.c_int, C.c_int, C.c_int, vp]),
        "orc_philox4x32_10": (None, [vp, vp, vp]),
        "orc_u01": (dbl, [u32, u32]),
        "orc_draw": (dbl, [u64, u64, u32, u32, u32]),
        "orc_target_weights": (i64, [vp, i64, C.c_float, C.c_int, C.c_float, vp, C.POINTER(dbl),
                                     C.POINTER(i32)]),
        "orc_accept_greedy": (None, [vp, i64, C.c_int, vp, C.POINTER(C.c_int), C.POINTER(i32), vp]),
        "orc_accept_stochastic": (None, [vp, i64, C.c_int, vp, C.c_float, C.c_int, C.c_float, u64,
                                         u64, u32, C.POINTER(C.c_int), C.POINTER(i32), vp, vp]),
        "orc_rmsnorm": (None, [vp, vp, vp, i32, C.c_float]),
        "orc_rmsnorm_inplace": (None, [vp, vp, i32, C.c_float]),
        "orc_l2norm_head": (None, [vp, i32, C.c_float, C.c_float]),
        "orc_rope": (None, [vp, i32, i32, i32, i32, i32, dbl]),
        "orc_sigmoid": (C.c_float, [C.c_float]),
        "orc_silu": (C.c_float, [C.c_float]),
        "orc_softplus": (C.c_float, [C.c_float]),
        "orc_gdn_scan": (None, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32]),
        "orc_gdn_norm_gate": (None, [vp, vp, vp, i32, i32, i32, C.c_float]),
        "orc_select_experts": (None, [vp, i32, i32, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def f16_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(h))


def f32_to_f16(f: float) -> int:
    return int(lib().orc_f32_to_f16(f))


def row_bytes(dtype: int, cols: int) -> int:
    return int(lib().orc_row_bytes(dtype, cols))


def dequantize(dtype: int, data: np.ndarray, rows: int, cols: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    rb = row_bytes(dtype, cols)
    out = np.empty((rows, cols), dtype=np.float32)
    for r in range(rows):
        row = data[r * rb:(r + 1) * rb]
        rc = lib().orc_dequantize_row(_ptr(out[r]), cols, dtype, _ptr(row), rb)
        if rc != 0:
            raise ValueError("dequantize failed")
    return out


def matmul(dtype: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int, workers: int = 0) -> np.ndarray:
    """dst[b, r] = sum_i x[b, i] * W[r, i] (tensor/quant.go:341-466)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty((x.shape[0], rows), dtype=np.float32)
    rc = lib().orc_matmul(_ptr(out), _ptr(x), x.shape[0], _ptr(w), rows, cols, dtype, workers)
    if rc != 0:
        raise ValueError("matmul failed")
    return out


def rmsnorm_rows(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """forward.go:460-470 rmsNorm applied to every row of x."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        lib().orc_rmsnorm(_ptr(out[r]), _ptr(x[r]), _ptr(w), x.shape[1], eps)
    return out


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """forward.go SwiGLU: silu(g) * u per element (float32)."""
    f = lib().orc_silu
    return np.array([f(float(a)) for a in g.ravel()], np.float32).reshape(g.shape) * u.astype(np.float32)


def select_experts(logits: np.ndarray, used: int):
    """forward.go:393-439 selectExperts: (ids, float32 weights)."""
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.zeros(used, np.int32)
    w = np.zeros(used, np.float32)
    lib().orc_select_experts(_ptr(logits), logits.size, used, _ptr(ids), _ptr(w))
    return ids, w


def argmax(logits: np.ndarray) -> int:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().orc_argmax(_ptr(logits), logits.size))


def lookup_draft(history, max_draft: int, min_match: int) -> list[int]:
    h = np.ascontiguousarray(history, dtype=np.int32)
    out = np.zeros(max(max_draft, 1), dtype=np.int32)
    n = lib().orc_lookup_draft(_ptr(h), h.size, max_draft, min_match, _ptr(out))
    return out[:n].tolist()


def philox(ctr, key) -> list[int]:
    c = np.array(ctr, dtype=np.uint32)
    k = np.array(key, dtype=np.uint32)
    o = np.zeros(4, dtype=np.uint32)
    lib().orc_philox4x32_10(_ptr(c), _ptr(k), _ptr(o))
    return o.tolist()


def draw(seed: int, step: int, row: int, request: int, purpose: int) -> float:
    return float(lib().orc_draw(seed, step, row, request, purpose))


def target_weights(logits: np.ndarray, temperature: float, top_k: int = 0, top_p: float = 1.0):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    w = np.zeros(logits.size, dtype=np.float64)
    total = C.c_double()
    best = C.c_int32()
    kept = lib().orc_target_weights(_ptr(logits), logits.size, temperature, top_k, top_p, _ptr(w),
                                    C.byref(total), C.byref(best))
    return int(kept), w, float(total.value), int(best.value)


def accept_greedy(logits: np.ndarray, drafts) -> tuple[int, int, list[int]]:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    k = len(drafts)
    V = logits.shape[-1]
    d = np.ascontiguousarray(drafts, dtype=np.int32) if k else np.zeros(1, np.int32)
    rows = np.zeros(k + 1, dtype=np.int32)
    a = C.c_int()
    nxt = C.c_int32()
    lib().orc_accept_greedy(_ptr(logits), V, k, _ptr(d), C.byref(a), C.byref(nxt), _ptr(rows))
    return a.value, nxt.value, rows.tolist()


def accept_stochastic(logits: np.ndarray, drafts, temperature: float, seed: int, step: int,
                      request: int, top_k: int = 0, top_p: float = 1.0):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    k = len(drafts)
    V = logits.shape[-1]
    d = np.ascontiguousarray(drafts, dtype=np.int32) if k else np.zeros(1, np.int32)
    pd = np.zeros(max(k, 1), dtype=np.float64)
    ua = np.zeros(max(k, 1), dtype=np.float64)
    a = C.c_int()
    nxt = C.c_int32()
    lib().orc_accept_stochastic(_ptr(logits), V, k, _ptr(d), temperature, top_k, top_p, seed, step,
                                request, C.byref(a), C.byref(nxt), _ptr(pd), _ptr(ua))
    return a.value, nxt.value, pd[:k].tolist(), ua[:k].tolist()


# ------------------------------------------------------------ qwen35 model

class orc_q35_config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "hidden", "ffn", "heads", "kv_heads", "head_dim", "rope_dim", "vocab", "conv_kernel",
        "state_size", "groups", "rank", "inner", "full_interval", "n_experts", "n_experts_used", "expert_ffn",
        "shared_ffn")] + [("rope_base", C.c_double), ("eps", C.c_float), ("matmul_workers", C.c_int32)]


class orc_q35_matrix(C.Structure):
    _fields_ = [("data", C.c_void_p), ("rows", C.c_int64), ("cols", C.c_int64), ("dtype", C.c_uint32),
                ("pad", C.c_uint32)]


_FP = C.POINTER(C.c_float)


class orc_q35_layer(C.Structure):
    _fields_ = [("attn_norm", _FP), ("post_norm", _FP)] + \
        [(n, orc_q35_matrix) for n in ("qkv", "gate", "out", "beta", "alpha")] + \
        [(n, _FP) for n in ("conv", "dt", "a", "ssm_norm")] + \
        [(n, orc_q35_matrix) for n in ("q", "k", "v", "o")] + \
        [("q_norm", _FP), ("k_norm", _FP)] + \
        [(n, orc_q35_matrix) for n in ("ffn_gate", "ffn_up", "ffn_down", "router")] + \
        [("shared_gate_vec", _FP)] + \
        [(n, orc_q35_matrix) for n in ("shared_gate", "shared_up", "shared_down", "gate_exps", "up_exps",
                                       "down_exps")]


class orc_q35_model(C.Structure):
    _fields_ = [("cfg", orc_q35_config), ("embedding", orc_q35_matrix), ("output", orc_q35_matrix),
                ("output_norm", _FP), ("layers", C.POINTER(orc_q35_layer))]


def _declare_q35(L):
    vp, i32 = C.c_void_p, C.c_int32
    sig = {
        "orc_q35_pool_new": (vp, [C.POINTER(orc_q35_config), i32, i32, i32]),
        "orc_q35_pool_free": (None, [vp]),
        "orc_q35_pool_data": (vp, [vp, i32, i32, C.POINTER(C.c_uint64)]),
        "orc_q35_state_new": (vp, [C.POINTER(orc_q35_config), vp, vp, i32, i32]),
        "orc_q35_state_free": (None, [vp]),
        "orc_q35_state_reset": (None, [vp]),
        "orc_q35_state_pos": (i32, [vp]),
        "orc_q35_state_set_pos": (C.c_int, [vp, i32]),
        "orc_q35_state_conv": (vp, [vp, i32]),
        "orc_q35_state_matrix": (vp, [vp, i32]),
        "orc_q35_snapshot_bytes": (C.c_uint64, [vp]),
        "orc_q35_snapshot": (None, [vp, vp]),
        "orc_q35_restore": (C.c_int, [vp, vp, C.c_uint64]),
        "orc_q35_forward": (C.c_int, [C.POINTER(orc_q35_model), vp, vp, i32, i32, vp, vp]),
        "orc_q35_forward_residual": (C.c_int, [C.POINTER(orc_q35_model), vp, vp, i32, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args


def _mat(t):
    if t is None:
        return orc_q35_matrix()
    return orc_q35_matrix(t["data"].ctypes.data_as(C.c_void_p), t["rows"], t["cols"], t["dtype"], 0)


class Q35:
    """The CPU reference decoder (model/qwen35 restatement) over host weights
    from yuuka_amd.model.make_weights. format: 0 F32, 1 F16 KV rows."""

    def __init__(self, cfg, weights, kv_format: int = 1, workers: int = 0):
        L = lib()
        if not hasattr(L, "_q35_declared"):
            _declare_q35(L)
            L._q35_declared = True
        self.cfg = cfg
        c = orc_q35_config()
        for n in ("n_layers", "hidden", "ffn", "heads", "kv_heads", "head_dim", "rope_dim", "vocab",
                  "conv_kernel", "state_size", "groups", "rank", "full_interval"):
            setattr(c, n, getattr(cfg, n))
        for n in ("n_experts", "n_experts_used", "expert_ffn", "shared_ffn"):
            setattr(c, n, getattr(cfg, n, 0))
        c.inner = cfg.inner
        c.rope_base = cfg.rope_base
        c.eps = cfg.eps
        c.matmul_workers = workers
        self.layers = (orc_q35_layer * cfg.n_layers)()
        for i, Lw in enumerate(weights["layers"]):
            s = self.layers[i]
            s.attn_norm = Lw["attn_norm"].ctypes.data_as(_FP)
            s.post_norm = Lw["post_norm"].ctypes.data_as(_FP)
            for n in ("qkv", "gate", "out", "beta", "alpha", "q", "k", "v", "o", "ffn_gate", "ffn_up", "ffn_down",
                      "router", "shared_gate", "shared_up", "shared_down", "gate_exps", "up_exps", "down_exps"):
                setattr(s, n, _mat(Lw.get(n)))
            for n in ("conv", "dt", "a", "ssm_norm", "q_norm", "k_norm", "shared_gate_vec"):
                if n in Lw:
                    setattr(s, n, Lw[n].ctypes.data_as(_FP))
        self.model = orc_q35_model(c, _mat(weights["embedding"]), _mat(weights["output"]),
                                   weights["output_norm"].ctypes.data_as(_FP), self.layers)
        self.weights = weights
        blocks = (cfg.capacity + cfg.block_size - 1) // cfg.block_size
        self.pool = L.orc_q35_pool_new(C.byref(self.model.cfg), blocks, cfg.block_size, kv_format)
        self.table = np.arange(blocks, dtype=np.int32)
        self.state = L.orc_q35_state_new(C.byref(self.model.cfg), self.pool, _ptr(self.table), blocks,
                                         cfg.capacity)

    def reset(self):
        lib().orc_q35_state_reset(self.state)

    @property
    def position(self) -> int:
        return int(lib().orc_q35_state_pos(self.state))

    def forward(self, tokens, all_logits: bool = False) -> np.ndarray:
        """Forward (last-token logits) or PrefillLogits (every row)."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros((t.size if all_logits else 1, self.cfg.vocab), np.float32)
        rc = lib().orc_q35_forward(C.byref(self.model), self.state, _ptr(t), t.size, int(all_logits), _ptr(out),
                                   None)
        if rc != 0:
            raise RuntimeError(f"orc_q35_forward failed ({rc})")
        return out if all_logits else out[0]

    def forward_residual(self, tokens) -> np.ndarray:
        """The residual stream after the last layer, one row per token."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros((t.size, self.cfg.hidden), np.float32)
        rc = lib().orc_q35_forward_residual(C.byref(self.model), self.state, _ptr(t), t.size, _ptr(out))
        if rc != 0:
            raise RuntimeError(f"orc_q35_forward_residual failed ({rc})")
        return out

    def forward_hidden(self, tokens) -> tuple[np.ndarray, np.ndarray]:
        """PrefillLogits plus the normalized hidden rows: (logits, hidden)."""
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros((t.size, self.cfg.vocab), np.float32)
        hid = np.zeros((t.size, self.cfg.hidden), np.float32)
        rc = lib().orc_q35_forward(C.byref(self.model), self.state, _ptr(t), t.size, 1, _ptr(out), _ptr(hid))
        if rc != 0:
            raise RuntimeError(f"orc_q35_forward failed ({rc})")
        return out, hid

    def snapshot(self):
        n = lib().orc_q35_snapshot_bytes(self.state)
        buf = np.zeros(n, np.uint8)
        lib().orc_q35_snapshot(self.state, _ptr(buf))
        return buf, self.position

    def restore(self, data, position):
        if lib().orc_q35_restore(self.state, _ptr(data), data.nbytes) != 0:
            raise ValueError("snapshot length mismatch")
        lib().orc_q35_state_set_pos(self.state, position)

    def close(self):
        if self.state:
            lib().orc_q35_state_free(self.state)
            lib().orc_q35_pool_free(self.pool)
            self.state = self.pool = None


def generate_greedy_speculative(oracle: Q35, prompt, max_tokens: int, max_draft: int = 4, min_match: int = 2):
    """engine/speculative.go:68-261 over the CPU decoder (greedy, no stop
    tokens): prompt-lookup drafts, PrefillLogits verify, snapshot/restore and
    replay on partial acceptance. Returns (tokens, draft_tokens, accepted)."""
    oracle.reset()
    logits = oracle.forward(prompt)
    history = list(prompt)
    out, drafts_n, acc_n = [], 0, 0
    while len(out) < max_tokens:
        limit = min(max_draft, max_tokens - len(out), oracle.cfg.capacity - len(history))
        if limit <= 0:
            break
        draft = lookup_draft(history, limit, min_match)
        if not draft:
            tok = argmax(logits)
            out.append(tok)
            history.append(tok)
            if len(out) >= max_tokens:
                break
            logits = oracle.forward([tok])
            continue
        snap, pos = oracle.snapshot()
        cand = oracle.forward(draft, all_logits=True)
        drafts_n += len(draft)
        accepted, before, correction = 0, logits, -1
        for i, d in enumerate(draft):
            want = argmax(before)
            if want == d:
                accepted += 1
                before = cand[i]
                continue
            correction = want
            break
        acc_n += accepted
        if accepted == len(draft):
            emitted, nxt = list(draft), cand[-1]
        else:
            oracle.restore(snap, pos)
            replay = list(draft[:accepted]) + [correction]
            nxt = oracle.forward(replay)
            emitted = replay
        for t in emitted:
            out.append(t)
            history.append(t)
            if len(out) >= max_tokens:
                break
        if len(out) >= max_tokens:
            break
        logits = nxt
    return out, drafts_n, acc_n
