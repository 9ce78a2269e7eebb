"""qwen35 model description, seeded synthetic weights, and the ctypes view of
the GPU engine (yuuka_q35_* in include/yuuka_hip.h).

The same host weight arrays are handed to the GPU engine and (in tests and
the CPU baseline) to the oracle, so both run the identical model.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, fields, replace  # noqa: F401 (replace re-exported)

import numpy as np

from . import hip, synth

F32, F16, Q4_K, Q6_K = 0, 1, 12, 14


@dataclass(frozen=True)
class Q35Config:
    """model/qwen35/config.go:18-45 (dense model fields) plus session geometry."""
    n_layers: int
    hidden: int
    ffn: int
    heads: int
    kv_heads: int
    head_dim: int
    rope_dim: int
    vocab: int
    conv_kernel: int = 4
    state_size: int = 128
    groups: int = 16
    rank: int = 16
    full_interval: int = 4
    rope_base: float = 10000000.0
    eps: float = 1e-6
    capacity: int = 1024
    block_size: int = 16
    kv_dtype: int = F16
    max_rows: int = 16
    batch: int = 1
    kv_blocks: int = 0
    n_experts: int = 0
    n_experts_used: int = 0
    expert_ffn: int = 0
    shared_ffn: int = 0
    router_normal_seed: int = 0  # nonzero: MoE router logits replaced by N(0,1) draws

    @property
    def inner(self) -> int:
        return self.rank * self.state_size

    @property
    def conv_dim(self) -> int:
        return 2 * self.groups * self.state_size + self.inner

    def is_recurrent(self, layer: int) -> bool:
        return (layer + 1) % self.full_interval != 0  # config.go:280-282


# Qwen3.5-4B-like hybrid decoder (16-head GDN
# geometry: groups = rank = 16, inner 2048, conv_dim 6144).
QWEN35_4B_LIKE = Q35Config(n_layers=32, hidden=2560, ffn=9216, heads=16, kv_heads=4, head_dim=256,
                           rope_dim=64, vocab=151936, groups=16, rank=16, capacity=1024)

# Qwen3.5-9B-like hybrid decoder (hidden 4096, FFN
# 12288, 16 Q / 4 KV heads of 256; GDN with 16 heads of 128).
QWEN35_9B_LIKE = Q35Config(n_layers=32, hidden=4096, ffn=12288, heads=16, kv_heads=4, head_dim=256,
                           rope_dim=64, vocab=151936, groups=16, rank=16, capacity=16384 + 64)

# Qwen3.5-MoE-like decoder (hidden 2048, 40 layers,
# 256 experts, top-8, expert FFN 512, one shared expert of 512).
QWEN35_MOE_LIKE = Q35Config(n_layers=40, hidden=2048, ffn=0, heads=16, kv_heads=4, head_dim=256, rope_dim=64,
                            vocab=151936, groups=16, rank=16, capacity=2048 + 64, n_experts=256,
                            n_experts_used=8, expert_ffn=512, shared_ffn=512)

# Small geometry for parity tests (every matrix width a multiple of 256).
TINY = Q35Config(n_layers=4, hidden=256, ffn=512, heads=2, kv_heads=1, head_dim=256, rope_dim=64,
                 vocab=1024, groups=1, rank=2, capacity=256)
TINY_MOE = replace(TINY, ffn=0, n_experts=16, n_experts_used=4, expert_ffn=256, shared_ffn=256)


def make_weights(cfg: Q35Config, seed: int = 0, q6_output: bool = True, q6_v: bool = True,
                 share_experts: bool = False) -> dict:
    """Seeded random-init weights: every 2-D matrix packed as Q4_K (Q6_K for
    the output head and attn_v, the Q4_K_M mix), dequantized std ~0.02;
    norm vectors near 1, conv weights and GDN dt/a chosen so the decay
    exp(softplus(alpha + dt) * a) stays inside (0, 1). MoE layers: FP32
    router scaled so router logits are ~N(0, 1), Q4_K experts and shared
    expert. share_experts: every layer holds the same expert bytes (one host
    copy; the engine still uploads one device copy per layer)."""
    rng = np.random.default_rng(seed)
    H, cd = cfg.hidden, cfg.conv_dim
    shared = {}

    def mat(rows, cols, dtype=Q4_K):
        return dict(data=synth.quant_matrix(rng, dtype, rows, cols, model_scale=True), rows=rows, cols=cols,
                    dtype=dtype)

    def norm(n):
        return (1.0 + rng.normal(0, 0.05, n)).astype(np.float32)

    w = dict(embedding=mat(cfg.vocab, H), output=mat(cfg.vocab, H, Q6_K if q6_output else Q4_K),
             output_norm=norm(H), layers=[])
    for i in range(cfg.n_layers):
        L = dict(attn_norm=norm(H), post_norm=norm(H))
        if cfg.is_recurrent(i):
            L.update(qkv=mat(cd, H), gate=mat(cfg.inner, H), out=mat(H, cfg.inner), beta=mat(cfg.rank, H),
                     alpha=mat(cfg.rank, H),
                     conv=rng.normal(0, 0.3, cd * cfg.conv_kernel).astype(np.float32),
                     dt=rng.normal(0, 0.5, cfg.rank).astype(np.float32),
                     a=(-rng.uniform(0.2, 2.0, cfg.rank)).astype(np.float32),
                     ssm_norm=norm(cfg.state_size))
        else:
            hd = cfg.head_dim
            L.update(q=mat(cfg.heads * hd * 2, H), k=mat(cfg.kv_heads * hd, H),
                     v=mat(cfg.kv_heads * hd, H, Q6_K if q6_v else Q4_K), o=mat(H, cfg.heads * hd),
                     q_norm=norm(hd), k_norm=norm(hd))
        if cfg.n_experts:
            E, ef, sf = cfg.n_experts, cfg.expert_ffn, cfg.shared_ffn
            if share_experts and shared:
                L.update(shared)
            else:
                ex = dict(gate_exps=mat(E * ef, H), up_exps=mat(E * ef, H), down_exps=mat(E * H, ef))
                if share_experts:
                    shared.update(ex)
                L.update(ex)
            L.update(router=dict(data=rng.normal(0, 1 / np.sqrt(H), (E, H)).astype(np.float32).view(np.uint8).ravel(),
                                 rows=E, cols=H, dtype=F32),
                     shared_gate_vec=rng.normal(0, 1 / np.sqrt(H), H).astype(np.float32),
                     shared_gate=mat(sf, H), shared_up=mat(sf, H), shared_down=mat(H, sf))
        else:
            L.update(ffn_gate=mat(cfg.ffn, H), ffn_up=mat(cfg.ffn, H), ffn_down=mat(H, cfg.ffn))
        w["layers"].append(L)
    return w


def weight_bytes(w: dict) -> int:
    """Bytes one verify step streams from the weights: every layer tensor,
    the output norm and the LM head (the embedding table is only gathered)."""
    n = w["output"]["data"].nbytes + w["output_norm"].nbytes
    for L in w["layers"]:
        for v in L.values():
            n += v["data"].nbytes if isinstance(v, dict) else v.nbytes
    return n


# ----------------------------------------------------------- ctypes structs

class yuuka_q35_config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_layers", "hidden", "ffn", "heads", "kv_heads", "head_dim",
                                         "rope_dim", "vocab", "conv_kernel", "state_size", "groups", "rank",
                                         "inner", "full_interval")] + [
        ("rope_base", C.c_double), ("eps", C.c_float), ("capacity", C.c_int32), ("block_size", C.c_int32),
        ("kv_dtype", C.c_uint32), ("max_rows", C.c_int32)] + [
        (n, C.c_int32) for n in ("batch", "kv_blocks", "n_experts", "n_experts_used", "expert_ffn", "shared_ffn")] + [
        ("router_normal_seed", C.c_uint32)]


class yuuka_q35_tensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("rows", C.c_uint64), ("cols", C.c_uint64), ("dtype", C.c_uint32),
                ("pad", C.c_uint32)]


_FP = C.POINTER(C.c_float)


class yuuka_q35_layer_weights(C.Structure):
    _fields_ = [("attn_norm", _FP), ("post_norm", _FP)] + \
        [(n, yuuka_q35_tensor) for n in ("qkv", "gate", "out", "beta", "alpha")] + \
        [(n, _FP) for n in ("conv", "dt", "a", "ssm_norm")] + \
        [(n, yuuka_q35_tensor) for n in ("q", "k", "v", "o")] + \
        [("q_norm", _FP), ("k_norm", _FP)] + \
        [(n, yuuka_q35_tensor) for n in ("ffn_gate", "ffn_up", "ffn_down", "router")] + \
        [("shared_gate_vec", _FP)] + \
        [(n, yuuka_q35_tensor) for n in ("shared_gate", "shared_up", "shared_down", "gate_exps", "up_exps",
                                         "down_exps")]


class yuuka_q35_weights(C.Structure):
    _fields_ = [("embedding", yuuka_q35_tensor), ("output", yuuka_q35_tensor), ("output_norm", _FP),
                ("layers", C.POINTER(yuuka_q35_layer_weights))]


class yuuka_q35_accept(C.Structure):
    _fields_ = [("mode", C.c_uint32), ("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float),
                ("seed", C.c_uint64)]


class yuuka_q35_generate_opts(C.Structure):
    _fields_ = [("max_tokens", C.c_int32), ("max_draft", C.c_int32), ("min_match", C.c_int32),
                ("stop_token", C.c_int32), ("accept", yuuka_q35_accept)]


class yuuka_q35_generate_stats(C.Structure):
    _fields_ = [("output_tokens", C.c_int32), ("steps", C.c_int32), ("draft_tokens", C.c_int32),
                ("accepted_draft", C.c_int32), ("prefill_ms", C.c_double), ("decode_ms", C.c_double)]


def config_struct(cfg: Q35Config) -> yuuka_q35_config:
    s = yuuka_q35_config()
    for f in fields(cfg):
        if hasattr(s, f.name):
            setattr(s, f.name, getattr(cfg, f.name))
    s.inner = cfg.inner
    return s


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_FP)


def _tensor(t: dict | None) -> yuuka_q35_tensor:
    if t is None:
        return yuuka_q35_tensor()
    return yuuka_q35_tensor(t["data"].ctypes.data_as(C.c_void_p), t["rows"], t["cols"], t["dtype"], 0)


def weights_struct(cfg: Q35Config, w: dict):
    layers = (yuuka_q35_layer_weights * cfg.n_layers)()
    for i, L in enumerate(w["layers"]):
        s = layers[i]
        s.attn_norm, s.post_norm = _ptr(L["attn_norm"]), _ptr(L["post_norm"])
        for n in ("qkv", "gate", "out", "beta", "alpha", "q", "k", "v", "o", "ffn_gate", "ffn_up", "ffn_down",
                  "router", "shared_gate", "shared_up", "shared_down", "gate_exps", "up_exps", "down_exps"):
            setattr(s, n, _tensor(L.get(n)))
        for n in ("conv", "dt", "a", "ssm_norm", "q_norm", "k_norm", "shared_gate_vec"):
            if n in L:
                setattr(s, n, _ptr(L[n]))
    ws = yuuka_q35_weights(_tensor(w["embedding"]), _tensor(w["output"]), _ptr(w["output_norm"]), layers)
    return ws, layers


def _declare(L):
    vp = C.c_void_p
    sig = {
        "yuuka_q35_create": (C.c_int, [vp, C.POINTER(yuuka_q35_config), C.POINTER(yuuka_q35_weights),
                                       C.POINTER(vp)]),
        "yuuka_q35_destroy": (None, [vp]),
        "yuuka_q35_reset": (C.c_int, [vp]),
        "yuuka_q35_position": (C.c_int32, [vp]),
        "yuuka_q35_last_step_ms": (C.c_float, [vp]),
        "yuuka_q35_prefill": (C.c_int, [vp, vp, C.c_int32, vp]),
        "yuuka_q35_verify": (C.c_int, [vp, vp, C.c_int32, C.POINTER(yuuka_q35_accept), vp]),
        "yuuka_q35_logits": (C.c_int, [vp, vp, C.c_int32]),
        "yuuka_q35_moe_counts": (C.c_int, [vp, C.c_int32, vp, C.c_int32]),
        "yuuka_q35_snapshot_bytes": (C.c_uint64, [vp]),
        "yuuka_q35_snapshot": (C.c_int, [vp, vp, C.POINTER(C.c_int32)]),
        "yuuka_q35_restore": (C.c_int, [vp, vp, C.c_uint64, C.c_int32]),
        "yuuka_q35_generate": (C.c_int, [vp, vp, C.c_int32, C.POINTER(yuuka_q35_generate_opts), vp,
                                         C.POINTER(yuuka_q35_generate_stats)]),
        "yuuka_q35_request_position": (C.c_int32, [vp, C.c_int32]),
        "yuuka_q35_reset_request": (C.c_int, [vp, C.c_int32]),
        "yuuka_q35_prefill_request": (C.c_int, [vp, C.c_int32, vp, C.c_int32, vp]),
        "yuuka_q35_fork": (C.c_int, [vp, C.c_int32, C.c_int32]),
        "yuuka_q35_step_batch": (C.c_int, [vp, C.c_int32, vp, C.c_int32, C.c_int32, C.POINTER(yuuka_q35_accept),
                                           vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args


def accept_struct(mode: int = 0, temperature: float = 0.0, seed: int = 0, top_k: int = 0,
                  top_p: float = 1.0) -> yuuka_q35_accept:
    return yuuka_q35_accept(mode, temperature, top_k, top_p, seed)


class Engine:
    """GPU verify engine (yuuka_q35_*): the Python mirror of the reference's
    gpu.Runtime / Session surface used by the speculative loop."""

    def __init__(self, dev: hip.Device, cfg: Q35Config, weights: dict):
        L = hip.lib()
        if not hasattr(L, "_q35_declared"):
            _declare(L)
            L._q35_declared = True
        self.cfg = cfg
        self._cs = config_struct(cfg)
        self._ws, self._layers = weights_struct(cfg, weights)
        p = C.c_void_p()
        hip.check(L.yuuka_q35_create(dev.ptr, C.byref(self._cs), C.byref(self._ws), C.byref(p)), "q35_create")
        self.ptr = p

    def reset(self):
        hip.check(hip.lib().yuuka_q35_reset(self.ptr), "q35_reset")

    @property
    def position(self) -> int:
        return int(hip.lib().yuuka_q35_position(self.ptr))

    def moe_counts(self, layer: int) -> np.ndarray:
        """Rows of the last step per expert of MoE layer `layer`."""
        out = np.zeros(self.cfg.n_experts, np.int32)
        hip.check(hip.lib().yuuka_q35_moe_counts(self.ptr, layer, out.ctypes.data_as(C.c_void_p), len(out)),
                  "q35_moe_counts")
        return out

    @property
    def last_step_ms(self) -> float:
        return float(hip.lib().yuuka_q35_last_step_ms(self.ptr))

    def prefill(self, tokens, want_logits=True):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros(self.cfg.vocab, np.float32) if want_logits else None
        hip.check(hip.lib().yuuka_q35_prefill(self.ptr, t.ctypes.data_as(C.c_void_p), t.size,
                                              None if out is None else out.ctypes.data_as(C.c_void_p)),
                  "q35_prefill")
        return out

    def verify(self, tokens, accept=None):
        t = np.ascontiguousarray(tokens, np.int32)
        res = np.zeros(4, np.int32)
        acc = accept or accept_struct()
        hip.check(hip.lib().yuuka_q35_verify(self.ptr, t.ctypes.data_as(C.c_void_p), t.size, C.byref(acc),
                                             res.ctypes.data_as(C.c_void_p)), "q35_verify")
        return res

    def request_position(self, r: int) -> int:
        return int(hip.lib().yuuka_q35_request_position(self.ptr, r))

    def reset_request(self, r: int):
        hip.check(hip.lib().yuuka_q35_reset_request(self.ptr, r), "q35_reset_request")

    def prefill_request(self, r: int, tokens, want_logits=False):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros(self.cfg.vocab, np.float32) if want_logits else None
        hip.check(hip.lib().yuuka_q35_prefill_request(self.ptr, r, t.ctypes.data_as(C.c_void_p), t.size,
                                                      None if out is None else out.ctypes.data_as(C.c_void_p)),
                  "q35_prefill_request")
        return out

    def fork(self, src: int, dst: int):
        hip.check(hip.lib().yuuka_q35_fork(self.ptr, src, dst), "q35_fork")

    def step_batch(self, tokens, mode: int = 0, accept=None, forced=None):
        """tokens [n_req][rows]; returns result [n_req][4] (mode 0)."""
        t = np.ascontiguousarray(tokens, np.int32)
        n_req, rows = t.shape
        res = np.zeros((n_req, 4), np.int32)
        acc = accept or accept_struct()
        f = None if forced is None else np.ascontiguousarray(forced, np.int32)
        hip.check(hip.lib().yuuka_q35_step_batch(self.ptr, n_req, t.ctypes.data_as(C.c_void_p), rows, mode,
                                                 C.byref(acc), None if f is None else f.ctypes.data_as(C.c_void_p),
                                                 res.ctypes.data_as(C.c_void_p)), "q35_step_batch")
        return res

    def logits(self, rows):
        out = np.zeros((rows, self.cfg.vocab), np.float32)
        hip.check(hip.lib().yuuka_q35_logits(self.ptr, out.ctypes.data_as(C.c_void_p), rows), "q35_logits")
        return out

    def snapshot(self):
        n = hip.lib().yuuka_q35_snapshot_bytes(self.ptr)
        buf = np.zeros(n, np.uint8)
        pos = C.c_int32()
        hip.check(hip.lib().yuuka_q35_snapshot(self.ptr, buf.ctypes.data_as(C.c_void_p), C.byref(pos)),
                  "q35_snapshot")
        return buf, pos.value

    def restore(self, data, position):
        hip.check(hip.lib().yuuka_q35_restore(self.ptr, data.ctypes.data_as(C.c_void_p), data.nbytes, position),
                  "q35_restore")

    def generate(self, prompt, max_tokens, max_draft=4, min_match=2, stop_token=-1, accept=None):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(max_tokens, np.int32)
        opts = yuuka_q35_generate_opts(max_tokens, max_draft, min_match, stop_token, accept or accept_struct())
        st = yuuka_q35_generate_stats()
        hip.check(hip.lib().yuuka_q35_generate(self.ptr, p.ctypes.data_as(C.c_void_p), p.size, C.byref(opts),
                                               out.ctypes.data_as(C.c_void_p), C.byref(st)), "q35_generate")
        return out[:st.output_tokens].tolist(), st

    def close(self):
        if self.ptr:
            hip.lib().yuuka_q35_destroy(self.ptr)
            self.ptr = None
