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
