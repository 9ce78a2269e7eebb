"""ctypes binding of libyuuka_hip.so — the Python counterpart of the
reference Go binding backend/hip/hip.go (Device, Buffer, Stream, Event, Plan).

The library is loaded from yuuka_amd/lib (built in-tree by yuuka_amd/build.py).
There is no fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libyuuka_hip.so"
HEADER = Path(__file__).resolve().parent.parent / "include" / "yuuka_hip.h"

OK, INVALID_ARGUMENT, UNSUPPORTED, DEVICE, ALLOCATION, INTERNAL = range(6)

# yuuka_dtype (include/yuuka_hip.h)
F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 6, 8, 12, 13, 14

# op codes used by the verify plan
OP = dict(
    SILU_MUL=9, ADD=10, COPY=11, GEMV_BATCH=17, RMSNORM_BATCH=18, RMSNORM_HEADS_BATCH=19,
    ROPE_BATCH=20, RECURRENT_CHUNK=23, EMBEDDING_BATCH=24, KV_WRITE_BATCH_PAGED=28,
    ATTENTION_PREFILL_PAGED=29, MOE_ROUTE=30, MOE_GATE_UP=31, MOE_DOWN=32, MOE_REDUCE_ADD=33, LM_HEAD=37,
    ACCEPT=66, GDN_COMMIT=67, ADVANCE=68, GEMM_FUSED=69, ROPE_TABLE=70, ATTN_VERIFY=71, MOE_ROUTER=72,
    MOE_COMBINE=73, ROUTER_NORMAL=74,
)
FLAG_MOE_SWIGLU = 0x800
FLAG_MOE_PACKED = 0x2000
EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU = 0, 1, 2
FLAG_TAIL = 0x1

ACCEPT_GREEDY, ACCEPT_STOCHASTIC = 0, 1


class HipError(RuntimeError):
    def __init__(self, status: int, what: str, message: str):
        super().__init__(f"{what}: status {status}: {message}")
        self.status = status


class Unsupported(HipError):
    pass


class yuuka_op(C.Structure):
    _fields_ = [
        ("code", C.c_uint32),
        ("flags", C.c_uint32),
        ("buf", C.c_void_p * 16),
        ("off", C.c_uint64 * 16),
        ("n", C.c_uint64 * 6),
        ("u", C.c_uint32 * 4),
        ("f", C.c_float * 4),
    ]


class yuuka_accept_params(C.Structure):
    _fields_ = [
        ("mode", C.c_uint32),
        ("batch", C.c_uint32),
        ("drafts", C.c_uint32),
        ("vocab", C.c_uint32),
        ("temperature", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("request_base", C.c_uint32),
        ("seed", C.c_uint64),
        ("step", C.c_uint64),
        ("row_stride", C.c_uint64),
    ]


class yuuka_device_info(C.Structure):
    _fields_ = [
        ("name", C.c_char * 256),
        ("gcn_arch", C.c_char * 64),
        ("hip_version", C.c_char * 64),
        ("total_memory", C.c_uint64),
        ("compute_units", C.c_uint32),
        ("clock_mhz", C.c_uint32),
        ("pci_domain", C.c_int32),
        ("pci_bus", C.c_int32),
        ("pci_device", C.c_int32),
    ]


_lib = None


def lib() -> C.CDLL:
    """Loads libyuuka_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: run __graft_entry__.build() (there is no CPU fallback)")
        _lib = C.CDLL(str(LIB_PATH), mode=os.RTLD_GLOBAL if hasattr(os, "RTLD_GLOBAL") else 0)
        _declare(_lib)
    return _lib


def _declare(L: C.CDLL) -> None:
    vp, u64, u32, i32 = C.c_void_p, C.c_uint64, C.c_uint32, C.c_int32
    sig = {
        "yuuka_abi_version": (u32, []),
        "yuuka_ext_version": (u32, []),
        "yuuka_last_error": (C.c_char_p, []),
        "yuuka_device_open": (C.c_int, [i32, C.POINTER(vp)]),
        "yuuka_device_close": (None, [vp]),
        "yuuka_device_info_get": (C.c_int, [vp, C.POINTER(yuuka_device_info)]),
        "yuuka_buffer_alloc": (C.c_int, [vp, u64, C.POINTER(vp)]),
        "yuuka_buffer_free": (None, [vp]),
        "yuuka_buffer_size": (u64, [vp]),
        "yuuka_buffer_ptr": (vp, [vp]),
        "yuuka_stream_create": (C.c_int, [vp, C.POINTER(vp)]),
        "yuuka_stream_destroy": (None, [vp]),
        "yuuka_stream_synchronize": (C.c_int, [vp]),
        "yuuka_event_create": (C.c_int, [vp, C.POINTER(vp)]),
        "yuuka_event_destroy": (None, [vp]),
        "yuuka_event_wait": (C.c_int, [vp]),
        "yuuka_memcpy_h2d": (C.c_int, [vp, vp, u64]),
        "yuuka_memcpy_d2h": (C.c_int, [vp, vp, u64]),
        "yuuka_memcpy_d2h_at": (C.c_int, [vp, vp, u64, u64]),
        "yuuka_memset": (C.c_int, [vp, vp, C.c_int, u64]),
        "yuuka_buffer_copy": (C.c_int, [vp, vp, u64, vp, u64, u64, vp]),
        "yuuka_dynamic_set": (C.c_int, [vp, vp, i32, u32]),
        "yuuka_add_f32": (C.c_int, [vp, vp, vp, vp, u64, vp]),
        "yuuka_lm_head": (C.c_int, [vp, vp, vp, vp, u64, u64, u64, u32, vp]),
        "yuuka_gemv": (C.c_int, [vp, vp, vp, vp, u64, u64, u32, vp]),
        "yuuka_gemv_batch": (C.c_int, [vp, vp, vp, vp, u64, u64, u64, u32, vp]),
        "yuuka_dequant_f32": (C.c_int, [vp, vp, vp, u64, u64, u32, vp]),
        "yuuka_moe_pack_q4k": (C.c_int, [vp, vp, vp, u64, u64, vp]),
        "yuuka_dequant_f16": (C.c_int, [vp, vp, vp, u64, u64, u32, vp]),
        "yuuka_verify_accept": (C.c_int, [vp, vp, u64, vp, u64, vp, u64, vp,
                                          C.POINTER(yuuka_accept_params), vp]),
        "yuuka_verify_accept_noalloc": (C.c_int, [vp, vp, u64, vp, u64, vp, u64, C.POINTER(yuuka_accept_params),
                                                  vp]),
        "yuuka_noalloc_accept_bytes": (u64, [C.POINTER(yuuka_accept_params)]),
        "yuuka_event_create_timed": (C.c_int, [vp, C.POINTER(vp)]),
        "yuuka_event_record": (C.c_int, [vp, vp]),
        "yuuka_event_elapsed_ms": (C.c_int, [vp, vp, C.POINTER(C.c_float)]),
        "yuuka_quantized_bytes": (u64, [u64, u64]),
        "yuuka_quantize_activations": (C.c_int, [vp, vp, vp, u64, u64, vp]),
        "yuuka_gemm_quantized": (C.c_int, [vp, vp, vp, vp, u64, u64, u64, u32, vp]),
        "yuuka_plan_create": (C.c_int, [vp, C.POINTER(vp)]),
        "yuuka_plan_destroy": (None, [vp]),
        "yuuka_plan_add": (C.c_int, [vp, C.POINTER(yuuka_op)]),
        "yuuka_plan_execute": (C.c_int, [vp, vp, i32, u32, C.c_int, vp]),
        "yuuka_plan_execute_profiled": (C.c_int, [vp, vp, i32, u32, C.c_int, C.POINTER(u32),
                                                  C.POINTER(u64), u64, C.POINTER(u64), vp]),
        "yuuka_graph_create": (C.c_int, [vp, vp, vp, C.c_int, C.POINTER(vp)]),
        "yuuka_graph_replay": (C.c_int, [vp, vp, vp]),
        "yuuka_graph_destroy": (None, [vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def header_symbols() -> list[str]:
    """Function names declared with YUUKA_API in include/yuuka_hip.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"YUUKA_API[^;(]*?\b(yuuka_\w+)\s*\(", text, re.S)))


def check(status: int, what: str) -> None:
    if status != OK:
        msg = lib().yuuka_last_error().decode(errors="replace")
        cls = Unsupported if status == UNSUPPORTED else HipError
        raise cls(status, what, msg)


class Device:
    def __init__(self, index: int = 0):
        p = C.c_void_p()
        check(lib().yuuka_device_open(index, C.byref(p)), "device_open")
        self.ptr = p

    def info(self) -> dict:
        inf = yuuka_device_info()
        check(lib().yuuka_device_info_get(self.ptr, C.byref(inf)), "device_info")
        return dict(name=inf.name.decode(), gcn_arch=inf.gcn_arch.decode(),
                    total_memory=inf.total_memory, compute_units=inf.compute_units,
                    clock_mhz=inf.clock_mhz)

    def close(self) -> None:
        if self.ptr:
            lib().yuuka_device_close(self.ptr)
            self.ptr = None

    def alloc(self, nbytes: int) -> "Buffer":
        return Buffer(self, nbytes)

    def upload(self, arr: np.ndarray) -> "Buffer":
        arr = np.ascontiguousarray(arr)
        b = Buffer(self, max(arr.nbytes, 1))
        b.write(arr)
        return b


class Buffer:
    def __init__(self, dev: Device, nbytes: int):
        p = C.c_void_p()
        check(lib().yuuka_buffer_alloc(dev.ptr, int(nbytes), C.byref(p)), "buffer_alloc")
        self.ptr = p
        self.nbytes = int(nbytes)

    def write(self, arr: np.ndarray, ) -> None:
        arr = np.ascontiguousarray(arr)
        check(lib().yuuka_memcpy_h2d(self.ptr, arr.ctypes.data_as(C.c_void_p), arr.nbytes), "memcpy_h2d")

    def read(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        check(lib().yuuka_memcpy_d2h_at(out.ctypes.data_as(C.c_void_p), self.ptr, offset, out.nbytes),
              "memcpy_d2h")
        return out

    @property
    def device_ptr(self) -> int:
        return lib().yuuka_buffer_ptr(self.ptr)

    def free(self) -> None:
        if self.ptr:
            lib().yuuka_buffer_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self, dev: Device):
        p = C.c_void_p()
        check(lib().yuuka_stream_create(dev.ptr, C.byref(p)), "stream_create")
        self.ptr = p

    def sync(self) -> None:
        check(lib().yuuka_stream_synchronize(self.ptr), "stream_synchronize")

    def destroy(self) -> None:
        if self.ptr:
            lib().yuuka_stream_destroy(self.ptr)
            self.ptr = None


class Event:
    def __init__(self, dev: Device, timed: bool = False):
        p = C.c_void_p()
        fn = lib().yuuka_event_create_timed if timed else lib().yuuka_event_create
        check(fn(dev.ptr, C.byref(p)), "event_create")
        self.ptr = p

    def record(self, stream: "Stream") -> None:
        check(lib().yuuka_event_record(self.ptr, stream.ptr), "event_record")

    def elapsed_ms(self, start: "Event") -> float:
        ms = C.c_float()
        check(lib().yuuka_event_elapsed_ms(start.ptr, self.ptr, C.byref(ms)), "event_elapsed")
        return float(ms.value)

    def wait(self) -> None:
        check(lib().yuuka_event_wait(self.ptr), "event_wait")

    def destroy(self) -> None:
        if self.ptr:
            lib().yuuka_event_destroy(self.ptr)
            self.ptr = None


def _p(b):
    return None if b is None else b.ptr


def lm_head(stream: Stream, out: Buffer, x: Buffer, w: Buffer, n_in: int, n_out: int, rows: int,
            dtype: int, event: Event | None = None) -> None:
    check(lib().yuuka_lm_head(stream.ptr, out.ptr, x.ptr, w.ptr, n_in, n_out, rows, dtype, _p(event)),
          "lm_head")


def quantized_bytes(n_in: int, rows: int) -> int:
    return int(lib().yuuka_quantized_bytes(n_in, rows))


def quantize_activations(stream: Stream, xq: Buffer, x: Buffer, n_in: int, rows: int) -> None:
    check(lib().yuuka_quantize_activations(stream.ptr, xq.ptr, x.ptr, n_in, rows, None),
          "quantize_activations")


def gemm_quantized(stream: Stream, out: Buffer, xq: Buffer, w: Buffer, n_in: int, n_out: int,
                   rows: int, dtype: int) -> None:
    check(lib().yuuka_gemm_quantized(stream.ptr, out.ptr, xq.ptr, w.ptr, n_in, n_out, rows, dtype, None),
          "gemm_quantized")


def dequant_f32(stream: Stream, dst: Buffer, src: Buffer, n_in: int, n_out: int, dtype: int) -> None:
    check(lib().yuuka_dequant_f32(stream.ptr, dst.ptr, src.ptr, n_in, n_out, dtype, None), "dequant_f32")


def moe_pack_q4k(stream: Stream, dst: Buffer, src: Buffer, rows: int, n_in: int) -> None:
    """Expert-stacked Q4_K rows into the packed layout of FLAG_MOE_PACKED."""
    check(lib().yuuka_moe_pack_q4k(stream.ptr, dst.ptr, src.ptr, rows, n_in, None), "moe_pack_q4k")


def verify_accept(stream: Stream, logits: Buffer, drafts: Buffer | None, result: Buffer,
                  params: yuuka_accept_params, debug: Buffer | None = None,
                  logits_offset: int = 0, drafts_offset: int = 0, result_offset: int = 0) -> None:
    check(lib().yuuka_verify_accept(stream.ptr, logits.ptr, logits_offset, _p(drafts), drafts_offset,
                                    result.ptr, result_offset, _p(debug), C.byref(params), None),
          "verify_accept")


def accept_params(mode: int, batch: int, drafts: int, vocab: int, temperature: float = 0.0,
                  top_k: int = 0, top_p: float = 1.0, seed: int = 0, step: int = 0,
                  request_base: int = 0, row_stride: int = 0) -> yuuka_accept_params:
    return yuuka_accept_params(mode, batch, drafts, vocab, temperature, top_k, top_p, request_base,
                               seed, step, row_stride)


def gemm_fused_op(plan: "Plan", x: Buffer, n_in: int, rows: int, segments, epilogue: int = 0,
                  norm: Buffer | None = None, eps: float = 1e-6) -> None:
    """Appends one GEMM_FUSED op. segments: [(w, dtype, n_out, out, residual)]
    (out / residual may be None where the epilogue does not use them)."""
    bufs = [None] * 14
    bufs[0], bufs[1] = x, norm
    n = [n_in, rows, 0, 0, 0, 0]
    dt = 0
    for i, (w, dtype, n_out, out, res) in enumerate(segments):
        bufs[2 + i], bufs[6 + i], bufs[10 + i] = w, out, res
        n[2 + i] = n_out
        dt |= dtype << (8 * i)
    plan.add(OP["GEMM_FUSED"], bufs, n=n, u=[dt, epilogue], f=[eps])


class Plan:
    """Mirror of hip.Plan (backend/hip/hip.go:365-430): ops are validated and
    appended; a rejected op raises and is not appended."""

    def __init__(self, dev: Device):
        p = C.c_void_p()
        check(lib().yuuka_plan_create(dev.ptr, C.byref(p)), "plan_create")
        self.ptr = p
        self.keep = []
        self.tail = False

    def mark_tail(self) -> None:
        self.tail = True

    def add(self, code: int, bufs=(), offs=(), n=(), u=(), f=(), flags: int = 0) -> None:
        op = yuuka_op()
        op.code = code
        op.flags = flags | (FLAG_TAIL if self.tail else 0)
        for i, b in enumerate(bufs):
            op.buf[i] = None if b is None else b.ptr.value
            if b is not None:
                self.keep.append(b)
        for i, v in enumerate(offs):
            op.off[i] = int(v)
        for i, v in enumerate(n):
            op.n[i] = int(v)
        for i, v in enumerate(u):
            op.u[i] = int(v)
        for i, v in enumerate(f):
            op.f[i] = float(v)
        check(lib().yuuka_plan_add(self.ptr, C.byref(op)), f"plan_add(op {code})")

    def execute(self, stream: Stream, token: int = 0, position: int = 0, run_tail: bool = True,
                event: Event | None = None) -> None:
        check(lib().yuuka_plan_execute(self.ptr, stream.ptr, token, position, int(run_tail), _p(event)),
              "plan_execute")

    def execute_profiled(self, stream: Stream, token: int = 0, position: int = 0,
                         run_tail: bool = True, capacity: int = 4096):
        codes = (C.c_uint32 * capacity)()
        times = (C.c_uint64 * capacity)()
        count = C.c_uint64()
        check(lib().yuuka_plan_execute_profiled(self.ptr, stream.ptr, token, position, int(run_tail),
                                                codes, times, capacity, C.byref(count), None),
              "plan_execute_profiled")
        k = min(count.value, capacity)
        return list(codes[:k]), list(times[:k])

    def destroy(self) -> None:
        if self.ptr:
            lib().yuuka_plan_destroy(self.ptr)
            self.ptr = None


class Graph:
    def __init__(self, plan: Plan, stream: Stream, dynamic: Buffer | None, run_tail: bool = True):
        p = C.c_void_p()
        check(lib().yuuka_graph_create(plan.ptr, stream.ptr, _p(dynamic), int(run_tail), C.byref(p)),
              "graph_create")
        self.ptr = p

    def replay(self, stream: Stream, event: Event | None = None) -> None:
        check(lib().yuuka_graph_replay(self.ptr, stream.ptr, _p(event)), "graph_replay")

    def destroy(self) -> None:
        if self.ptr:
            lib().yuuka_graph_destroy(self.ptr)
            self.ptr = None
