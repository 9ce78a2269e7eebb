"""Seeded synthetic inputs of the benchmark configurations.

Weights are generated directly as packed GGUF super-blocks with numpy:
random quant bytes, random 6-bit (Q4_K) or int8 (Q6_K) sub-block scales and
fp16 super-block scales. Configuration 1 draws d and dmin from |N(0, 0.02)|
as specified. The model configurations instead choose the fp16 scale spread
so that the dequantized weights have a standard deviation near 0.02 (the
"normal(0, 0.02) before quantization" of the model configs is matched in
spread, not by running a quantizer).
"""
from __future__ import annotations

import numpy as np

Q4_K, Q6_K = 12, 14
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210}


def _f16_bits(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def q4k_blocks(rng: np.random.Generator, nblocks: int, d_sigma: float = 0.02,
               dmin_ratio: float | None = None) -> np.ndarray:
    """nblocks Q4_K super-blocks (144 B each): d, dmin fp16, 12 B packed
    6-bit scales/mins (uniform 0..63), 128 B of uniform nibbles."""
    b = rng.integers(0, 256, size=(nblocks, 144), dtype=np.uint8)
    d = np.abs(rng.normal(0.0, d_sigma, size=nblocks)).astype(np.float32)
    if dmin_ratio is None:
        dmin = np.abs(rng.normal(0.0, d_sigma, size=nblocks)).astype(np.float32)
    else:
        dmin = d * np.float32(dmin_ratio)
    b[:, 0:2] = _f16_bits(d).view(np.uint8).reshape(nblocks, 2)
    b[:, 2:4] = _f16_bits(dmin).view(np.uint8).reshape(nblocks, 2)
    return b


def q6k_blocks(rng: np.random.Generator, nblocks: int, d_sigma: float = 0.02,
               scale_max: int = 127) -> np.ndarray:
    """nblocks Q6_K super-blocks (210 B): ql, qh uniform bytes, int8 scales
    uniform in [-scale_max, scale_max], fp16 d from |N(0, d_sigma)|."""
    b = rng.integers(0, 256, size=(nblocks, 210), dtype=np.uint8)
    sc = rng.integers(-scale_max, scale_max + 1, size=(nblocks, 16)).astype(np.int8)
    b[:, 192:208] = sc.view(np.uint8)
    d = np.abs(rng.normal(0.0, d_sigma, size=nblocks)).astype(np.float32)
    b[:, 208:210] = _f16_bits(d).view(np.uint8).reshape(nblocks, 2)
    return b


def quant_matrix(rng: np.random.Generator, dtype: int, rows: int, cols: int,
                 model_scale: bool = False) -> np.ndarray:
    """Packed [rows, cols] matrix as a flat uint8 array."""
    assert cols % 256 == 0
    nb = rows * (cols // 256)
    if dtype == Q4_K:
        blk = q4k_blocks(rng, nb, d_sigma=1.4e-4, dmin_ratio=3.75) if model_scale else q4k_blocks(rng, nb)
    elif dtype == Q6_K:
        blk = q6k_blocks(rng, nb, d_sigma=1.0e-4, scale_max=31) if model_scale else q6k_blocks(rng, nb)
    else:
        raise ValueError(dtype)
    return blk.reshape(-1)


def config1(seed: int = 0):
    """Configuration 1: one Q4_K 9216x2560 layer, M=5 fp32 rows ~ N(0,1),
    logits 5 x 151936 ~ N(0, 3), 4 drafts uniform in the vocabulary."""
    rng = np.random.default_rng(seed)
    N, K, M, V, k = 9216, 2560, 5, 151936, 4
    w = quant_matrix(rng, Q4_K, N, K)
    x = rng.normal(0.0, 1.0, size=(M, K)).astype(np.float32)
    logits = rng.normal(0.0, 3.0, size=(k + 1, V)).astype(np.float32)
    drafts = rng.integers(0, V, size=k, dtype=np.int32)
    return dict(N=N, K=K, M=M, V=V, k=k, w=w, x=x, logits=logits, drafts=drafts)


def q4k_from_int(w: np.ndarray, d: float = 1.0) -> np.ndarray:
    """Packs an integer matrix with entries in [-8, 7] as Q4_K so that it
    dequantizes to exactly d * w (tensor/quant.go:96-125 layout): fp16 d and
    dmin = d, every 6-bit sub-block scale 1 and min 8, nibble = w + 8. d must
    be representable in fp16. Used to build models whose layers reduce to
    closed forms."""
    w = np.asarray(w)
    rows, cols = w.shape
    assert cols % 256 == 0 and w.min() >= -8 and w.max() <= 7
    q = (w + 8).astype(np.uint8).reshape(rows * cols // 256, 4, 2, 32)
    nb = q.shape[0]
    b = np.zeros((nb, 144), np.uint8)
    hd = _f16_bits(np.full(nb, d, np.float32)).view(np.uint8).reshape(nb, 2)
    b[:, 0:2] = hd
    b[:, 2:4] = hd
    b[:, 4:8] = 1            # sub-block scales 0..3 (high bits of 4..7 zero)
    b[:, 8:12] = 8           # sub-block mins 0..3
    b[:, 12:16] = 0x81       # scale 1 | min 8 << 4 for sub-blocks 4..7
    b[:, 16:144] = (q[:, :, 0, :] | (q[:, :, 1, :] << 4)).reshape(nb, 128)
    return b.reshape(-1)
