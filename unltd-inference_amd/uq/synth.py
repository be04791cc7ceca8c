"""Seeded synthetic GGUF blocks and activations for the quantized linear path.

Field distributions follow the benchmark configurations of the path:
  Q4_K (144 B / 256 weights): d, dmin = f16(|N(0, sigma)|), scales[12] and
      qs[128] uniform random bytes (every 6-bit sc/m uniform 0..63, every
      nibble uniform 0..15).
  Q6_K (210 B / 256 weights): ql[128], qh[64] uniform bytes, scales[16] int8
      uniform in [-64, 63], d = f16(|N(0, sigma)|) stored last.
  Q8_0 (34 B / 32 weights): d = f16(|N(0, sigma)|), qs[32] int8 uniform in
      [-127, 127].
  activations: N(0, 1) float32.
Block layouts: crates/unltd-tensor/src/quants.rs:116-124 (Q4_K), :158-165
(Q6_K); Q8_0 per ggml_type_blocksize(8) = (34, 32), gguf.rs:202.
The generator is numpy's PCG64 with an explicit seed, so every run (CPU or
GPU host) sees the same bytes.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, Q8_0: 34}
BLOCK_ELEMS = {Q4_K: 256, Q6_K: 256, Q8_0: 32}
DEFAULT_SIGMA = {Q4_K: 2e-3, Q6_K: 1e-3, Q8_0: 5e-3}
SEED_BASE = 0x554E4C5400000000


def seed_for(config_id: int, salt: int = 0) -> int:
    return (SEED_BASE + config_id + (salt << 8)) & ((1 << 64) - 1)


def row_bytes(dtype: int, dim_in: int) -> int:
    if dtype == F32:
        return 4 * dim_in
    return dim_in // BLOCK_ELEMS[dtype] * BLOCK_BYTES[dtype]


def _f16_bytes(rng, n: int, sigma: float) -> np.ndarray:
    v = np.abs(rng.normal(0.0, sigma, n)).astype(np.float16)
    return v.view(np.uint8).reshape(n, 2)


def blocks(dtype: int, nblocks: int, rng, sigma: float | None = None) -> np.ndarray:
    """nblocks blocks of `dtype`, as a flat uint8 array in GGUF layout."""
    sigma = DEFAULT_SIGMA[dtype] if sigma is None else sigma
    nb = BLOCK_BYTES[dtype]
    b = rng.integers(0, 256, size=(nblocks, nb), dtype=np.uint8)
    if dtype == Q4_K:
        b[:, 0:2] = _f16_bytes(rng, nblocks, sigma)
        b[:, 2:4] = _f16_bytes(rng, nblocks, sigma)
    elif dtype == Q6_K:
        b[:, 192:208] = rng.integers(-64, 64, size=(nblocks, 16), dtype=np.int8).view(np.uint8)
        b[:, 208:210] = _f16_bytes(rng, nblocks, sigma)
    elif dtype == Q8_0:
        b[:, 0:2] = _f16_bytes(rng, nblocks, sigma)
        b[:, 2:34] = rng.integers(-127, 128, size=(nblocks, 32), dtype=np.int8).view(np.uint8)
    else:
        raise ValueError(f"dtype {dtype}")
    return b.reshape(-1)


def weights(dtype: int, dim_out: int, dim_in: int, seed: int, sigma: float | None = None):
    """Row-major [dim_out] rows of packed blocks, dim_in weights per row."""
    rng = np.random.Generator(np.random.PCG64(seed))
    if dtype == F32:
        return rng.normal(0.0, 0.05, dim_out * dim_in).astype(np.float32).view(np.uint8)
    return blocks(dtype, dim_out * dim_in // BLOCK_ELEMS[dtype], rng, sigma)


def activations(n: int, seed: int, rows: int = 1) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed ^ 0x5A5A5A5A))
    x = rng.standard_normal(rows * n, dtype=np.float32)
    return x if rows == 1 else x.reshape(rows, n)
