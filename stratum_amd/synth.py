"""Seeded synthetic k-quant weights and activations (numpy, host side).

The benchmark configurations name synthetic inputs: random super-blocks
with the field distributions below and x ~ N(0, 1) in binary32.  These
generators produce those bytes deterministically from a seed
(numpy PCG64), so the GPU run, the CPU baseline and the parity tests all
see identical inputs.

  Q4_K  d, dmin = fp16(|N(0,1)| * 0.01); 8 scales and 8 mins uniform
        0..63 packed by inverting q4k_get_scale_min (stratum_q4k.h:57-65);
        nibbles uniform 0..15.
  Q6_K  ql, qh uniform bytes; int8 scales uniform -128..127;
        d = fp16(|N(0,1)| * 0.01).
  Q2_K  scale bytes uniform 0..255; qs uniform; d, dmin as Q4_K.
  type 42  the Q2_K blocks above re-laid by the converter.
  Q5_K  d, dmin and scales as Q4_K; qh and qs uniform bytes.
  Q3_K  hmask, qs and the 12 packed scale bytes uniform; d as Q4_K.
  Q8_0  per 32 weights d = fp16(|N(0,1)| * 0.01), int8 quants uniform.
  F16   weights fp16(N(0,1) * 0.05).   F32  weights N(0,1) * 0.05.

fp16 fields use numpy's round-to-nearest-even binary32 -> binary16.
"""
from __future__ import annotations

import numpy as np

from . import (BLOCK_BYTES, TYPE_F16, TYPE_F32, TYPE_Q2_K, TYPE_Q2K_NIB, TYPE_Q3_K, TYPE_Q4_K,
               TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0)


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def gaussian(r: np.random.Generator, n: int) -> np.ndarray:
    return r.standard_normal(n, dtype=np.float32)


def _fp16_scale(r: np.random.Generator, n: int) -> np.ndarray:
    v = np.abs(r.standard_normal(n, dtype=np.float32)) * np.float32(0.01)
    return v.astype(np.float16).view(np.uint16)


def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of q4k_get_scale_min: [n, 8] scales and mins (0..63) -> [n, 12]."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.empty((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = m[:, 0:4] | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    return out


def q4k_blocks(r: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 144), np.uint8)
    b[:, 0:2] = _fp16_scale(r, nblocks).view(np.uint8).reshape(nblocks, 2)
    b[:, 2:4] = _fp16_scale(r, nblocks).view(np.uint8).reshape(nblocks, 2)
    sc = r.integers(0, 64, (nblocks, 8), dtype=np.uint8)
    m = r.integers(0, 64, (nblocks, 8), dtype=np.uint8)
    b[:, 4:16] = pack_q4k_scales(sc, m)
    b[:, 16:144] = r.integers(0, 256, (nblocks, 128), dtype=np.uint8)
    return b.reshape(-1)


def q6k_blocks(r: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 210), np.uint8)
    b[:, 0:208] = r.integers(0, 256, (nblocks, 208), dtype=np.uint8)  # ql, qh, scales
    b[:, 208:210] = _fp16_scale(r, nblocks).view(np.uint8).reshape(nblocks, 2)
    return b.reshape(-1)


def q2k_blocks(r: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 84), np.uint8)
    b[:, 0:80] = r.integers(0, 256, (nblocks, 80), dtype=np.uint8)  # scales, qs
    b[:, 80:82] = _fp16_scale(r, nblocks).view(np.uint8).reshape(nblocks, 2)
    b[:, 82:84] = _fp16_scale(r, nblocks).view(np.uint8).reshape(nblocks, 2)
    return b.reshape(-1)


def q5k_blocks(r: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 176), np.uint8)
    b[:, 0:2] = _fp16_scale(r, nblocks).view(np.uint8).reshape(nblocks, 2)
    b[:, 2:4] = _fp16_scale(r, nblocks).view(np.uint8).reshape(nblocks, 2)
    sc = r.integers(0, 64, (nblocks, 8), dtype=np.uint8)
    m = r.integers(0, 64, (nblocks, 8), dtype=np.uint8)
    b[:, 4:16] = pack_q4k_scales(sc, m)
    b[:, 16:176] = r.integers(0, 256, (nblocks, 160), dtype=np.uint8)   # qh, qs
    return b.reshape(-1)


def q3k_blocks(r: np.random.Generator, nblocks: int) -> np.ndarray:
    b = np.empty((nblocks, 110), np.uint8)
    b[:, 0:108] = r.integers(0, 256, (nblocks, 108), dtype=np.uint8)  # hmask, qs, scales
    b[:, 108:110] = _fp16_scale(r, nblocks).view(np.uint8).reshape(nblocks, 2)
    return b.reshape(-1)


def q8_0_blocks(r: np.random.Generator, nblocks: int) -> np.ndarray:
    """nblocks super-blocks of 256 weights: eight 34-byte Q8_0 blocks each."""
    n = 8 * nblocks
    b = np.empty((n, 34), np.uint8)
    b[:, 0:2] = _fp16_scale(r, n).view(np.uint8).reshape(n, 2)
    b[:, 2:34] = r.integers(0, 256, (n, 32), dtype=np.uint8)
    return b.reshape(-1)


def f16_blocks(r: np.random.Generator, nblocks: int) -> np.ndarray:
    v = r.standard_normal(256 * nblocks, dtype=np.float32) * np.float32(0.05)
    return v.astype(np.float16).view(np.uint8).copy()


def f32_blocks(r: np.random.Generator, nblocks: int) -> np.ndarray:
    v = r.standard_normal(256 * nblocks, dtype=np.float32) * np.float32(0.05)
    return v.view(np.uint8).copy()


def q2k_to_nib(q2k: np.ndarray) -> np.ndarray:
    """Type-42 layout of Q2_K blocks (tools_gguf_nib_convert.c:99-120).

    Weight p (0..255) of a block holds (qs[32*(p//128) + p%32] >> 2*((p%128)//32)) & 3
    in Q2_K; type 42 stores it in byte 16 + 16*(p//32) + p%16, low nibble
    when p%32 < 16, else high nibble.  scales stay at bytes 0..15, d and
    dmin move to bytes 144..147.
    """
    src = q2k.reshape(-1, 84)
    n = src.shape[0]
    out = np.zeros((n, 148), np.uint8)
    out[:, 0:16] = src[:, 0:16]
    out[:, 144:148] = src[:, 80:84]
    qs = src[:, 16:80]
    p = np.arange(256)
    vals = (qs[:, 32 * (p // 128) + p % 32] >> (2 * ((p % 128) // 32))) & 3  # [n, 256]
    lo = vals[:, (p % 32) < 16].reshape(n, 8, 16)
    hi = vals[:, (p % 32) >= 16].reshape(n, 8, 16)
    out[:, 16:144] = (lo | (hi << 4)).reshape(n, 128).astype(np.uint8)
    return out.reshape(-1)


def blocks(qtype: int, r: np.random.Generator, nblocks: int) -> np.ndarray:
    if qtype == TYPE_Q4_K:
        return q4k_blocks(r, nblocks)
    if qtype == TYPE_Q6_K:
        return q6k_blocks(r, nblocks)
    if qtype == TYPE_Q2_K:
        return q2k_blocks(r, nblocks)
    if qtype == TYPE_Q2K_NIB:
        return q2k_to_nib(q2k_blocks(r, nblocks))
    if qtype == TYPE_Q5_K:
        return q5k_blocks(r, nblocks)
    if qtype == TYPE_Q3_K:
        return q3k_blocks(r, nblocks)
    if qtype == TYPE_Q8_0:
        return q8_0_blocks(r, nblocks)
    if qtype == TYPE_F16:
        return f16_blocks(r, nblocks)
    if qtype == TYPE_F32:
        return f32_blocks(r, nblocks)
    raise ValueError(f"type {qtype}")


def tensor(qtype: int, N: int, K: int, seed: int) -> np.ndarray:
    """N x K weight tensor (rows contiguous) as raw block bytes."""
    assert K % 256 == 0
    return blocks(qtype, rng(seed), N * (K // 256))


def row_bytes(qtype: int, K: int) -> int:
    return (K // 256) * BLOCK_BYTES[qtype]
