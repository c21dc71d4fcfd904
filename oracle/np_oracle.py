"""Independent numpy restatement of the Q8_0 / Q4_0 codec (test infrastructure only).

Written separately from ``oracle.c`` (vectorised, and leaning on numpy's IEEE float16 casts for
the scale instead of bit manipulation) so the two can check each other: a dropped term, a wrong
rounding mode or a swapped nibble in either shows up as a byte mismatch. Follows
ferrum_gguf/src/codec/quant.rs:50-136.
"""
from __future__ import annotations

import numpy as np


def _round_half_away(v: np.ndarray) -> np.ndarray:
    """Rust's f32::round: the fractional part of |v| is exact in f32, so compare it to 0.5."""
    a = np.abs(v)
    t = np.trunc(a)
    r = t + (a - t >= np.float32(0.5)).astype(np.float32)
    return np.where(v < 0, -r, r).astype(np.float32)


def _sat_trunc(v: np.ndarray, lo: int, hi: int) -> np.ndarray:
    """Rust `as` cast to an integer: truncate, saturate, NaN -> 0."""
    v = np.where(np.isnan(v), np.float32(0), v)
    return np.clip(np.trunc(v), lo, hi).astype(np.int32)


def encode_q8_0(data: np.ndarray) -> np.ndarray:
    """quant.rs:111-119"""
    b = np.asarray(data, np.float32).reshape(-1, 32)
    with np.errstate(all="ignore"):
        amax = np.fmax.reduce(np.abs(b), axis=1, initial=np.float32(0)).astype(np.float32)
        d = (amax / np.float32(127)).astype(np.float32)
        idv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
        q = _sat_trunc(_round_half_away((b * idv[:, None]).astype(np.float32)), -128, 127)
    out = np.empty((b.shape[0], 34), np.uint8)
    with np.errstate(all="ignore"):
        d = d.astype(np.float16)
    out[:, :2] = d.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def encode_q4_0(data: np.ndarray) -> np.ndarray:
    """quant.rs:120-133"""
    b = np.asarray(data, np.float32).reshape(-1, 32)
    a = np.abs(b)
    a_nan = np.where(np.isnan(a), -np.inf, a)
    # first index of the largest magnitude; NaN never wins (the reference's strict `>` fold)
    idx = np.argmax(a_nan, axis=1)
    mx = b[np.arange(b.shape[0]), idx]
    mx = np.where((a_nan.max(axis=1) > 0), mx, np.float32(0)).astype(np.float32)
    with np.errstate(all="ignore"):
        d = (mx / np.float32(-8)).astype(np.float32)
        idv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
        t = ((b * idv[:, None]).astype(np.float32) + np.float32(8.5)).astype(np.float32)
        q = np.clip(_sat_trunc(t, -(2**31), 2**31 - 1), 0, 15).astype(np.uint8)
    out = np.empty((b.shape[0], 18), np.uint8)
    with np.errstate(all="ignore"):
        d = d.astype(np.float16)
    out[:, :2] = d.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.reshape(-1)


def decode_q8_0(data: np.ndarray) -> np.ndarray:
    """quant.rs:71-77"""
    b = np.asarray(data, np.uint8).reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    with np.errstate(all="ignore"):
        return (d * q).astype(np.float32).reshape(-1)


def decode_q4_0(data: np.ndarray) -> np.ndarray:
    """quant.rs:78-86: low nibbles are elements 0..16, high nibbles 16..32."""
    b = np.asarray(data, np.uint8).reshape(-1, 18)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    lo = (b[:, 2:] & 0x0F).astype(np.float32) - np.float32(8)
    hi = (b[:, 2:] >> 4).astype(np.float32) - np.float32(8)
    with np.errstate(all="ignore"):
        return (d * np.concatenate([lo, hi], axis=1)).astype(np.float32).reshape(-1)
