"""Helpers shared by the test modules (bit views, seeded inputs, tolerances)."""

from __future__ import annotations

import numpy as np
import torch


def bits16(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit patterns (host)."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bits8(t: torch.Tensor) -> np.ndarray:
    """int8 / e4m3fn tensor -> uint8 codes (host)."""
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def from_bits16(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def activations(m: int, k: int, seed: int = 0, outlier_channels: int = 0, outlier_scale: float = 20.0,
                student_t: bool = False) -> torch.Tensor:
    """N(0,1) activations with a few seeded outlier channels (the BASELINE.json configurations)."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=gen)
    if outlier_channels:
        idx = torch.randperm(k, generator=gen)[:outlier_channels]
        if student_t:
            df = 3.0
            z = torch.randn(m, outlier_channels, generator=gen)
            chi = torch.distributions.Chi2(torch.full((outlier_channels,), df)).sample((m,))
            x[:, idx] = z / torch.sqrt(chi / df)
        else:
            x[:, idx] *= outlier_scale
    return x.to(torch.bfloat16)


def weights(n: int, k: int, seed: int = 1, std: float = 0.02) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(n, k, generator=gen) * std).to(torch.bfloat16)


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |v| (8 significant bits)."""
    a = np.abs(v.astype(np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def fp32_gemm_bound(k: int, abs_sum: np.ndarray) -> np.ndarray:
    """Worst-case error of a binary32 accumulation of k terms: k * 2^-24 * sum|terms|."""
    return k * 2.0 ** -24 * abs_sum


def to_tiled(codes: np.ndarray) -> np.ndarray:
    """Row-major [R, K] codes (R % 16 == 0, K % 128 == 0) -> the bytes of the
    tiled layout, as an [R, K] array: 16-row x 128-byte blocks of 2 KiB, block
    (b, s) at (b * K / 128 + s) * 2048, inside it byte k of row r at
    (k % 32 // 16) * 1024 + (r % 16 + 16 * (k % 128 // 32)) * 16 + k % 16."""
    r, k = codes.shape
    c = np.ascontiguousarray(codes).reshape(r // 16, 16, k // 128, 4, 2, 16)  # b, r16, s, q, h, byte
    return np.ascontiguousarray(c.transpose(0, 2, 4, 3, 1, 5)).reshape(r, k)  # b, s, h, q, r16, byte


def from_tiled(tiled: np.ndarray, r: int, k: int) -> np.ndarray:
    """Inverse of to_tiled: the tiled bytes of an [R, K] code matrix -> row-major [R, K]."""
    t = np.ascontiguousarray(tiled).reshape(r // 16, k // 128, 2, 4, 16, 16)  # b, s, h, q, r16, byte
    return np.ascontiguousarray(t.transpose(0, 4, 1, 3, 2, 5)).reshape(r, k)
