"""Seeded synthetic inputs of the BASELINE configurations (C1..C5).

Config i (0-based position in BASELINE.json ``configs``) uses seed 42 + i; 42 is the
reference's SEED (STRATA_KV.py:271).  Every generator draws from an explicit
``torch.Generator`` on the requested device, so the same call gives the same tensors.
The reference holds no datasets for this path; these are the input definitions.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

SEED = 42


@dataclass(frozen=True)
class DecodeShape:
    name: str
    B: int
    Hq: int
    Hkv: int
    d: int
    T: int                # tokens in the cache at the decode step (packed + exact)
    window: int           # exact residual rows
    group_k: int
    group_v: int
    bits: int
    dtype: torch.dtype
    seed: int


C1 = DecodeShape("C1", 1, 8, 8, 128, 4096, 128, 32, 32, 4, torch.float32, SEED + 0)
C2 = DecodeShape("C2", 16, 32, 8, 128, 32768, 128, 64, 64, 4, torch.bfloat16, SEED + 1)


def gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def student_t3(shape, g: torch.Generator, device) -> torch.Tensor:
    """Student-t with 3 degrees of freedom: N / sqrt(chi2_3 / 3), all from ``g``."""
    z = torch.randn(shape, generator=g, device=device)
    chi = torch.randn((*shape, 3), generator=g, device=device).pow(2).sum(-1)
    return z / torch.sqrt(chi / 3.0)


@torch.no_grad()
def decode_inputs(shape: DecodeShape, device="cpu", T: int | None = None, B: int | None = None):
    """(q (B,Hq,1,d), K, V (B,Hkv,T,d)) in shape.dtype.

    C1: K, V, q ~ N(0,1); 4 key channels (drawn without replacement) scaled x10.
    C2: K = N(0,1) * |t3| with one Student-t(3) magnitude per (b, h, channel); V, q ~ N(0,1).
    ``T``/``B`` override the sizes for reduced parity cases (same distributions)."""
    T = shape.T if T is None else T
    B = shape.B if B is None else B
    g = gen(device, shape.seed)
    d = shape.d
    K = torch.randn((B, shape.Hkv, T, d), generator=g, device=device)
    V = torch.randn((B, shape.Hkv, T, d), generator=g, device=device)
    q = torch.randn((B, shape.Hq, 1, d), generator=g, device=device)
    if shape.name == "C1":
        ch = torch.randperm(d, generator=g, device=device)[:4]
        K[..., ch] *= 10.0
    elif shape.name == "C2":
        mag = student_t3((B, shape.Hkv, 1, d), g, device).abs()
        K *= mag
    return q.to(shape.dtype), K.to(shape.dtype), V.to(shape.dtype)
