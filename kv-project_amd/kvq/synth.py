"""Seeded synthetic inputs of the BASELINE configurations (C1..C5).

Config i (0-based position in BASELINE.json ``configs``) uses seed 42 + i; 42 is the
reference's SEED (STRATA_KV.py:271).  Every generator draws from an explicit
``torch.Generator`` on the requested device, so the same call gives the same tensors.
The reference holds no datasets for this path; these are the input definitions.
"""
from __future__ import annotations

import math
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


# ---------------------------------------------------------------------------------------------
# C3 (mixed widths), C4 (eviction), C5 (DCT): BASELINE.json configs 2, 3, 4 (seeds 44, 45, 46)

@dataclass(frozen=True)
class CodedShape:
    name: str
    B: int
    Hq: int
    Hkv: int
    d: int
    T: int
    dtype: torch.dtype
    seed: int


C3 = CodedShape("C3", 8, 32, 8, 128, 16384, torch.bfloat16, SEED + 2)
C4 = CodedShape("C4", 4, 32, 8, 128, 65536, torch.bfloat16, SEED + 3)
C5 = CodedShape("C5", 1, 64, 8, 128, 131072, torch.bfloat16, SEED + 4)
C4_KEEP, C4_WINDOW, C4_STEPS, C4_GROUP = 2048, 256, 32, 64


@torch.no_grad()
def c3_inputs(device="cpu", T: int | None = None, B: int | None = None):
    """(q, K, V, importance): K, V, q ~ N(0,1) (the config states no distribution for them) in
    bf16; block importance ~ LogNormal(0, 1) per (b, KV head, 64-token block)."""
    s = C3
    T = s.T if T is None else T
    B = s.B if B is None else B
    g = gen(device, s.seed)
    K = torch.randn((B, s.Hkv, T, s.d), generator=g, device=device)
    V = torch.randn((B, s.Hkv, T, s.d), generator=g, device=device)
    q = torch.randn((B, s.Hq, 1, s.d), generator=g, device=device)
    imp = torch.exp(torch.randn((B, s.Hkv, T // 64), generator=g, device=device))
    return q.to(s.dtype), K.to(s.dtype), V.to(s.dtype), imp


@torch.no_grad()
def c4_inputs(device="cpu", T: int | None = None, B: int | None = None, steps: int | None = None):
    """(q_steps (steps, B, Hq, 1, d), K, V): K, V, q ~ N(0,1); a seeded 1% of the key positions of
    every (b, KV head) get +3 added to every channel (heavy hitters); bf16."""
    s = C4
    T = s.T if T is None else T
    B = s.B if B is None else B
    steps = C4_STEPS if steps is None else steps
    g = gen(device, s.seed)
    K = torch.randn((B, s.Hkv, T, s.d), generator=g, device=device)
    V = torch.randn((B, s.Hkv, T, s.d), generator=g, device=device)
    q = torch.randn((steps, B, s.Hq, 1, s.d), generator=g, device=device)
    n_hot = max(1, T // 100)
    hot = torch.rand((B, s.Hkv, T), generator=g, device=device).argsort(-1)[..., :n_hot]
    shift = torch.zeros((B, s.Hkv, T), device=device)
    shift.scatter_(2, hot, 3.0)
    K += shift[..., None]
    return q.to(s.dtype), K.to(s.dtype), V.to(s.dtype)


@torch.no_grad()
def ar1(shape, rho: float, g: torch.Generator, device, chunk: int = 256) -> torch.Tensor:
    """Stationary AR(1) along the last axis: x_t = rho x_{t-1} + sqrt(1 - rho^2) e_t, x_{-1} ~ N(0,1),
    float32, computed chunk by chunk with the closed form x = A e + rho^(i+1) x_prev."""
    *lead, T = shape
    e = torch.randn((*lead, T), generator=g, device=device) * math.sqrt(1.0 - rho * rho)
    x_prev = torch.randn(lead, generator=g, device=device)
    i = torch.arange(chunk, device=device, dtype=torch.float64)
    A = torch.where(i[:, None] >= i[None, :], rho ** (i[:, None] - i[None, :]), torch.zeros((), dtype=torch.float64,
                                                                                          device=device)).float()
    carry = (rho ** (i + 1)).float()
    out = torch.empty_like(e)
    for t0 in range(0, T, chunk):
        L = min(chunk, T - t0)
        blk = e[..., t0:t0 + L] @ A[:L, :L].T + carry[:L] * x_prev[..., None]
        out[..., t0:t0 + L] = blk
        x_prev = blk[..., -1]
    return out


@torch.no_grad()
def c5_inputs(device="cpu", T: int | None = None):
    """(q, K, V): per (KV head, channel) a stationary AR(1) series along tokens (rho = 0.95) plus
    N(0, 0.1^2) noise, in bf16; q ~ N(0,1)."""
    s = C5
    T = s.T if T is None else T
    g = gen(device, s.seed)
    K = ar1((s.B, s.Hkv, s.d, T), 0.95, g, device).transpose(2, 3)
    K = K + 0.1 * torch.randn(K.shape, generator=g, device=device)
    V = ar1((s.B, s.Hkv, s.d, T), 0.95, g, device).transpose(2, 3)
    V = V + 0.1 * torch.randn(V.shape, generator=g, device=device)
    q = torch.randn((s.B, s.Hq, 1, s.d), generator=g, device=device)
    return q.to(s.dtype), K.contiguous().to(s.dtype), V.contiguous().to(s.dtype)
