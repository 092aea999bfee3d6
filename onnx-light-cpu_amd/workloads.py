"""Seeded synthetic MatMulNBits workloads (the measurement configurations).

Shapes, distributions and block sizes of the five benchmark configurations:
c1 is the reference-scale GEMV, c2 the Llama-3-8B gate/up decode projection,
c3 the down projection (long K), c4 the prefill GEMM and c5 a stack of 32
Llama-3-8B-shaped decoder layers. Weights are uniform random bytes (so every
nibble is uniform in 0..15), scales uniform in a per-config range, zero points
uniform nibbles when present. Host generation uses numpy's PCG64 with
``seed = 0x4D4E42 + 1000 * config_index + M`` for A and ``0x4D4E42 + 1000 *
config_index`` for the weights.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

SEED_BASE = 0x4D4E42


@dataclass(frozen=True)
class Projection:
    """One MatMulNBits node: attributes plus the synthetic distributions."""
    name: str
    K: int
    N: int
    block_size: int
    has_zero_points: bool
    a_sigma: float = 1.0
    scale_lo: float = 0.005
    scale_hi: float = 0.02

    @property
    def nb(self) -> int:
        return (self.K + self.block_size - 1) // self.block_size

    @property
    def row_bytes(self) -> int:
        return self.nb * self.block_size // 2

    @property
    def zp_row_bytes(self) -> int:
        return (self.nb + 1) // 2

    def weight_bytes(self) -> int:
        """Packed B + fp32 scales + packed zero points, each counted once."""
        return self.N * (self.row_bytes + 4 * self.nb +
                         (self.zp_row_bytes if self.has_zero_points else 0))

    def algorithmic_bytes(self, M: int) -> int:
        """Weights + A (fp32) + Y (fp32): the bytes one call must move."""
        return self.weight_bytes() + 4 * M * self.K + 4 * M * self.N

    def flops(self, M: int) -> int:
        return 2 * M * self.N * self.K


@dataclass(frozen=True)
class Config:
    index: int
    name: str
    projections: tuple
    Ms: tuple
    layers: int = 1
    description: str = ""


C1 = Config(0, "c1", (Projection("c1", 4096, 4096, 32, False),), (1,),
            description="M=1 K=4096 N=4096 bs=32 symmetric (implicit zp=8)")
C2 = Config(1, "c2", (Projection("c2", 4096, 14336, 128, True),), (1, 4, 16),
            description="Llama-3-8B gate/up decode: K=4096 N=14336 bs=128 asymmetric")
C3 = Config(2, "c3", (Projection("c3", 14336, 4096, 32, True, 0.5, 0.002, 0.01),),
            (1, 2, 8, 16),
            description="Llama-3-8B down decode: K=14336 N=4096 bs=32 asymmetric")
C4 = Config(3, "c4", (Projection("c4", 4096, 4096, 128, False),), (2048,),
            description="prefill GEMM: M=2048 K=4096 N=4096 bs=128 symmetric")
C5 = Config(4, "c5", (
    Projection("qkv", 4096, 6144, 128, True),
    Projection("o", 4096, 4096, 128, True),
    Projection("gate_up", 4096, 28672, 128, True),
    Projection("down", 14336, 4096, 128, True),
), (1, 512), layers=32,
            description="32 Llama-3-8B decoder layers, bs=128 asymmetric")

CONFIGS = {c.name: c for c in (C1, C2, C3, C4, C5)}


def weight_seed(config_index: int, layer: int = 0, proj: int = 0) -> int:
    return SEED_BASE + 1000 * config_index + 100000 * layer + 10 * proj


def activation_seed(config_index: int, M: int) -> int:
    return SEED_BASE + 1000 * config_index + M


def make_weights(p: Projection, seed: int):
    """(B [N, nb, bs/2] uint8, scales [N, nb] fp32, zero_points [N, ceil(nb/2)] uint8 | None)."""
    rng = np.random.default_rng(seed)
    B = rng.integers(0, 256, size=(p.N, p.nb, p.block_size // 2), dtype=np.uint8)
    scales = rng.uniform(p.scale_lo, p.scale_hi, size=(p.N, p.nb)).astype(np.float32)
    zp = None
    if p.has_zero_points:
        # With an odd block count the last byte's high nibble is unused; it stays
        # random so that the kernels are seen to ignore it.
        zp = rng.integers(0, 256, size=(p.N, p.zp_row_bytes), dtype=np.uint8)
    return B, scales, zp


def make_activations(M: int, K: int, sigma: float, seed: int):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(size=(M, K)) * sigma).astype(np.float32)
