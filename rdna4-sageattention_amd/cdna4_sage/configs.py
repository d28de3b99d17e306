"""Seeded synthetic inputs for the benchmark configurations of this path.

Every tensor is drawn on the CPU with ``torch.Generator().manual_seed(config index)`` (float32 normal samples, then
rounded to the target dtype) so a CPU checker sees exactly the bits the GPU receives.  Distributions are written as
N(mean, variance): N(0, 3) has standard deviation sqrt(3).

  1  HND [1, 8, 1024, 64] bf16, Q, K, V ~ N(0, 1)                               (plumbing; below MIN_WORK)
  2  HND [1, 24, 4608, 128] bf16, Q, V ~ N(0, 1); K ~ N(0, 1) + offset[c] on 8 random channels, offset ~ N(0, 3)
     shared over tokens and heads                                                 (Flux joint attention)
  3  HND [1, 40, 32760, 128] bf16, N(0, 1); ceil(0.02 * 128) = 3 random channels x10 in K and in V  (Wan 2.1 14B)
  4  HND [1, 24, 67320, 128] bf16, Q, K, V ~ N(0, 0.5^2); K += bias[c] ~ N(0, 2) shared over tokens and heads
                                                                                  (HunyuanVideo)
  5a Q [2, 32, 8192, 128], K/V [2, 8, 8192, 128] bf16, N(0, 1), causal, return_lse  (GQA 4)
  5b Q [2, 16, 8192, 64],  K/V [2, 4, 8192, 64]  bf16, N(0, 1), causal, return_lse

Two more shapes of the reference's model benchmark (tests/bench_models.py:27, :38; README.md:192, :196), for the head
dims the configurations above do not time:
  lumina    HND [1, 24, 4352, 96] bf16, N(0, 1)              (Neta Lumina 1024: head dim 96, no rotation)
  auraflow  HND [2, 12, 4360, 256] fp16, N(0, 1)             (AuraFlow 1024 joint: head dim 256, batch 2)
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Config:
    name: str
    seed: int
    B: int
    H: int
    Hkv: int
    S: int
    D: int
    causal: bool = False
    return_lse: bool = False
    dtype: torch.dtype = torch.bfloat16

    @property
    def shape_q(self):
        return (self.B, self.H, self.S, self.D)

    @property
    def shape_kv(self):
        return (self.B, self.Hkv, self.S, self.D)

    def pairs(self) -> int:
        """(query, key) pairs per head: S^2, or S(S+1)/2 for causal."""
        return self.S * (self.S + 1) // 2 if self.causal else self.S * self.S

    def attention_ops(self) -> int:
        """Algorithmic int8 + fp8 MFMA ops: QK^T and PV, 2 ops per multiply-add each."""
        return 4 * self.B * self.H * self.pairs() * self.D

    def quant_q_bytes(self) -> int:
        n = self.B * self.H * self.S
        return n * self.D * (2 + 1) + 4 * n

    def quant_kv_bytes(self, kv_pad: int) -> int:
        n = self.B * self.Hkv
        return (2 * n * self.S * self.D * 2 + 2 * n * kv_pad * self.D + 4 * n * kv_pad // 32 + 4 * n * self.D)


CONFIGS = {
    "1": Config("plumbing 1x8x1024x64", 1, 1, 8, 8, 1024, 64),
    "2": Config("flux 1x24x4608x128", 2, 1, 24, 24, 4608, 128),
    "3": Config("wan14b 1x40x32760x128", 3, 1, 40, 40, 32760, 128),
    "4": Config("hunyuan 1x24x67320x128", 4, 1, 24, 24, 67320, 128),
    "5a": Config("causal-gqa 2x32/8x8192x128", 5, 2, 32, 8, 8192, 128, causal=True, return_lse=True),
    "5b": Config("causal-gqa 2x16/4x8192x64", 5, 2, 16, 4, 8192, 64, causal=True, return_lse=True),
    "lumina": Config("lumina 1x24x4352x96", 6, 1, 24, 24, 4352, 96),
    "auraflow": Config("auraflow 2x12x4360x256", 7, 2, 12, 12, 4360, 256, dtype=torch.float16),
}


def _normal(g, shape, std=1.0):
    return torch.randn(shape, generator=g, dtype=torch.float32) * std


def make_inputs(cfg: Config, heads: slice | None = None):
    """CPU tensors (q, k, v) in HND layout and cfg.dtype.  ``heads`` restricts the returned KV heads (and the query
    heads that read them) after drawing the full tensors, so a sample matches the full problem bit for bit."""
    g = torch.Generator().manual_seed(cfg.seed)
    key = cfg.name.split()[0]
    if key in ("plumbing", "causal-gqa", "lumina", "auraflow"):
        q, k, v = (_normal(g, s) for s in (cfg.shape_q, cfg.shape_kv, cfg.shape_kv))
    elif key == "flux":
        q, k, v = (_normal(g, s) for s in (cfg.shape_q, cfg.shape_kv, cfg.shape_kv))
        ch = torch.randperm(cfg.D, generator=g)[:8]
        k[..., ch] += _normal(g, (8,), math.sqrt(3.0))
    elif key == "wan14b":
        q, k, v = (_normal(g, s) for s in (cfg.shape_q, cfg.shape_kv, cfg.shape_kv))
        n = math.ceil(0.02 * cfg.D)
        k[..., torch.randperm(cfg.D, generator=g)[:n]] *= 10.0
        v[..., torch.randperm(cfg.D, generator=g)[:n]] *= 10.0
    elif key == "hunyuan":
        q, k, v = (_normal(g, s, 0.5) for s in (cfg.shape_q, cfg.shape_kv, cfg.shape_kv))
        k += _normal(g, (cfg.D,), math.sqrt(2.0))
    else:
        raise KeyError(cfg.name)
    q, k, v = (t.to(cfg.dtype) for t in (q, k, v))
    if heads is not None:
        grp = cfg.H // cfg.Hkv
        k, v = k[:, heads], v[:, heads]
        q = q[:, heads.start * grp: heads.stop * grp]
    return q, k, v


# The model shapes of the reference's benchmark (tests/bench_models.py:15-42): name, B, Sq, Skv, H, D, layout,
# dtype name, causal.  bench.py --models times them with the reference's method (3 warm-ups, median of 10 calls each
# followed by a synchronisation, tests/bench_models.py:45-53) on random N(0, 1) inputs; tests/test_gpu_models.py
# checks the kernel on each of them against the oracle.
MODEL_SHAPES = [
    ("SD1.5 512 (d40->sdpa)", 2, 4096, 4096, 8, 40, "NHD", "f16", False),
    ("SDXL 1024 lvl1 self", 2, 4096, 4096, 10, 64, "NHD", "f16", False),
    ("SDXL 1024 lvl2 self", 2, 1024, 1024, 20, 64, "NHD", "f16", False),
    ("SDXL 1024 lvl1 cross77", 2, 4096, 77, 10, 64, "NHD", "f16", False),
    ("SD3.5L joint", 2, 4250, 4250, 38, 64, "NHD", "f16", False),
    ("Flux 1024 joint", 1, 4352, 4352, 24, 128, "HND", "bf16", False),
    ("Flux 768 joint", 1, 2560, 2560, 24, 128, "HND", "bf16", False),
    ("Flux 512 joint", 1, 1280, 1280, 24, 128, "HND", "bf16", False),
    ("Flux.2 1024 joint", 1, 4608, 4608, 48, 128, "HND", "bf16", False),
    ("Qwen-Image 1328 joint", 1, 6989, 6989, 24, 128, "HND", "bf16", False),
    ("HiDream 1024 joint", 1, 4480, 4480, 20, 128, "NHD", "bf16", False),
    ("Neta Lumina 1024", 1, 4352, 4352, 24, 96, "HND", "bf16", False),
    ("Anima 1024 self", 2, 4096, 4096, 16, 128, "HND", "bf16", False),
    ("Anima 1024 cross512", 2, 4096, 512, 16, 128, "HND", "bf16", False),
    ("Wan1.3B 480p self", 1, 32760, 32760, 12, 128, "NHD", "f16", False),
    ("Wan1.3B 480p cross512", 1, 32760, 512, 12, 128, "NHD", "f16", False),
    ("Wan14B 480p self", 1, 32760, 32760, 40, 128, "NHD", "f16", False),
    ("Wan2.2-5B 704p self", 1, 27280, 27280, 24, 128, "NHD", "f16", False),
    ("HunyuanVideo 544p", 1, 67320, 67320, 24, 128, "HND", "bf16", False),
    ("LTXV-2B 768x512x97", 1, 4992, 4992, 32, 64, "NHD", "bf16", False),
    ("LTXV-2B cross128", 1, 4992, 128, 32, 64, "NHD", "bf16", False),
    ("CogVideoX-5B joint", 1, 17776, 17776, 48, 64, "NHD", "bf16", False),
    ("AuraFlow 1024 joint d256", 2, 4360, 4360, 12, 256, "HND", "f16", False),
    ("causal d128 4k", 1, 4096, 4096, 32, 128, "HND", "bf16", True),
    ("causal d128 16k", 1, 16384, 16384, 32, 128, "HND", "bf16", True),
    ("causal d64 8k", 1, 8192, 8192, 32, 64, "HND", "bf16", True),
]
