"""Seeded synthetic KV-cache pages for the benchmark configurations.

No model weights or datasets are available offline, so KV values are drawn
from the distributions the benchmark configurations describe and laid out
exactly as the reference's connector sees vLLM 0.23 pages: one page holds
``[2 (K/V), layers, block_tokens, kv_heads, head_dim]`` BF16 values
(vllm_v1_compressed_offload.py:874-886, 1355-1357), flattened.

Layer-bound profile: the reference's measured Qwen2.5-1.5B profile puts
layers {0, 1, 2, 5, 19, 20, 21} at REL 1e-5 and the other 21 at 1e-4
(data/qwen2.5-1.5b_mixed_21x1e-4_7x1e-5.json).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

QWEN15B_SENSITIVE_LAYERS = (0, 1, 2, 5, 19, 20, 21)


@dataclass(frozen=True)
class KVShape:
    layers: int
    kv_heads: int
    head_dim: int
    tokens: int
    block_tokens: int = 16

    @property
    def pages(self) -> int:
        return self.tokens // self.block_tokens

    @property
    def page_numel(self) -> int:
        return 2 * self.layers * self.block_tokens * self.kv_heads * self.head_dim

    @property
    def elements_per_layer(self) -> int:
        """Elements of one layer inside a page, per K or V (the `E` of the
        layer-indexed calls: view(2, layers, E))."""
        return self.block_tokens * self.kv_heads * self.head_dim


QWEN25_1P5B_4K = KVShape(layers=28, kv_heads=2, head_dim=128, tokens=4096)
QWEN25_7B_32K = KVShape(layers=28, kv_heads=4, head_dim=128, tokens=32768)
LLAMA3_8B_64K = KVShape(layers=32, kv_heads=8, head_dim=128, tokens=65536)


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def layer_kv(shape: KVShape, layer: int, seed: int, device="cpu",
             tokens: int | None = None):
    """K and V of one layer, each [tokens, kv_heads, head_dim] BF16.

    Per (head, channel) scale sigma ~ LogNormal(0, 0.5); in K, 4 of the 128
    channels of every head are outlier channels scaled x15; values are
    bf16(sigma * z) with z ~ N(0, 1)."""
    tokens = shape.tokens if tokens is None else tokens
    g = _gen(seed * 1000003 + layer, device)
    h, d = shape.kv_heads, shape.head_dim
    out = []
    for kind in range(2):
        sigma = torch.exp(0.5 * torch.randn(h, d, generator=g, device=device))
        if kind == 0:
            for head in range(h):
                idx = torch.randperm(d, generator=g, device=device)[:4]
                sigma[head, idx] *= 15.0
        z = torch.randn(tokens, h, d, generator=g, device=device)
        out.append((z * sigma).to(torch.bfloat16))
    return out[0], out[1]


def paged_kv(shape: KVShape, seed: int = 0, device="cpu",
             tokens: int | None = None) -> torch.Tensor:
    """All layers laid out as vLLM pages: [pages, page_numel] BF16."""
    tokens = shape.tokens if tokens is None else tokens
    pages = tokens // shape.block_tokens
    b, h, d = shape.block_tokens, shape.kv_heads, shape.head_dim
    out = torch.empty(pages, 2, shape.layers, b, h, d, dtype=torch.bfloat16,
                      device=device)
    for layer in range(shape.layers):
        k, v = layer_kv(shape, layer, seed, device, tokens)
        out[:, 0, layer] = k.view(pages, b, h, d)
        out[:, 1, layer] = v.view(pages, b, h, d)
    return out.view(pages, -1)


def rope_kv(shape: KVShape, seed: int = 0, device="cpu",
            tokens: int | None = None) -> torch.Tensor:
    """Qwen2.5-7B-like pages: K has channel pairs rotated by position-dependent
    angles theta_i = 10000^(-2i/head_dim) with 6 outlier channels x20; V is
    N(0, 0.6^2)."""
    tokens = shape.tokens if tokens is None else tokens
    pages = tokens // shape.block_tokens
    b, h, d = shape.block_tokens, shape.kv_heads, shape.head_dim
    out = torch.empty(pages, 2, shape.layers, b, h, d, dtype=torch.bfloat16,
                      device=device)
    pos = torch.arange(tokens, device=device, dtype=torch.float32)
    theta = 10000.0 ** (-2.0 * torch.arange(d // 2, device=device,
                                            dtype=torch.float32) / d)
    ang = pos[:, None] * theta[None, :]
    cos, sin = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    for layer in range(shape.layers):
        g = _gen(seed * 1000003 + layer, device)
        sigma = torch.exp(0.5 * torch.randn(h, d // 2, generator=g, device=device))
        x = torch.randn(tokens, h, d // 2, generator=g, device=device) * sigma
        y = torch.randn(tokens, h, d // 2, generator=g, device=device) * sigma
        k = torch.empty(tokens, h, d, device=device)
        k[..., 0::2] = x * cos - y * sin
        k[..., 1::2] = x * sin + y * cos
        idx = torch.randperm(d, generator=g, device=device)[:6]
        k[..., idx] *= 20.0
        v = 0.6 * torch.randn(tokens, h, d, generator=g, device=device)
        out[:, 0, layer] = k.to(torch.bfloat16).view(pages, b, h, d)
        out[:, 1, layer] = v.to(torch.bfloat16).view(pages, b, h, d)
    return out.view(pages, -1)


def stress_pages(shape: KVShape, seed: int = 0, device="cpu",
                 tokens: int | None = None) -> tuple[torch.Tensor, list[str]]:
    """Llama-3-8B-like stress pages: by seed 10% all-zero pages, 5% constant
    pages, 10% heavy-tailed pages (Student-t nu=2, x50 outliers), the rest
    Gaussian.  Returns (pages, class per page)."""
    tokens = shape.tokens if tokens is None else tokens
    pages = tokens // shape.block_tokens
    g = _gen(seed, device)
    u = torch.rand(pages, generator=g, device=device).cpu()
    classes = []
    out = torch.empty(pages, shape.page_numel, dtype=torch.bfloat16,
                      device=device)
    for p in range(pages):
        r = float(u[p])
        if r < 0.10:
            classes.append("zero")
            out[p].zero_()
        elif r < 0.15:
            classes.append("constant")
            c = torch.randn(1, generator=g, device=device)
            out[p].fill_(float(c))
        elif r < 0.25:
            classes.append("heavy")
            z = torch.randn(shape.page_numel, generator=g, device=device)
            chi = torch.randn(2, shape.page_numel, generator=g, device=device)
            t = z / torch.sqrt((chi * chi).sum(0) / 2.0)
            mask = torch.rand(shape.page_numel, generator=g, device=device) < 1e-3
            t = torch.where(mask, t * 50.0, t)
            out[p] = t.clamp(-3e38, 3e38).to(torch.bfloat16)
        else:
            classes.append("gaussian")
            out[p] = torch.randn(shape.page_numel, generator=g,
                                 device=device).to(torch.bfloat16)
    return out, classes


def mixed_bound_groups(layers: int = 28,
                       sensitive=QWEN15B_SENSITIVE_LAYERS,
                       low: float = 1e-5, high: float = 1e-4):
    """Layer groups in the connector's order (sorted by bound,
    vllm_v1_compressed_offload.py:1312-1317, 1343-1345):
    [(bound, layers), ...]."""
    lo = [l for l in range(layers) if l in sensitive]
    hi = [l for l in range(layers) if l not in sensitive]
    groups = sorted({low: lo, high: hi}.items())
    return [(b, tuple(ls)) for b, ls in groups if ls]


def alternating_bound_groups(layers: int = 32, even: float = 1e-4,
                             odd: float = 1e-5):
    """Per-layer bound alternating even/odd, grouped like the connector."""
    lo = tuple(l for l in range(layers) if l % 2 == 1)
    hi = tuple(l for l in range(layers) if l % 2 == 0)
    return sorted({odd: lo, even: hi}.items())
