"""Seeded synthetic workloads of the five BASELINE configurations and of the
paged prefill / KV append rows, and the algorithmic FLOP / byte counts used
for throughput and roofline figures.

Inputs are drawn N(0, 1) in float32 from one torch.Generator seeded with 42
(the reference benchmarks' seed, benchmarks/config.py:29) in the order q, k, v
and cast once, so the GPU kernels and the CPU oracle see identical values.
The paged-decode workload draws its integers first (context lengths, then the
page permutation) because the pool size depends on them.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional

import torch

SEED = 42

# name -> shape parameters; the first is the reference's CPU-runnable case.
CONFIGS: Dict[str, dict] = {
    "flash_fp32_bshd": dict(kind="flash", dtype=torch.float32, layout="BSHD",
                            B=2, S=1024, H=12, D=64, causal=True),
    "flash_bf16_bhsd": dict(kind="flash", dtype=torch.bfloat16, layout="BHSD",
                            B=4, S=4096, H=32, D=128, causal=True),
    "window_bf16_bshd": dict(kind="window", dtype=torch.bfloat16, layout="BSHD",
                             B=2, S=8192, H=32, D=128, causal=True, window=4096),
    "paged_decode_fp16": dict(kind="paged", dtype=torch.float16, B=64, H=32, D=128,
                              ctx_lo=512, ctx_hi=8192, block_size=16),
    # The same decode with grouped-query heads: 32 query heads over 8 K/V heads.
    "paged_decode_gqa_fp16": dict(kind="paged", dtype=torch.float16, B=64, H=32, H_kv=8,
                                  D=128, ctx_lo=512, ctx_hi=8192, block_size=16),
    "chunked_bf16": dict(kind="chunked", dtype=torch.bfloat16, B=1, H=16, D=64,
                         Sq=512, Skv=65536, chunk_size=1024, causal=False),
    # Prompt processing over a paged cache: the headline shape (4 x 4096 tokens,
    # 32 heads of 128, causal) with its K/V in 16-token pages of a permuted pool,
    # and the append that writes those prompts into the pages.
    "paged_prefill_bf16": dict(kind="paged_prefill", dtype=torch.bfloat16, B=4, S=4096, H=32,
                               D=128, block_size=16, causal=True),
    "kv_append_bf16": dict(kind="append", dtype=torch.bfloat16, B=4, S=4096, H=32, D=128,
                           block_size=16),
}


@dataclass
class PagedInputs:
    q: torch.Tensor             # (B, 1, H, D)
    k_pool: torch.Tensor        # (N, bs, H, D)
    v_pool: torch.Tensor
    block_tables: torch.Tensor  # int32 (B, max_blocks), -1 padded
    context_lens: torch.Tensor  # int32 (B,)
    block_size: int


def _randn(gen: torch.Generator, shape, device) -> torch.Tensor:
    return torch.randn(shape, generator=gen, dtype=torch.float32, device=device)


def qkv_shapes(cfg: dict):
    if cfg["kind"] == "chunked":
        B, H, D = cfg["B"], cfg["H"], cfg["D"]
        return (B, cfg["Sq"], H, D), (B, cfg["Skv"], H, D)
    B, S, H, D = cfg["B"], cfg["S"], cfg["H"], cfg["D"]
    shape = (B, H, S, D) if cfg.get("layout") == "BHSD" else (B, S, H, D)
    return shape, shape


def make_qkv(cfg: dict, device="cpu", seed: int = SEED, scale_inputs: float = 1.0):
    """q, k, v of a dense-attention config, drawn on ``device`` and cast."""
    gen = torch.Generator(device=device).manual_seed(seed)
    qs, kvs = qkv_shapes(cfg)
    q = _randn(gen, qs, device) * scale_inputs
    k = _randn(gen, kvs, device) * scale_inputs
    v = _randn(gen, kvs, device)
    dt = cfg["dtype"]
    return q.to(dt), k.to(dt), v.to(dt)


def make_paged(cfg: dict, device="cpu", seed: int = SEED) -> PagedInputs:
    """Paged-decode inputs: ctx ~ U{lo..hi}, pages = a random permutation of the
    pool cut consecutively in sequence order, -1 padded tables."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    B, H, D, bs = cfg["B"], cfg["H"], cfg["D"], cfg["block_size"]
    H_kv = cfg.get("H_kv", H)
    ctx = torch.randint(cfg["ctx_lo"], cfg["ctx_hi"] + 1, (B,), generator=gen, dtype=torch.int64)
    pages = (ctx + bs - 1) // bs
    n_pages = int(pages.sum())
    perm = torch.randperm(n_pages, generator=gen)
    width = int(pages.max())
    tables = torch.full((B, width), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(pages[b])
        tables[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    dgen = gen if device == "cpu" else torch.Generator(device=device).manual_seed(seed + 1)
    dt = cfg["dtype"]
    q = _randn(dgen, (B, 1, H, D), device).to(dt)
    k_pool = torch.empty((n_pages, bs, H_kv, D), dtype=dt, device=device)
    v_pool = torch.empty((n_pages, bs, H_kv, D), dtype=dt, device=device)
    step = 1024
    for pool in (k_pool, v_pool):
        for s in range(0, n_pages, step):
            e = min(s + step, n_pages)
            pool[s:e] = _randn(dgen, (e - s, bs, H_kv, D), device).to(dt)
    return PagedInputs(q, k_pool, v_pool, tables.to(device), ctx.to(torch.int32).to(device), bs)


@dataclass
class PrefillInputs:
    q: torch.Tensor             # (B, S, H, D)
    k_pool: torch.Tensor        # (B * S / bs, bs, H, D)
    v_pool: torch.Tensor
    block_tables: torch.Tensor  # int32 (B, S / bs), a permutation of the pool
    context_lens: torch.Tensor  # int32 (B,) = S
    block_size: int


def _permuted_tables(gen: torch.Generator, B: int, pages: int) -> torch.Tensor:
    return torch.randperm(B * pages, generator=gen).to(torch.int32).reshape(B, pages)


def make_paged_prefill(cfg: dict, device="cpu", seed: int = SEED) -> PrefillInputs:
    """Prefill inputs: every sequence's context is its own S-token prompt, stored
    in S / bs pages drawn from a random permutation of the pool."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    B, S, H, D, bs = cfg["B"], cfg["S"], cfg["H"], cfg["D"], cfg["block_size"]
    pages = (S + bs - 1) // bs
    tables = _permuted_tables(gen, B, pages)
    dgen = gen if device == "cpu" else torch.Generator(device=device).manual_seed(seed + 1)
    dt = cfg["dtype"]
    q = _randn(dgen, (B, S, H, D), device).to(dt)
    k_pool = _randn(dgen, (B * pages, bs, H, D), device).to(dt)
    v_pool = _randn(dgen, (B * pages, bs, H, D), device).to(dt)
    ctx = torch.full((B,), S, dtype=torch.int32)
    return PrefillInputs(q, k_pool, v_pool, tables.to(device), ctx.to(device), bs)


@dataclass
class AppendInputs:
    k: torch.Tensor             # (B, S, H, D) new tokens
    v: torch.Tensor
    k_pool: torch.Tensor        # (B * S / bs, bs, H, D), written in place
    v_pool: torch.Tensor
    block_tables: torch.Tensor  # int32 (B, S / bs), a permutation of the pool
    start_pos: torch.Tensor     # int32 (B,) zeros


def make_append(cfg: dict, device="cpu", seed: int = SEED) -> AppendInputs:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    B, S, H, D, bs = cfg["B"], cfg["S"], cfg["H"], cfg["D"], cfg["block_size"]
    pages = (S + bs - 1) // bs
    tables = _permuted_tables(gen, B, pages)
    dgen = gen if device == "cpu" else torch.Generator(device=device).manual_seed(seed + 1)
    dt = cfg["dtype"]
    k = _randn(dgen, (B, S, H, D), device).to(dt)
    v = _randn(dgen, (B, S, H, D), device).to(dt)
    k_pool = torch.zeros((B * pages, bs, H, D), dtype=dt, device=device)
    v_pool = torch.zeros_like(k_pool)
    return AppendInputs(k, v, k_pool, v_pool, tables.to(device),
                        torch.zeros(B, dtype=torch.int32, device=device))


# ---- algorithmic work -------------------------------------------------------

def flash_flops(B: int, H: int, S: int, D: int, causal: bool) -> float:
    """4*B*H*S^2*D, halved for causal (the S^2/2 convention of FlashAttention
    papers and of the reference's derived figures)."""
    f = 4.0 * B * H * S * S * D
    return f / 2 if causal else f


def flash_bwd_flops(B: int, H: int, S: int, D: int, causal: bool) -> float:
    """2.5x the forward: the five S^2*D products of the gradient (S = QK^T
    recomputed, dP = dO V^T, dV, dQ, dK), FlashAttention-2's convention."""
    return 2.5 * flash_flops(B, H, S, D, causal)


def window_flops(B: int, H: int, S: int, D: int, window: int) -> float:
    """4*D per (query, visible key) pair; query i sees min(i, W) + 1 keys."""
    pairs = sum(min(i, window) + 1 for i in range(S))
    return 4.0 * B * H * D * pairs


def chunked_flops(B: int, H: int, Sq: int, Skv: int, D: int) -> float:
    return 4.0 * B * H * Sq * Skv * D


def paged_bytes(ctx: torch.Tensor, H: int, D: int, elem_bytes: int, max_blocks: int,
                H_kv: Optional[int] = None) -> float:
    """Valid K+V bytes (each K/V head once) + q + o + block tables + context
    lengths (no padding)."""
    B = int(ctx.numel())
    kv = 2.0 * float(ctx.to(torch.int64).sum()) * (H if H_kv is None else H_kv) * D * elem_bytes
    qo = 2.0 * B * H * D * elem_bytes
    return kv + qo + B * max_blocks * 4 + B * 4


def append_bytes(B: int, T: int, H: int, D: int, elem_bytes: int, max_blocks: int) -> float:
    """K and V rows read once and written once, + tables, starts and counts."""
    return 4.0 * B * T * H * D * elem_bytes + B * max_blocks * 4 + 2 * B * 4


def config_work(name: str, paged: Optional[PagedInputs] = None) -> float:
    cfg = CONFIGS[name]
    if cfg["kind"] in ("flash", "paged_prefill"):
        # prefill with context == prompt is the causal square of flash
        return flash_flops(cfg["B"], cfg["H"], cfg["S"], cfg["D"], cfg.get("causal", True))
    if cfg["kind"] == "append":
        pages = (cfg["S"] + cfg["block_size"] - 1) // cfg["block_size"]
        return append_bytes(cfg["B"], cfg["S"], cfg["H"], cfg["D"],
                            torch.finfo(cfg["dtype"]).bits // 8, pages)
    if cfg["kind"] == "window":
        return window_flops(cfg["B"], cfg["H"], cfg["S"], cfg["D"], cfg["window"])
    if cfg["kind"] == "chunked":
        return chunked_flops(cfg["B"], cfg["H"], cfg["Sq"], cfg["Skv"], cfg["D"])
    assert paged is not None
    return paged_bytes(paged.context_lens.cpu(), cfg["H"], cfg["D"],
                       torch.finfo(cfg["dtype"]).bits // 8, paged.block_tables.shape[1],
                       cfg.get("H_kv"))


def default_scale(D: int) -> float:
    return 1.0 / math.sqrt(D)
