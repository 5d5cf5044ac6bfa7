"""Writes the golden fixtures of tests/golden/*.npz.

Each fixture holds seeded inputs (values already rounded to the case's dtype,
stored as float32, which represents bf16/fp16 exactly), the expected output in
float64 and a JSON `meta` string (no pickled objects: np.load with
allow_pickle=False reads them).

The expected output is the float64 oracle (oracle/attention.py,
oracle/attention_grad.py, oracle/paged.py, oracle/kv_cache.py). Before a fixture is written it is checked
against an independent evaluation: for attention,
torch.nn.functional.scaled_dot_product_attention in float64 with an explicit
mask, the library routine the reference's own
parity suite compares with (tests/parity/pytorch/test_attention_parity.py:87-105,
288-337). The reference ships no golden files (its generator recipes are
scripts/validation/generators/attention/sdpa.py:93-141 and efficient.py:276-339);
these fixtures follow the same idea at small sizes. Windows follow the
production convention |i - j| <= W (W+1 keys including self with causal,
attention/sliding_window.py:151-157), not the generator's W-key variant.

Run from the repository root:  python tests/golden/make_golden.py [name ...]
(with names, only those fixtures are rewritten).
"""

from __future__ import annotations

import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import attention as oa  # noqa: E402
from oracle import attention_grad as oag  # noqa: E402
from oracle import kv_cache as ok  # noqa: E402
from oracle import paged as op  # noqa: E402

DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
# Oracle vs torch SDPA, both float64. The tiled paths normalise by l + 1e-6
# (attention/flash.py:312, sliding_window.py:115, chunked.py:169) where SDPA is
# exact; with l >= 1 that moves outputs by <= 1e-6 relative. Paged decode is
# exact in both.
AGREE_TILED = 1e-5
AGREE_EXACT = 1e-9


def rounded(shape, dtype, gen, mult=1.0):
    x = torch.randn(shape, generator=gen, dtype=torch.float32) * mult
    return x.to(DTYPES[dtype]).to(torch.float32).numpy()


def sdpa_rows(q, k, v, scale, keep):
    """softmax(q k^T * scale, masked by keep) v per (b, h); q/k/v (B, H, S, D)."""
    qt, kt, vt = (torch.from_numpy(np.ascontiguousarray(x)).double() for x in (q, k, v))
    out = torch.nn.functional.scaled_dot_product_attention(
        qt, kt, vt, attn_mask=torch.from_numpy(keep), scale=scale)
    return out.numpy()


def window_keep(Sq, Sk, causal, left, right):
    i = np.arange(Sq)[:, None]
    j = np.arange(Sk)[None, :]
    keep = np.ones((Sq, Sk), dtype=bool)
    if causal:
        keep &= j <= i
    if left >= 0:
        keep &= j >= i - left
    if right >= 0:
        keep &= j <= i + right
    return keep


def to_bhsd(x, layout):
    return x if layout == "BHSD" else np.transpose(x, (0, 2, 1, 3))


ONLY = set(sys.argv[1:])  # fixture names to (re)write; empty = all


def save(name, meta, **arrays):
    if ONLY and name not in ONLY:
        return
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, meta=np.array(json.dumps(meta, sort_keys=True)), **arrays)
    print(f"{name}: {', '.join(f'{k}{tuple(v.shape)}' for k, v in arrays.items())}")


def agree(name, a, b, tol=AGREE_TILED):
    err = float(np.nanmax(np.abs(a - b)))
    assert err <= tol, f"{name}: oracle and SDPA disagree by {err}"


def flash_case(name, shape, dtype, layout, causal, seed, scale=None):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (rounded(shape, dtype, g) for _ in range(3))
    D = shape[-1]
    s = 1.0 / math.sqrt(D) if scale is None else scale
    exp = oa.flash_attention(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                             scale=scale, causal=causal, layout=layout)
    Sq = shape[2] if layout == "BHSD" else shape[1]
    keep = window_keep(Sq, Sq, causal, -1, -1)
    ref = sdpa_rows(to_bhsd(q, layout), to_bhsd(k, layout), to_bhsd(v, layout), s, keep)
    agree(name, to_bhsd(exp, layout), ref)
    save(name, {"kind": "flash", "dtype": dtype, "layout": layout, "causal": causal,
                "scale": scale}, q=q, k=k, v=v, expected=exp)


def flash_default_case(name, qshape, kvlen, dtype, layout, seed):
    """Causal flash_attention with Sq != Sk on the reference's default (SDPA)
    route: key j visible to query i iff j <= i + max(0, Sk - Sq)."""
    g = torch.Generator().manual_seed(seed)
    q = rounded(qshape, dtype, g)
    kshape = list(qshape)
    kshape[2 if layout == "BHSD" else 1] = kvlen
    k, v = (rounded(tuple(kshape), dtype, g) for _ in range(2))
    exp = oa.flash_attention_default_route(q.astype(np.float64), k.astype(np.float64),
                                           v.astype(np.float64), causal=True, layout=layout)
    Sq = qshape[2] if layout == "BHSD" else qshape[1]
    keep = np.tril(np.ones((Sq, kvlen), dtype=bool), k=max(0, kvlen - Sq))
    ref = sdpa_rows(to_bhsd(q, layout), to_bhsd(k, layout), to_bhsd(v, layout),
                    1.0 / math.sqrt(qshape[-1]), keep)
    agree(name, to_bhsd(exp, layout), ref, AGREE_EXACT)
    save(name, {"kind": "flash_default", "dtype": dtype, "layout": layout, "causal": True},
         q=q, k=k, v=v, expected=exp)


def grad_case(name, shape, dtype, layout, causal, window, seed):
    """dq, dk, dv (stacked) of sum(out * dout) for flash (window < 0) or sliding
    window attention; checked against torch autograd through float64 SDPA."""
    g = torch.Generator().manual_seed(seed)
    q, k, v, d = (rounded(shape, dtype, g) for _ in range(4))
    D = shape[-1]
    s = 1.0 / math.sqrt(D)
    wl, wr = (window, -1 if causal else window) if window >= 0 else (-1, -1)
    exp = np.stack(oag.attention_grad(*(x.astype(np.float64) for x in (q, k, v, d)), s, causal,
                                      wl, wr, layout=layout))
    ts = [torch.from_numpy(np.ascontiguousarray(to_bhsd(x, layout))).double().requires_grad_(True)
          for x in (q, k, v)]
    Sq = ts[0].shape[2]
    keep = torch.from_numpy(window_keep(Sq, Sq, causal, wl, wr))
    out = torch.nn.functional.scaled_dot_product_attention(*ts, attn_mask=keep, scale=s)
    (out * torch.from_numpy(np.ascontiguousarray(to_bhsd(d, layout))).double()).sum().backward()
    ref = np.stack([t.grad.numpy() for t in ts])
    if layout == "BSHD":
        ref = np.swapaxes(ref, 2, 3)
    agree(name, exp, ref)
    save(name, {"kind": "grad", "dtype": dtype, "layout": layout, "causal": causal,
                "window": window}, q=q, k=k, v=v, dout=d, expected=exp)


def window_case(name, shape, dtype, W, causal, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (rounded(shape, dtype, g) for _ in range(3))
    exp = oa.sliding_window_attention(q.astype(np.float64), k.astype(np.float64),
                                      v.astype(np.float64), W, causal=causal)
    S = shape[1]
    keep = window_keep(S, S, causal, W, -1 if causal else W)
    ref = sdpa_rows(to_bhsd(q, "BSHD"), to_bhsd(k, "BSHD"), to_bhsd(v, "BSHD"),
                    1.0 / math.sqrt(shape[-1]), keep)
    agree(name, to_bhsd(exp, "BSHD"), ref)
    save(name, {"kind": "window", "dtype": dtype, "window": W, "causal": causal},
         q=q, k=k, v=v, expected=exp)


def chunked_case(name, qshape, kvlen, dtype, chunk, causal, seed):
    g = torch.Generator().manual_seed(seed)
    B, Sq, H, D = qshape
    q = rounded(qshape, dtype, g)
    k = rounded((B, kvlen, H, D), dtype, g)
    v = rounded((B, kvlen, H, D), dtype, g)
    exp = oa.chunked_cross_attention(q.astype(np.float64), k.astype(np.float64),
                                     v.astype(np.float64), chunk_size=chunk, causal=causal)
    keep = window_keep(Sq, kvlen, causal, -1, -1)
    ref = sdpa_rows(to_bhsd(q, "BSHD"), to_bhsd(k, "BSHD"), to_bhsd(v, "BSHD"),
                    1.0 / math.sqrt(D), keep)
    # Skv <= chunk takes the exact dense branch (chunked.py:113-114, 172-203)
    agree(name, to_bhsd(exp, "BSHD"), ref, AGREE_EXACT if kvlen <= chunk else AGREE_TILED)
    save(name, {"kind": "chunked", "dtype": dtype, "chunk_size": chunk, "causal": causal},
         q=q, k=k, v=v, expected=exp)


def paged_case(name, lens, tables, num_blocks, bs, H, D, dtype, seed, alibi=False):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    q = rounded((B, 1, H, D), dtype, g)
    kp = rounded((num_blocks, bs, H, D), dtype, g)
    vp = rounded((num_blocks, bs, H, D), dtype, g)
    tables = np.asarray(tables, dtype=np.int32)
    lens = np.asarray(lens, dtype=np.int32)
    slopes = op.get_alibi_slopes(H) if alibi else None
    scale = 1.0 / math.sqrt(D)
    exp = op.paged_attention_decode(q.astype(np.float64), kp.astype(np.float64),
                                    vp.astype(np.float64), tables, lens, scale, bs,
                                    alibi_slopes=slopes)
    # Independent check: gather each sequence's valid tokens, then SDPA with the
    # ALiBi bias slope_h * (pos - ctx) (cache/paged_attention.py:163-178).
    for b in range(B):
        pos = np.arange(int(lens[b]))
        pages = tables[b, pos // bs]
        ok = pages >= 0
        kk = kp[pages[ok], (pos % bs)[ok]].transpose(1, 0, 2)[None].astype(np.float64)
        vv = vp[pages[ok], (pos % bs)[ok]].transpose(1, 0, 2)[None].astype(np.float64)
        qq = q[b:b + 1].transpose(0, 2, 1, 3).astype(np.float64)
        bias = np.zeros((1, H, 1, kk.shape[2]))
        if alibi:
            bias = (slopes[:, None] * (pos[ok] - int(lens[b]))[None, :])[None, :, None, :]
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(qq), torch.from_numpy(kk), torch.from_numpy(vv),
            attn_mask=torch.from_numpy(bias), scale=scale).numpy()
        agree(f"{name}[{b}]", exp[b:b + 1].transpose(0, 2, 1, 3), ref, AGREE_EXACT)
    save(name, {"kind": "paged", "dtype": dtype, "block_size": bs, "alibi": alibi},
         q=q, k_pool=kp, v_pool=vp, block_tables=tables, context_lens=lens, expected=exp)


def paged_prefill_case(name, Sq, lens, tables, num_blocks, bs, H, D, dtype, causal, seed,
                       alibi=False):
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    q = rounded((B, Sq, H, D), dtype, g)
    kp = rounded((num_blocks, bs, H, D), dtype, g)
    vp = rounded((num_blocks, bs, H, D), dtype, g)
    tables = np.asarray(tables, dtype=np.int32)
    lens = np.asarray(lens, dtype=np.int32)
    slopes = op.get_alibi_slopes(H) if alibi else None
    scale = 1.0 / math.sqrt(D)
    exp = op.paged_attention_prefill(q.astype(np.float64), kp.astype(np.float64),
                                     vp.astype(np.float64), tables, lens, scale, bs, causal,
                                     alibi_slopes=slopes)
    # Independent check: the valid tokens of each sequence gathered in order,
    # SDPA with an additive mask = ALiBi slope_h * (kv - q) (paged_attention.py:
    # 266-285), -inf where kv > q under the causal flag (300-309).
    for b in range(B):
        pos = np.arange(int(lens[b]))
        pages = tables[b, pos // bs]
        ok_ = pages >= 0
        pos = pos[ok_]
        kk = kp[pages[ok_], pos % bs].transpose(1, 0, 2)[None].astype(np.float64)
        vv = vp[pages[ok_], pos % bs].transpose(1, 0, 2)[None].astype(np.float64)
        qq = q[b:b + 1].transpose(0, 2, 1, 3).astype(np.float64)
        diff = (pos[None, :] - np.arange(Sq)[:, None]).astype(np.float64)
        mask = np.zeros((1, H, Sq, len(pos)))
        if alibi:
            mask = mask + slopes[None, :, None, None] * diff[None, None]
        if causal:
            mask = np.where(diff[None, None] > 0, -np.inf, mask)
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(qq), torch.from_numpy(kk), torch.from_numpy(vv),
            attn_mask=torch.from_numpy(mask), scale=scale).numpy()
        agree(f"{name}[{b}]", exp[b:b + 1].transpose(0, 2, 1, 3), ref, AGREE_EXACT)
    save(name, {"kind": "paged_prefill", "dtype": dtype, "block_size": bs, "alibi": alibi,
                "causal": causal},
         q=q, k_pool=kp, v_pool=vp, block_tables=tables, context_lens=lens, expected=exp)


def kv_append_case(name, T, starts, counts, tables, num_blocks, bs, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    B = len(starts)
    k = rounded((B, T, H, D), dtype, g)
    v = rounded((B, T, H, D), dtype, g)
    kp = rounded((num_blocks, bs, H, D), dtype, g)
    vp = rounded((num_blocks, bs, H, D), dtype, g)
    tables = np.asarray(tables, dtype=np.int32)
    starts = np.asarray(starts, dtype=np.int32)
    counts = np.asarray(counts, dtype=np.int32)
    ek, ev = kp.copy(), vp.copy()
    ok.kv_append(ek, ev, tables, k, v, starts, counts, bs)
    # Independent check: token by token, position -> (page, slot) directly.
    ik, iv = kp.copy(), vp.copy()
    for b in range(B):
        for t in range(int(counts[b])):
            p = int(starts[b]) + t
            ik[tables[b, p // bs], p % bs] = k[b, t]
            iv[tables[b, p // bs], p % bs] = v[b, t]
    if not (np.array_equal(ek, ik) and np.array_equal(ev, iv)):
        raise SystemExit(f"{name}: oracle append disagrees with the per-token placement")
    save(name, {"kind": "kv_append", "dtype": dtype, "block_size": bs},
         k=k, v=v, k_pool=kp, v_pool=vp, block_tables=tables, start_pos=starts,
         n_tokens=counts, expected=np.stack([ek, ev]))


def main():
    flash_case("flash_causal_f32_bshd", (1, 37, 2, 32), "float32", "BSHD", True, 101)
    flash_case("flash_full_bf16_bhsd", (2, 3, 70, 64), "bfloat16", "BHSD", False, 102)
    flash_case("flash_causal_f16_bshd_d128", (1, 129, 2, 128), "float16", "BSHD", True, 103)
    flash_case("flash_full_f32_negscale", (1, 20, 1, 64), "float32", "BSHD", False, 104, scale=-0.3)
    window_case("window_causal_f32_w7", (1, 100, 2, 64), "float32", 7, True, 105)
    window_case("window_full_bf16_w16", (1, 90, 2, 32), "bfloat16", 16, False, 106)
    chunked_case("chunked_full_f32", (1, 16, 2, 64), 300, "float32", 64, False, 107)
    chunked_case("chunked_causal_bf16", (1, 40, 2, 64), 200, "bfloat16", 64, True, 108)
    # Skv <= chunk_size: the dense branch, top-left causal with more queries than keys
    chunked_case("chunked_dense_causal_f16", (1, 48, 2, 64), 40, "float16", 64, True, 117)
    # causal with Sq != Sk on the default route: decode-style (bottom right) and Sq > Sk
    flash_default_case("flash_default_causal_bf16_bhsd_sq5_sk70", (1, 2, 5, 64), 70, "bfloat16",
                       "BHSD", 118)
    flash_default_case("flash_default_causal_f32_bshd_sq40_sk17", (1, 40, 2, 32), 17, "float32",
                       "BSHD", 119)
    # tests/cache/test_paged_attention.py:164-197 (hand-built tables, page 8 unused)
    paged_case("paged_ref_tables_f32", [16, 32, 48, 25], [[0, -1, -1], [1, 2, -1], [3, 4, 5],
                                                          [6, 7, -1]], 9, 16, 2, 32, "float32", 109)
    paged_case("paged_alibi_f16", [5, 40, 17], [[3, -1, -1], [0, 4, 1], [2, 5, -1]], 6, 16, 4,
               64, "float16", 110, alibi=True)
    # prefill: ragged contexts (longer / shorter than the queries), a missing page
    paged_prefill_case("paged_prefill_alibi_bf16", 24, [40, 13], [[4, -1, 1], [0, 3, -1]], 5,
                       16, 2, 64, "bfloat16", True, 111, alibi=True)
    paged_prefill_case("paged_prefill_full_f32", 12, [30, 20], [[2, 0], [3, 1]], 4, 16, 2, 32,
                       "float32", False, 112)
    # append: starts inside a page, spans over pages, a decode-style single token, nothing
    kv_append_case("kv_append_ragged_bf16", 20, [3, 16, 0], [20, 1, 0],
                   [[5, 0, 7], [2, 6, 1], [3, 4, 8]], 9, 8, 2, 64, "bfloat16", 113)
    # gradients (dq, dk, dv of sum(out * dout)): flash causal / full, sliding window
    grad_case("grad_causal_bf16_bhsd", (1, 2, 50, 64), "bfloat16", "BHSD", True, -1, 114)
    grad_case("grad_full_f16_bshd_d128", (1, 33, 2, 128), "float16", "BSHD", False, -1, 115)
    grad_case("grad_window_f32_w9", (1, 60, 2, 64), "float32", "BSHD", True, 9, 116)


if __name__ == "__main__":
    main()
