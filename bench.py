"""Benchmark of the attention hot path on one MI355X.

A step is one forward pass of the headline workload, flash_attention bf16
BHSD B=4 H=32 S=4096 D=128 causal (the configuration the metric is quoted
on). The same run also times paged-KV decode fp16 (64 sequences, H=32, D=128,
context ~ U{512..8192}, 16-token pages) under "paged_decode", the same decode
with 32 query heads over 8 K/V heads (enable_gqa) under "paged_decode_gqa", paged prefill of
the headline shape over 16-token pages under "paged_prefill", the KV append
that writes those prompts into pages under "kv_append", and fused RoPE + flash
attention at the headline shape (BSHD) under "rope_attention", the backward pass of the
headline attention (dQ, dK, dV from the saved output and row log-sum-exp)
under "flash_backward", and the sliding-window (config 3) and chunked
cross-attention (config 5) workloads under "sliding_window" and "chunked_cross".
Inputs are synthetic (seeded N(0,1)) and resident in HBM before timing.

BASELINE config 1 (flash_attention fp32 BSHD B=2 S=1024 H=12 D=64 causal, the
reference's CPU-runnable case) is timed under "flash_fp32" against the fp32
matrix peak, next to the oracle's restatement of the reference's Python tiled
path (32x32 blocks) on host cores.

Prints ONE JSON line. Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]

`--only flash|fp32|window|chunked|paged|gqa|prefill|append|rope|bwd|dropout|d256|copy` runs a single leg
(no CPU baseline) for profiler passes; `copy` streams a 1 GiB float32 buffer through an elementwise kernel,
the known-size reference for scaling the HBM byte counters. The HBM traffic
per launch measured by those passes (rocprofv3 FETCH_SIZE / WRITE_SIZE) is read
from profiles/hbm_traffic.json when present.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "mlx-primitives_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

import workloads as wl  # noqa: E402

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3     # MI355X fp32 matrix (MFMA)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
TRAFFIC_FILE = os.path.join(REPO, "profiles", "hbm_traffic.json")
FLASH_KERNEL = "fa_fwd16_kernel<128,128,8,bf16>"
FP32_KERNEL = "fa_fwd32_kernel<64,64,4>"
WINDOW_KERNEL = "fa_fwd16_kernel<128,128,8,bf16>"
CHUNKED_KERNELS = "fa_fwd16_kernel<64,128,8,bf16> (split-KV) + fa_split_merge_kernel"
PAGED_KERNELS = "paged_decode_part_kernel + paged_decode_merge_kernel"
GQA_KERNELS = "paged_decode_gqa_kernel + paged_decode_merge_kernel"
PREFILL_KERNEL = "fa_fwd16_kernel<128,128,8,bf16,paged>"
APPEND_KERNEL = "kv_append_kernel (+ the 12-byte fill that clears the error words)"
BWD_KERNELS = "fa_bwd_dq_kernel<128,bf16> (+ Dvec) + fa_bwd_dkdv_fused_kernel<bf16>"
DROPOUT_P = 0.1
DROPOUT_KERNEL = "fa_fwd16_drop_kernel<128,128,8,bf16>"
DROPOUT_BWD_KERNELS = ("stored dS: fa_bwd_dvec_kernel + fa_bwd_dkdv_fused_kernel<bf16,drop,ds> "
                       "+ fa_bwd_dq_ds_kernel<128,bf16>")


def measured_traffic(key: str):
    """HBM bytes per launch recorded by the counter passes, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)[key]["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def compact(obj, digits: int = 4):
    """The result with every float rounded to `digits` significant digits
    (timings and rates carry no more than that), so the one JSON line stays a
    few KB long."""
    if isinstance(obj, float):
        return float(f"{obj:.{digits}g}")
    if isinstance(obj, dict):
        return {k: compact(v, digits) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return [compact(v, digits) for v in obj]
    return obj


# Untimed seconds of the workload run before the warmup steps of each leg.
SETTLE_S = 0.3


def time_steps(fn, steps: int, warmup: int, settle_s: float = SETTLE_S):
    """Settle, warmup, then `steps` timed calls; returns (wall ms/step, mean,
    min and median event ms/call).

    The GPU's clocks take ~0.1-0.2 s of sustained load to reach their steady
    state, longer than a few warmup steps of a sub-millisecond kernel, so the
    leg first runs the same call untimed for settle_s seconds; the timed
    region is still exactly `steps` calls. Events are recorded on torch's
    current stream, the stream the kernels are launched on, around every
    call."""
    t_end = time.perf_counter() + settle_s
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ev = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
    return wall_ms, sum(ev) / len(ev), ev[0], ev[len(ev) // 2]


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        n = [d.get("num_threads", 1) for d in threadpool_info() if d.get("user_api") == "blas"]
        if n:
            return int(max(n))
    except Exception:
        pass
    return len(os.sched_getaffinity(0))


def cpu_baseline_flash(cfg: dict, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       budget_s: float) -> dict:
    """The oracle's restatement of the reference's BHSD branch (dense masked
    softmax, flash.py:172-192) in float32 on host cores, over whole heads of the
    same workload until ~budget_s of CPU work."""
    import numpy as np

    from oracle import attention as oa

    B, H, S, D = q.shape
    scale = wl.default_scale(D)
    heads_done, t_total = 0, 0.0
    order = [(b, h) for b in range(B) for h in range(H)]
    for b, h in order:
        qs, ks, vs = (x[b:b + 1, h:h + 1].float().cpu().numpy() for x in (q, k, v))
        t0 = time.perf_counter()
        oa.dense_attention_bhsd(qs, ks, vs, scale, True)
        t_total += time.perf_counter() - t0
        heads_done += 1
        if t_total >= budget_s:
            break
    flops = wl.flash_flops(1, heads_done, S, D, True)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": blas_threads(),
            "kind": "port",
            "sample": f"{heads_done} of {B * H} (b,h) pairs, "
                      f"oracle dense BHSD branch (f32 numpy), {t_total:.1f} s"}


def cpu_baseline_tiled(cfg: dict, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       budget_s: float) -> dict:
    """The oracle's restatement of the reference's Python tiled path
    (_tiled_flash_attention, flash.py:257-316: 32x32 blocks, online softmax
    merge, o / (l + 1e-6)) (f32 numpy) over the whole config-1 workload,
    repeated until ~budget_s of CPU work."""
    from oracle import attention as oa

    B, S, H, D = q.shape
    scale = wl.default_scale(D)
    qs, ks, vs = (x.float().cpu().numpy() for x in (q, k, v))
    t_total, runs = 0.0, 0
    while t_total < budget_s:
        t0 = time.perf_counter()
        oa.tiled_flash_attention(qs, ks, vs, scale, True, 32, 32)
        t_total += time.perf_counter() - t0
        runs += 1
    flops = runs * wl.flash_flops(B, H, S, D, True)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": blas_threads(),
            "kind": "port",
            "sample": f"the whole workload {runs} times, oracle tiled path (32x32 blocks, "
                      f"flash.py:257-316) (f32 numpy), {t_total:.1f} s"}


def cpu_baseline_window(cfg: dict, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        budget_s: float) -> dict:
    """The oracle's restatement of the reference's tiled window path
    (_tiled_sliding_window_attention, sliding_window.py:363-511: 32-query
    blocks, KV from q0 - W in 32-key steps) (f32 numpy), whole (batch,
    head) slices of the config-3 workload until ~budget_s of CPU work."""
    from oracle import attention as oa

    B, S, H, D = q.shape
    W = cfg["window"]
    scale = wl.default_scale(D)
    t_total, done = 0.0, 0
    for b in range(B):
        for h in range(H):
            qs, ks, vs = (x[b:b + 1, :, h:h + 1].float().cpu().numpy() for x in (q, k, v))
            t0 = time.perf_counter()
            oa.tiled_sliding_window_attention(qs, ks, vs, W, scale, True, block_q=32)
            t_total += time.perf_counter() - t0
            done += 1
            if t_total >= budget_s:
                break
        if t_total >= budget_s:
            break
    flops = wl.window_flops(1, done, S, D, W)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": blas_threads(),
            "kind": "port",
            "sample": f"{done} of {B * H} (b,h) slices, oracle tiled "
                      f"window path (sliding_window.py:363-511) (f32 numpy), {t_total:.1f} s"}


def cpu_baseline_chunked(cfg: dict, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         budget_s: float) -> dict:
    """The oracle's restatement of the reference's chunk loop
    (_chunked_cross_attention_impl, chunked.py:129-169, chunk 1024) in float32
    numpy, whole heads of the config-5 workload until ~budget_s of CPU work."""
    from oracle import attention as oa

    B, Sq, H, D = q.shape
    Skv = k.shape[1]
    scale = wl.default_scale(D)
    t_total, done = 0.0, 0
    for b in range(B):
        for h in range(H):
            qs, ks, vs = (x[b:b + 1, :, h:h + 1].float().cpu().numpy() for x in (q, k, v))
            t0 = time.perf_counter()
            oa.chunked_cross_attention_impl(qs, ks, vs, cfg["chunk_size"], scale, False)
            t_total += time.perf_counter() - t0
            done += 1
            if t_total >= budget_s:
                break
        if t_total >= budget_s:
            break
    flops = wl.chunked_flops(1, done, Sq, Skv, D)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": blas_threads(),
            "kind": "port",
            "sample": f"{done} of {B * H} (b,h) slices, oracle chunk "
                      f"loop (chunked.py:129-169, chunk 1024) (f32 numpy), {t_total:.1f} s"}


def cpu_baseline_paged(inp, cfg: dict, budget_s: float) -> dict:
    """The oracle's paged decode (gather + dense masked softmax,
    paged_attention.py:108-208) in float32 over whole sequences."""
    from oracle import paged as op

    lens = inp.context_lens.cpu()
    tables = inp.block_tables.cpu().numpy()
    t_total, nbytes, done = 0.0, 0.0, 0
    for b in range(lens.numel()):
        row = tables[b:b + 1]
        used = row[row >= 0]
        kp = inp.k_pool[torch.as_tensor(used, device=inp.k_pool.device).long()].float().cpu().numpy()
        vp = inp.v_pool[torch.as_tensor(used, device=inp.v_pool.device).long()].float().cpu().numpy()
        local = row.copy()
        local[row >= 0] = range(len(used))
        q = inp.q[b:b + 1].float().cpu().numpy()
        t0 = time.perf_counter()
        op.paged_attention_decode(q, kp, vp, local, lens[b:b + 1].numpy(),
                                  wl.default_scale(cfg["D"]), inp.block_size)
        t_total += time.perf_counter() - t0
        nbytes += wl.paged_bytes(lens[b:b + 1], cfg["H"], cfg["D"], 2, row.shape[1])
        done += 1
        if t_total >= budget_s:
            break
    return {"value": nbytes / t_total / 1e9, "unit": "GB/s", "cores": blas_threads(),
            "kind": "port",
            "sample": f"{done} of {lens.numel()} sequences, oracle paged "
                      f"decode (f32 numpy), {t_total:.1f} s"}


def cpu_baseline_prefill(inp, cfg: dict, budget_s: float) -> dict:
    """The oracle's paged prefill (gather + dense masked softmax,
    paged_attention.py:211-320) in float32, one whole sequence at a time."""
    from oracle import paged as op

    B = inp.q.shape[0]
    per_seq = wl.flash_flops(1, cfg["H"], cfg["S"], cfg["D"], True)
    t_total, done = 0.0, 0
    for b in range(B):
        row = inp.block_tables[b:b + 1]
        kp = inp.k_pool[row[0].long()].float().cpu().numpy()
        vp = inp.v_pool[row[0].long()].float().cpu().numpy()
        local = torch.arange(row.shape[1], dtype=torch.int32)[None].numpy()
        q = inp.q[b:b + 1].float().cpu().numpy()
        t0 = time.perf_counter()
        op.paged_attention_prefill(q, kp, vp, local, inp.context_lens[b:b + 1].cpu().numpy(),
                                   wl.default_scale(cfg["D"]), inp.block_size, True)
        t_total += time.perf_counter() - t0
        done += 1
        if t_total >= budget_s:
            break
    return {"value": done * per_seq / t_total / 1e12, "unit": "TFLOP/s", "cores": blas_threads(),
            "kind": "port",
            "sample": f"{done} of {B} sequences, oracle paged prefill in "
                      f"float32 numpy, {t_total:.1f} s"}


def cpu_baseline_append(inp, cfg: dict, budget_s: float) -> dict:
    """The oracle's KVCache._store_kv page-chunk loop (kv_cache.py:219-264) on
    host arrays, whole sequences, repeated until about budget_s / 4 seconds."""
    from oracle import kv_cache as ok

    B, T, H, D = inp.k.shape
    k = inp.k.view(torch.int16).cpu().numpy(); v = inp.v.view(torch.int16).cpu().numpy()
    kp = torch.zeros(inp.k_pool.shape, dtype=torch.int16).numpy(); vp = kp.copy()
    tables = inp.block_tables.cpu().numpy()
    per_seq = 4.0 * T * H * D * 2
    t_total, done = 0.0, 0
    while t_total < budget_s / 4:
        b = done % B
        t0 = time.perf_counter()
        ok.store_kv(kp, vp, tables[b], k[b], v[b], 0, cfg["block_size"])
        t_total += time.perf_counter() - t0
        done += 1
    return {"value": done * per_seq / t_total / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{done} sequence appends of {T} tokens (the workload's sequences in turn), "
                      f"oracle page-chunk loop in numpy, {t_total:.1f} s"}


def cpu_baseline_bwd(cfg: dict, q, k, v, dout, budget_s: float) -> dict:
    """The oracle's closed-form attention gradient (oracle/attention_grad.py)
    (f32 numpy) on host cores, whole heads of the same workload until
    ~budget_s of CPU work."""
    from oracle import attention_grad as oag

    B, H, S, D = q.shape
    scale = wl.default_scale(D)
    t_total, done = 0.0, 0
    for b in range(B):
        for h in range(H):
            xs = [x[b:b + 1, h:h + 1].float().cpu().numpy() for x in (q, k, v, dout)]
            t0 = time.perf_counter()
            oag.attention_grad(*xs, scale, True, layout="BHSD")
            t_total += time.perf_counter() - t0
            done += 1
            if t_total >= budget_s:
                break
        if t_total >= budget_s:
            break
    flops = wl.flash_bwd_flops(1, done, S, D, True)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": blas_threads(),
            "kind": "port",
            "sample": f"{done} of {B * H} (b,h) pairs, oracle "
                      f"closed-form gradient (f32 numpy), {t_total:.1f} s"}


def bwd_step(dev):
    """dQ, dK, dV of the headline attention: the forward (with its row
    log-sum-exp) runs once; a step is the backward alone."""
    from mlx_primitives.attention import flash_attention

    cfg = wl.CONFIGS["flash_bf16_bhsd"]
    q, k, v = (x.requires_grad_(True) for x in wl.make_qkv(cfg, device=dev))
    dout = wl.make_qkv(cfg, device=dev, seed=wl.SEED + 1)[0]
    out = flash_attention(q, k, v, causal=True, layout="BHSD")
    fn = lambda: torch.autograd.grad(out, (q, k, v), dout, retain_graph=True)
    return (q, k, v, dout), fn


def dropout_steps(dev, p: float):
    """The headline attention with dropout_p = p: a no-grad forward step and
    a backward step (the forward with its row log-sum-exp runs once). The
    BHSD tensors are passed as their BSHD views (the API applies dropout to
    BSHD); the kernels see the same strides either way."""
    from mlx_primitives.attention import flash_attention

    cfg = wl.CONFIGS["flash_bf16_bhsd"]
    q, k, v = (x.requires_grad_(True) for x in wl.make_qkv(cfg, device=dev))
    dout = wl.make_qkv(cfg, device=dev, seed=wl.SEED + 1)[0]
    qs, ks, vs, ds = (x.transpose(1, 2) for x in (q, k, v, dout))
    qn, kn, vn = (x.detach() for x in (qs, ks, vs))
    fwd = lambda: flash_attention(qn, kn, vn, causal=True, dropout_p=p)
    out = flash_attention(qs, ks, vs, causal=True, dropout_p=p)
    bwd = lambda: torch.autograd.grad(out, (q, k, v), ds, retain_graph=True)
    return fwd, bwd


D256_SHAPE = (2, 16, 4096, 256)  # (B, H, S, D), bf16 BHSD causal


def d256_step(dev):
    """flash_attention at head dim 256 (bf16 BHSD causal, D256_SHAPE): the
    D = 256 kernel. Returns (step, FLOP per step)."""
    from mlx_primitives.attention import flash_attention

    B, H, S, D = D256_SHAPE
    g = torch.Generator(device=dev).manual_seed(wl.SEED)
    q, k, v = (torch.randn(D256_SHAPE, generator=g, device=dev).to(torch.bfloat16)
               for _ in range(3))
    return (lambda: flash_attention(q, k, v, causal=True, layout="BHSD"),
            wl.flash_flops(B, H, S, D, True))


def cpu_baseline_dropout(cfg: dict, q, k, v, p: float, budget_s: float) -> dict:
    """The dropout oracle (oracle/dropout.py: keep mask from the hash, dense
    masked softmax) (f32 numpy) on host cores, whole heads of the same
    workload until ~budget_s of CPU work."""
    from oracle import dropout as od

    B, H, S, D = q.shape
    scale = wl.default_scale(D)
    t_total, done = 0.0, 0
    for b in range(B):
        for h in range(H):
            xs = [x[b:b + 1, h:h + 1].float().cpu().numpy() for x in (q, k, v)]
            t0 = time.perf_counter()
            od.attention_dropout(*xs, scale, True, p, seed=12345 + done, layout="BHSD")
            t_total += time.perf_counter() - t0
            done += 1
            if t_total >= budget_s:
                break
        if t_total >= budget_s:
            break
    flops = wl.flash_flops(1, done, S, D, True)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": blas_threads(),
            "kind": "port",
            "sample": f"{done} of {B * H} (b,h) pairs, oracle "
                      f"dropout forward (hash mask, dense softmax) (f32 numpy), "
                      f"{t_total:.1f} s"}


def prefill_step(dev):
    from mlx_primitives.cache import paged_attention

    inp = wl.make_paged_prefill(wl.CONFIGS["paged_prefill_bf16"], device=dev)
    fn = lambda: paged_attention(inp.q, inp.k_pool, inp.v_pool, inp.block_tables,
                                 inp.context_lens, block_size=inp.block_size, causal=True)
    return inp, fn


def append_step(dev):
    """store_kv over the whole workload, as a serving step calls it: no wait
    for the error words, which go to a buffer the caller keeps (the call
    allocates nothing)."""
    from mlx_primitives.cache import store_kv

    inp = wl.make_append(wl.CONFIGS["kv_append_bf16"], device=dev)
    B, T, H, D = inp.k.shape
    errors = torch.zeros(3, dtype=torch.int32, device=dev)
    counts = torch.full((B,), T, dtype=torch.int32, device=dev)
    fn = lambda: store_kv(inp.k_pool, inp.v_pool, inp.block_tables, inp.k, inp.v, inp.start_pos,
                          counts, check=False, errors=errors)
    return inp, fn, errors


def rope_attention_step(dev):
    """fused_rope_attention at the headline shape in BSHD, caches precomputed."""
    from mlx_primitives.kernels import fused_rope_attention, precompute_rope_cache

    cfg = wl.CONFIGS["flash_bf16_bhsd"]
    B, S, H, D = cfg["B"], cfg["S"], cfg["H"], cfg["D"]
    q, k, v = wl.make_qkv(dict(cfg, layout="BSHD"), device=dev)
    cos, sin = precompute_rope_cache(S, D, dtype=q.dtype, device=dev)
    fn = lambda: fused_rope_attention(q, k, v, cos_cache=cos, sin_cache=sin, causal=True)
    return fn


def fp32_step(dev):
    """flash_attention fp32 BSHD (2, 1024, 12, 64), causal."""
    from mlx_primitives.attention import flash_attention

    q, k, v = wl.make_qkv(wl.CONFIGS["flash_fp32_bshd"], device=dev)
    return (q, k, v), lambda: flash_attention(q, k, v, causal=True)


def window_step(dev):
    """sliding_window_attention bf16 BSHD, W = 4096, causal."""
    from mlx_primitives.attention import sliding_window_attention

    cfg = wl.CONFIGS["window_bf16_bshd"]
    q, k, v = wl.make_qkv(cfg, device=dev)
    return (q, k, v), lambda: sliding_window_attention(q, k, v, cfg["window"], causal=True)


def chunked_step(dev):
    """chunked_cross_attention bf16, 512 queries x 65536 keys."""
    from mlx_primitives.attention import chunked_cross_attention

    cfg = wl.CONFIGS["chunked_bf16"]
    q, k, v = wl.make_qkv(cfg, device=dev)
    return (q, k, v), lambda: chunked_cross_attention(q, k, v, chunk_size=cfg["chunk_size"])


def run_one_leg(args) -> int:
    """One leg for a profiler pass: warmup + steps calls, timing on stderr/stdout."""
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.only == "copy":
        n = 1 << 28  # 2^28 float32 = 1 GiB read + 1 GiB written per launch
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        fn = lambda: torch.mul(src, 1.0, out=dst)
        work, unit = 2.0 * n * 4, "bytes"
    elif args.only == "flash":
        from mlx_primitives.attention import flash_attention

        cfg = wl.CONFIGS["flash_bf16_bhsd"]
        q, k, v = wl.make_qkv(cfg, device=dev)
        fn = lambda: flash_attention(q, k, v, causal=True, layout="BHSD")
        work, unit = wl.config_work("flash_bf16_bhsd"), "flop"
    elif args.only == "fp32":
        fn = fp32_step(dev)[1]
        work, unit = wl.config_work("flash_fp32_bshd"), "flop"
    elif args.only == "window":
        fn = window_step(dev)[1]
        work, unit = wl.config_work("window_bf16_bshd"), "flop"
    elif args.only == "chunked":
        fn = chunked_step(dev)[1]
        work, unit = wl.config_work("chunked_bf16"), "flop"
    elif args.only == "prefill":
        _, fn = prefill_step(dev)
        work, unit = wl.config_work("paged_prefill_bf16"), "flop"
    elif args.only == "append":
        _, fn, _ = append_step(dev)
        work, unit = wl.config_work("kv_append_bf16"), "bytes"
    elif args.only == "rope":
        fn = rope_attention_step(dev)
        work, unit = wl.config_work("flash_bf16_bhsd"), "flop"
    elif args.only == "bwd":
        _, fn = bwd_step(dev)
        work, unit = 2.5 * wl.config_work("flash_bf16_bhsd"), "flop"
    elif args.only == "dropout":
        d_fwd, d_bwd = dropout_steps(dev, DROPOUT_P)
        fn = lambda: (d_fwd(), d_bwd())
        work, unit = 3.5 * wl.config_work("flash_bf16_bhsd"), "flop"
    elif args.only == "d256":
        fn, work = d256_step(dev)
        unit = "flop"
    else:
        from mlx_primitives.cache import paged_attention

        pname = "paged_decode_gqa_fp16" if args.only == "gqa" else "paged_decode_fp16"
        pin = wl.make_paged(wl.CONFIGS[pname], device=dev)
        fn = lambda: paged_attention(pin.q, pin.k_pool, pin.v_pool, pin.block_tables,
                                     pin.context_lens, block_size=pin.block_size,
                                     enable_gqa=args.only == "gqa")
        work, unit = wl.config_work(pname, pin), "bytes"
    # Counter passes profile every dispatch: no settling phase by default. A
    # kernel-trace pass settles the clocks like the full bench (--settle 0.3);
    # its timed calls are the last `steps` dispatches of each kernel.
    wall_ms, ev_ms, ev_min, ev_med = time_steps(fn, args.steps, args.warmup,
                                                settle_s=args.settle)
    print(json.dumps({"leg": args.only, "steps": args.steps, "warmup": args.warmup,
                      "settle_s": args.settle, "ms_per_call": ev_ms, "median_ms": ev_med,
                      "min_ms": ev_min, "work_per_call": work, "work_unit": unit,
                      "rate": work / (ev_ms * 1e-3) / (1e12 if unit == "flop" else 1e9),
                      "rate_unit": "TFLOP/s" if unit == "flop" else "GB/s"}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU work per baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only",
                    choices=["flash", "fp32", "window", "chunked", "paged", "gqa", "prefill",
                             "append", "rope", "bwd", "dropout", "d256", "copy"],
                    default=None,
                    help="run one leg only (profiler passes); prints that leg's timing")
    ap.add_argument("--settle", type=float, default=0.0,
                    help="--only: seconds of untimed calls before the warmup")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path)", file=sys.stderr)
        return 2
    if args.only is not None:
        return run_one_leg(args)

    from mlx_primitives.attention import flash_attention
    from mlx_primitives.cache import paged_attention

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    # ---- headline: causal flash fwd, bf16 BHSD B=4 H=32 S=4096 D=128 -------------
    name = "flash_bf16_bhsd"
    cfg = wl.CONFIGS[name]
    q, k, v = wl.make_qkv(cfg, device=dev)
    flops = wl.config_work(name)
    step = lambda: flash_attention(q, k, v, causal=True, layout="BHSD")
    log(f"[bench] {name}: warmup {args.warmup}, steps {args.steps}")
    wall_ms, ev_ms, ev_min, ev_med = time_steps(step, args.steps, args.warmup)
    achieved = flops / (ev_ms * 1e-3) / 1e12
    log(f"[bench] {name}: {wall_ms:.3f} ms/step wall, kernel {ev_ms:.3f} ms "
        f"(min {ev_min:.3f}) -> {achieved:.1f} TFLOP/s")

    # ---- paged decode, fp16 --------------------------------------------------------
    pname = "paged_decode_fp16"
    pcfg = wl.CONFIGS[pname]
    pin = wl.make_paged(pcfg, device=dev)
    pbytes = wl.config_work(pname, pin)
    pstep = lambda: paged_attention(pin.q, pin.k_pool, pin.v_pool, pin.block_tables,
                                    pin.context_lens, block_size=pin.block_size)
    log(f"[bench] {pname}: warmup {args.warmup}, steps {args.steps}")
    p_wall, p_ev, p_min, p_med = time_steps(pstep, args.steps, args.warmup)
    p_gbs = pbytes / (p_ev * 1e-3) / 1e9
    log(f"[bench] {pname}: {p_wall:.3f} ms/step wall, kernels {p_ev:.3f} ms -> {p_gbs:.1f} GB/s")

    # ---- paged decode, fp16, grouped-query heads (32 over 8) --------------------------
    gname = "paged_decode_gqa_fp16"
    gcfg = wl.CONFIGS[gname]
    gin = wl.make_paged(gcfg, device=dev)
    gbytes = wl.config_work(gname, gin)
    gstep = lambda: paged_attention(gin.q, gin.k_pool, gin.v_pool, gin.block_tables,
                                    gin.context_lens, block_size=gin.block_size, enable_gqa=True)
    log(f"[bench] {gname}: warmup {args.warmup}, steps {args.steps}")
    g_wall, g_ev, g_min, g_med = time_steps(gstep, args.steps, args.warmup)
    g_gbs = gbytes / (g_ev * 1e-3) / 1e9
    log(f"[bench] {gname}: {g_wall:.3f} ms/step wall, kernels {g_ev:.3f} ms -> {g_gbs:.1f} GB/s "
        f"(distinct K/V bytes)")
    del gin

    # ---- paged prefill, bf16 (prompt processing over pages) ------------------------
    fname = "paged_prefill_bf16"
    finp, fstep = prefill_step(dev)
    fflops = wl.config_work(fname)
    log(f"[bench] {fname}: warmup {args.warmup}, steps {args.steps}")
    f_wall, f_ev, f_min, f_med = time_steps(fstep, args.steps, args.warmup)
    f_tf = fflops / (f_ev * 1e-3) / 1e12
    log(f"[bench] {fname}: {f_wall:.3f} ms/step wall, kernel {f_ev:.3f} ms -> {f_tf:.1f} TFLOP/s")

    # ---- KV append, bf16 (write the prompts into their pages) ------------------------
    aname = "kv_append_bf16"
    ainp, astep, aerr = append_step(dev)
    abytes = wl.config_work(aname)
    log(f"[bench] {aname}: warmup {args.warmup}, steps {args.steps}")
    a_wall, a_ev, a_min, a_med = time_steps(astep, args.steps, args.warmup)
    a_gbs = abytes / (a_ev * 1e-3) / 1e9
    if aerr.tolist() != [0, 0, 0]:
        raise RuntimeError(f"kv append reported errors {aerr.tolist()}")
    log(f"[bench] {aname}: {a_wall:.3f} ms/step wall, kernel {a_ev:.3f} ms -> {a_gbs:.1f} GB/s")
    # Reference point for a read + write stream of the same bytes: the
    # runtime's device-to-device copy of K and V into same-size buffers.
    kdst, vdst = torch.empty_like(ainp.k), torch.empty_like(ainp.v)
    cstep = lambda: (kdst.copy_(ainp.k), vdst.copy_(ainp.v))
    _, c_ev, _, _ = time_steps(cstep, args.steps, args.warmup)
    c_gbs = 4.0 * ainp.k.numel() * ainp.k.element_size() / (c_ev * 1e-3) / 1e9
    del kdst, vdst
    log(f"[bench] {aname}: device-to-device copy of the same bytes {c_gbs:.1f} GB/s")
    # The same append with K rotated to each token's position on the way in
    # (store_kv rope=...): the bytes above plus the cos / sin rows it reads.
    from mlx_primitives.cache import store_kv
    from mlx_primitives.kernels import precompute_rope_cache
    aB, aT, _, aD = ainp.k.shape
    rcos, rsin = precompute_rope_cache(aT, aD, device=dev)
    rerr = torch.zeros(4, dtype=torch.int32, device=dev)
    rcounts = torch.full((aB,), aT, dtype=torch.int32, device=dev)
    arstep = lambda: store_kv(ainp.k_pool, ainp.v_pool, ainp.block_tables, ainp.k, ainp.v,
                              ainp.start_pos, rcounts, check=False, errors=rerr,
                              rope=(rcos, rsin))
    _, ar_ev, _, _ = time_steps(arstep, args.steps, args.warmup)
    if rerr.tolist() != [0, 0, 0, 0]:
        raise RuntimeError(f"kv append with rope reported errors {rerr.tolist()}")
    ar_gbs = abytes / (ar_ev * 1e-3) / 1e9
    log(f"[bench] {aname}: with K rotated on the way in {ar_ev:.3f} ms -> {ar_gbs:.1f} GB/s")

    # ---- fused RoPE + flash, bf16 BSHD (rotation kernels + attention) ----------------
    rstep = rope_attention_step(dev)
    log(f"[bench] rope_attention: warmup {args.warmup}, steps {args.steps}")
    r_wall, r_ev, r_min, r_med = time_steps(rstep, args.steps, args.warmup)
    r_tf = flops / (r_ev * 1e-3) / 1e12
    log(f"[bench] rope_attention: {r_wall:.3f} ms/step wall, kernels {r_ev:.3f} ms -> "
        f"{r_tf:.1f} TFLOP/s")

    # ---- backward of the headline attention (dQ, dK, dV), bf16 BHSD -------------------
    (bq, bk, bv, bdo), bstep = bwd_step(dev)
    bflops = 2.5 * flops
    log(f"[bench] flash_backward: warmup {args.warmup}, steps {args.steps}")
    b_wall, b_ev, b_min, b_med = time_steps(bstep, args.steps, args.warmup)
    b_tf = bflops / (b_ev * 1e-3) / 1e12
    log(f"[bench] flash_backward: {b_wall:.3f} ms/step wall, kernels {b_ev:.3f} ms -> "
        f"{b_tf:.1f} TFLOP/s")

    # ---- the headline attention with dropout_p = 0.1, forward and backward ------------
    d_fwd, d_bwd = dropout_steps(dev, DROPOUT_P)
    log(f"[bench] flash_dropout: warmup {args.warmup}, steps {args.steps}")
    df_wall, df_ev, df_min, df_med = time_steps(d_fwd, args.steps, args.warmup)
    db_wall, db_ev, db_min, db_med = time_steps(d_bwd, args.steps, args.warmup)
    del d_fwd, d_bwd
    df_tf = flops / (df_ev * 1e-3) / 1e12
    db_tf = bflops / (db_ev * 1e-3) / 1e12
    log(f"[bench] flash_dropout: forward {df_ev:.3f} ms -> {df_tf:.1f} TFLOP/s "
        f"({df_ev / ev_ms:.2f}x plain), backward {db_ev:.3f} ms -> {db_tf:.1f} TFLOP/s "
        f"({db_ev / b_ev:.2f}x plain)")

    # ---- head dim 256 (the D = 256 kernel), bf16 BHSD causal ----------------------------
    h_fn, hflops = d256_step(dev)
    log(f"[bench] flash_d256: warmup {args.warmup}, steps {args.steps}")
    h_wall, h_ev, h_min, h_med = time_steps(h_fn, args.steps, args.warmup)
    del h_fn
    h_tf = hflops / (h_ev * 1e-3) / 1e12
    log(f"[bench] flash_d256: {h_wall:.3f} ms/step wall, kernel {h_ev:.3f} ms -> {h_tf:.1f} TFLOP/s")

    # ---- config 3: sliding window W=4096, config 5: chunked cross attention ------------
    wcfg = wl.CONFIGS["window_bf16_bshd"]
    (wq, wk, wv), wstep = window_step(dev)
    wflops = wl.config_work("window_bf16_bshd")
    log(f"[bench] sliding_window: warmup {args.warmup}, steps {args.steps}")
    w_wall, w_ev, w_min, w_med = time_steps(wstep, args.steps, args.warmup)
    w_tf = wflops / (w_ev * 1e-3) / 1e12
    log(f"[bench] sliding_window: kernel {w_ev:.3f} ms -> {w_tf:.1f} TFLOP/s")
    ccfg = wl.CONFIGS["chunked_bf16"]
    (cq, ck, cv), cstep2 = chunked_step(dev)
    cflops = wl.config_work("chunked_bf16")
    cbytes = 2.0 * (cq.numel() * 2 + ck.numel() + cv.numel())  # q, o + k, v once, bf16
    log(f"[bench] chunked_cross: warmup {args.warmup}, steps {args.steps}")
    k_wall, k_ev, k_min, k_med = time_steps(cstep2, args.steps, args.warmup)
    k_tf = cflops / (k_ev * 1e-3) / 1e12
    k_gbs = cbytes / (k_ev * 1e-3) / 1e9
    log(f"[bench] chunked_cross: kernels {k_ev:.3f} ms -> {k_tf:.1f} TFLOP/s, {k_gbs:.0f} GB/s")

    # ---- config 1: flash fp32 BSHD (2, 1024, 12, 64), causal ----------------------------
    (oq, ok_, ov), ostep = fp32_step(dev)
    oflops = wl.config_work("flash_fp32_bshd")
    log(f"[bench] flash_fp32: warmup {args.warmup}, steps {args.steps}")
    o_wall, o_ev, o_min, o_med = time_steps(ostep, args.steps, args.warmup)
    o_tf = oflops / (o_ev * 1e-3) / 1e12
    log(f"[bench] flash_fp32: kernel {o_ev:.4f} ms -> {o_tf:.1f} TFLOP/s")

    cpu = pcpu = fcpu = acpu = bcpu = wcpu = kcpu = ocpu = dcpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baselines (oracle restatement on host cores)")
        cpu = cpu_baseline_flash(cfg, q, k, v, args.cpu_budget)
        pcpu = cpu_baseline_paged(pin, pcfg, args.cpu_budget)
        fcpu = cpu_baseline_prefill(finp, wl.CONFIGS[fname], args.cpu_budget)
        acpu = cpu_baseline_append(ainp, wl.CONFIGS[aname], args.cpu_budget)
        bcpu = cpu_baseline_bwd(cfg, bq.detach(), bk.detach(), bv.detach(), bdo,
                                args.cpu_budget)
        wcpu = cpu_baseline_window(wcfg, wq, wk, wv, args.cpu_budget)
        kcpu = cpu_baseline_chunked(ccfg, cq, ck, cv, args.cpu_budget)
        ocpu = cpu_baseline_tiled(wl.CONFIGS["flash_fp32_bshd"], oq, ok_, ov, args.cpu_budget)
        dcpu = cpu_baseline_dropout(cfg, q, k, v, DROPOUT_P, args.cpu_budget)
    del wq, wk, wv, cq, ck, cv

    result = {
        "metric": "causal fwd TFLOP/s @S=4096,D=128 + paged-decode HBM GB/s, % of roofline",
        "value": flops / (wall_ms * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1), cast to bf16)",
        "config": {"workload": "flash_attention fwd bf16 BHSD B=4 H=32 S=4096 D=128 causal, "
                               "scale 1/sqrt(128)",
                   "global_batch": cfg["B"], "seq_len": cfg["S"], "heads": cfg["H"],
                   "head_dim": cfg["D"], "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS,
                     "traffic": measured_traffic("flash_bf16_bhsd"),
                     "kernel": FLASH_KERNEL, "traffic_unit": "bytes per launch",
                     "flop_per_launch": flops, "launch_ms": ev_ms, "launch_ms_median": ev_med,
                     "launch_ms_min": ev_min},
        "cpu_baseline": cpu,
        "paged_prefill": {
            "workload": "paged prefill bf16 4x4096 tok H=32 D=128 causal, 16-token pages",
            "value": f_tf, "unit": "TFLOP/s", "ms_per_step": f_wall, "kernel_ms": f_ev, "flop_per_step": fflops,
            "roofline": {"bound": "mfma", "achieved": f_tf, "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": f_tf / PEAK_BF16_TFLOPS,
                         "traffic": measured_traffic(fname), "kernel": PREFILL_KERNEL},
            "cpu_baseline": fcpu,
        },
        "rope_attention": {
            "workload": "fused_rope_attention bf16 BSHD B=4 S=4096 H=32 D=128 causal",
            "value": r_tf, "unit": "TFLOP/s", "ms_per_step": r_wall, "kernel_ms": r_ev, "flop_per_step": flops,
            "roofline": {"bound": "mfma", "achieved": r_tf, "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": r_tf / PEAK_BF16_TFLOPS,
                         "kernel": "rope_kernel (K) + fa_fwd16_kernel<128,128,8,bf16> (Q)"},
        },
        "kv_append": {
            "workload": "store_kv bf16 4x4096 new tok H=32 D=128 into 16-token pages",
            "value": a_gbs, "unit": "GB/s", "ms_per_step": a_wall, "kernel_ms": a_ev, "bytes_per_step": abytes,
            "roofline": {"bound": "hbm", "achieved": a_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": a_gbs / PEAK_HBM_GBS, "traffic": measured_traffic(aname),
                         "kernel": APPEND_KERNEL},
            "d2d_copy_same_bytes_gbs": c_gbs,
            "with_rope": {"kernel": "kv_append_rope_kernel", "kernel_ms": ar_ev,
                          "value": ar_gbs},
            "cpu_baseline": acpu,
        },
        "sliding_window": {
            "workload": "config 3: window bf16 BSHD B=2 S=8192 H=32 D=128 causal W=4096",
            "value": w_tf, "unit": "TFLOP/s", "ms_per_step": w_wall, "kernel_ms": w_ev, "flop_per_step": wflops,
            "roofline": {"bound": "mfma", "achieved": w_tf, "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": w_tf / PEAK_BF16_TFLOPS,
                         "traffic": measured_traffic("window_bf16_bshd"),
                         "kernel": WINDOW_KERNEL},
            "cpu_baseline": wcpu,
        },
        "chunked_cross": {
            "workload": "config 5: chunked cross bf16 BSHD Lq=512 Lkv=65536 H=16 D=64",
            "value": k_tf, "unit": "TFLOP/s", "ms_per_step": k_wall, "kernel_ms": k_ev, "flop_per_step": cflops,
            "bytes_per_step": cbytes,
            "roofline": {"bound": "mfma", "achieved": k_tf, "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": k_tf / PEAK_BF16_TFLOPS,
                         "traffic": measured_traffic("chunked_bf16"),
                         "kernel": CHUNKED_KERNELS},
            "hbm_roofline": {"achieved": k_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                             "frac": k_gbs / PEAK_HBM_GBS},
            "cpu_baseline": kcpu,
        },
        "flash_fp32": {
            "workload": "config 1: flash fp32 BSHD B=2 S=1024 H=12 D=64 causal",
            "value": o_tf, "unit": "TFLOP/s", "ms_per_step": o_wall, "kernel_ms": o_ev, "flop_per_step": oflops,
            "roofline": {"bound": "mfma", "achieved": o_tf, "peak": PEAK_F32_TFLOPS,
                         "unit": "TFLOP/s", "frac": o_tf / PEAK_F32_TFLOPS,
                         "traffic": measured_traffic("flash_fp32_bshd"),
                         "kernel": FP32_KERNEL},
            "cpu_baseline": ocpu,
        },
        "flash_backward": {
            "workload": "backward (dQ, dK, dV) of the headline attention",
            "value": b_tf, "unit": "TFLOP/s", "ms_per_step": b_wall, "kernel_ms": b_ev, "flop_per_step": bflops,
            "roofline": {"bound": "mfma", "achieved": b_tf, "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": b_tf / PEAK_BF16_TFLOPS,
                         "traffic": measured_traffic("flash_backward_bf16"),
                         "kernel": BWD_KERNELS,
                         "flop": "2.5x forward"},
            "cpu_baseline": bcpu,
        },
        "flash_d256": {
            "workload": f"flash bf16 BHSD (B,H,S,D)={D256_SHAPE} causal",
            "value": h_tf, "unit": "TFLOP/s", "ms_per_step": h_wall, "kernel_ms": h_ev, "flop_per_step": hflops,
            "roofline": {"bound": "mfma", "achieved": h_tf, "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": h_tf / PEAK_BF16_TFLOPS,
                         "kernel": "fa_fwd16_wide_kernel<256,64,4,bf16>",
                         "traffic": measured_traffic("flash_d256_bf16")},
        },
        "flash_dropout": {
            "workload": f"headline shape as BSHD views, dropout_p={DROPOUT_P}, fwd and bwd",
            "value": df_tf, "unit": "TFLOP/s", "ms_per_step": df_wall, "kernel_ms": df_ev, "flop_per_step": flops,
            "vs_plain_forward": df_ev / ev_ms,
            "roofline": {"bound": "mfma", "achieved": df_tf, "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": df_tf / PEAK_BF16_TFLOPS,
                         "kernel": DROPOUT_KERNEL, "traffic": None},
            "backward": {"value": db_tf, "unit": "TFLOP/s", "ms_per_step": db_wall,
                         "kernel_ms": db_ev,
                         "flop_per_step": bflops, "frac": db_tf / PEAK_BF16_TFLOPS,
                         "vs_plain_backward": db_ev / b_ev, "kernel": DROPOUT_BWD_KERNELS},
            "cpu_baseline": dcpu,
        },
        "paged_decode_gqa": {
            "workload": "config 4 with enable_gqa: 32 query heads over 8 K/V heads",
            "value": g_gbs, "unit": "GB/s", "ms_per_step": g_wall, "kernel_ms": g_ev, "bytes_per_step": gbytes,
            "roofline": {"bound": "hbm", "achieved": g_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": g_gbs / PEAK_HBM_GBS,
                         "traffic": measured_traffic(gname),
                         "kernel": GQA_KERNELS},
        },
        "paged_decode": {
            "workload": "config 4: paged decode fp16, 64 seqs, H=32, D=128, ctx~U{512..8192}, "
                        "16-token pages, permuted block table",
            "value": p_gbs, "unit": "GB/s", "ms_per_step": p_wall, "kernel_ms": p_ev,
            "kernel_ms_median": p_med, "kernel_ms_min": p_min,
            "bytes_per_step": pbytes,
            "roofline": {"bound": "hbm", "achieved": p_gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": p_gbs / PEAK_HBM_GBS,
                         "traffic": measured_traffic("paged_decode_fp16"),
                         "kernel": PAGED_KERNELS, "traffic_unit": "bytes per launch"},
            "cpu_baseline": pcpu,
        },
    }
    # Config 4 (paged decode) is half of the headline metric: it is the last key, and the
    # line is compact (4 significant digits, no spaces), so a reader of only the last
    # couple of KB of stdout still sees its roofline and CPU baseline.
    print(json.dumps(compact(result), separators=(",", ":")), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
