"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture (a regression guard on the oracle; the
fixtures themselves were cross-checked against torch SDPA in float64 when they
were written). GPU: the HIP kernels, called through the drop-in API, match the
fixtures at the parity tolerances (float32 rtol 1e-4 / atol 1e-5; bf16 / fp16
max-abs 2e-2).
"""

import glob
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import attention_grad as oag
from oracle import kv_cache as ok
from oracle import paged as op

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))
TORCH_DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def load(path):
    with np.load(path, allow_pickle=False) as z:
        arrays = {k: z[k] for k in z.files}
    meta = json.loads(str(arrays.pop("meta")))
    return meta, arrays


def fixture_id(path):
    return os.path.splitext(os.path.basename(path))[0]


def oracle_output(meta, a):
    f64 = {k: v.astype(np.float64) if v.dtype == np.float32 else v for k, v in a.items()}
    kind = meta["kind"]
    if kind == "flash":
        return oa.flash_attention(f64["q"], f64["k"], f64["v"], scale=meta["scale"],
                                  causal=meta["causal"], layout=meta["layout"])
    if kind == "flash_default":
        return oa.flash_attention_default_route(f64["q"], f64["k"], f64["v"],
                                                causal=meta["causal"], layout=meta["layout"])
    if kind == "window":
        return oa.sliding_window_attention(f64["q"], f64["k"], f64["v"], meta["window"],
                                           causal=meta["causal"])
    if kind == "chunked":
        return oa.chunked_cross_attention(f64["q"], f64["k"], f64["v"],
                                          chunk_size=meta["chunk_size"], causal=meta["causal"])
    if kind == "grad":
        W = meta["window"]
        wl, wr = (W, -1 if meta["causal"] else W) if W >= 0 else (-1, -1)
        D = a["q"].shape[-1]
        return np.stack(oag.attention_grad(f64["q"], f64["k"], f64["v"], f64["dout"],
                                           1.0 / math.sqrt(D), meta["causal"], wl, wr,
                                           layout=meta["layout"]))
    if kind == "kv_append":
        kp, vp = f64["k_pool"].copy(), f64["v_pool"].copy()
        ok.kv_append(kp, vp, a["block_tables"], f64["k"], f64["v"], a["start_pos"],
                     a["n_tokens"], meta["block_size"])
        return np.stack([kp, vp])
    H, D = a["q"].shape[2], a["q"].shape[3]
    slopes = op.get_alibi_slopes(H) if meta["alibi"] else None
    if kind == "paged_prefill":
        return op.paged_attention_prefill(f64["q"], f64["k_pool"], f64["v_pool"],
                                          a["block_tables"], a["context_lens"],
                                          1.0 / math.sqrt(D), meta["block_size"], meta["causal"],
                                          alibi_slopes=slopes)
    return op.paged_attention_decode(f64["q"], f64["k_pool"], f64["v_pool"], a["block_tables"],
                                     a["context_lens"], 1.0 / math.sqrt(D), meta["block_size"],
                                     alibi_slopes=slopes)


def test_fixtures_present():
    assert len(FIXTURES) >= 16


@pytest.mark.parametrize("path", FIXTURES, ids=fixture_id)
def test_oracle_matches_golden(path):
    meta, a = load(path)
    np.testing.assert_allclose(oracle_output(meta, a), a["expected"], rtol=1e-12, atol=1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=fixture_id)
def test_kernel_matches_golden(device, path):
    from mlx_primitives.attention import chunked_cross_attention, flash_attention, sliding_window_attention
    from mlx_primitives.cache import get_alibi_slopes, paged_attention, store_kv

    meta, a = load(path)
    dt = TORCH_DTYPES[meta["dtype"]]
    t = {k: torch.from_numpy(v).to(dt if v.dtype == np.float32 else torch.int32).to(device)
         for k, v in a.items() if k != "expected"}
    kind = meta["kind"]
    if kind == "grad":
        # gradients through autograd -> mpx_attn_bwd, at the reference's gradient bar
        # (tests/parity/shared/tolerance_config.py:57, 363-387: 10x the forward's)
        qg, kg, vg = (t[n].clone().requires_grad_(True) for n in ("q", "k", "v"))
        if meta["window"] >= 0:
            out = sliding_window_attention(qg, kg, vg, meta["window"], causal=meta["causal"])
        else:
            out = flash_attention(qg, kg, vg, causal=meta["causal"], layout=meta["layout"])
        out.backward(t["dout"])
        got = torch.stack([qg.grad, kg.grad, vg.grad]).double().cpu().numpy()
        rtol, atol = {torch.float32: (1e-3, 1e-4), torch.float16: (1e-2, 1e-2),
                      torch.bfloat16: (1e-1, 1e-1)}[dt]
        np.testing.assert_allclose(got, a["expected"], rtol=rtol, atol=atol)
        return
    if kind == "flash":
        out = flash_attention(t["q"], t["k"], t["v"], scale=meta["scale"], causal=meta["causal"],
                              layout=meta["layout"])
    elif kind == "flash_default":
        out = flash_attention(t["q"], t["k"], t["v"], causal=meta["causal"], layout=meta["layout"])
    elif kind == "window":
        out = sliding_window_attention(t["q"], t["k"], t["v"], meta["window"], causal=meta["causal"])
    elif kind == "chunked":
        out = chunked_cross_attention(t["q"], t["k"], t["v"], chunk_size=meta["chunk_size"],
                                      causal=meta["causal"])
    elif kind == "kv_append":
        store_kv(t["k_pool"], t["v_pool"], t["block_tables"], t["k"], t["v"], t["start_pos"],
                 t["n_tokens"])
        # a copy: the pools must equal the expected ones exactly
        got = torch.stack([t["k_pool"], t["v_pool"]]).double().cpu().numpy()
        np.testing.assert_array_equal(got, a["expected"])
        return
    else:
        H = a["q"].shape[2]
        slopes = get_alibi_slopes(H).to(device) if meta["alibi"] else None
        out = paged_attention(t["q"], t["k_pool"], t["v_pool"], t["block_tables"],
                              t["context_lens"], block_size=meta["block_size"],
                              causal=meta.get("causal", True), alibi_slopes=slopes)
    assert out.dtype == dt
    got = out.double().cpu().numpy()
    exp = a["expected"]
    assert got.shape == exp.shape
    if dt == torch.float32:
        np.testing.assert_allclose(got, exp, rtol=1e-4, atol=1e-5)
    else:
        err = float(np.abs(got - exp).max())
        assert err <= 2e-2, f"max abs err {err}"
