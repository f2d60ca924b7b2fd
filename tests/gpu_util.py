"""Helpers for the GPU parity tests: seeded synthetic pools on the device and
their numpy mirrors for the oracle."""

from __future__ import annotations

import numpy as np
import torch

from oracle import paged_ref as R

NP = {torch.float32: np.float32, torch.float16: np.float16, torch.bfloat16: np.float32}


def dev():
    return torch.device("cuda:0")


def to_np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        return t.float().cpu().numpy()
    return t.cpu().numpy()


def fill_cache(cache, gen: torch.Generator):
    """Random pool contents: N(0,1) for fp pools; for int8 pools, N(0,1) fp16
    values quantized by the oracle (the configs' recipe), so the attention
    tests do not depend on the write kernel."""
    if cache.k_cache.dtype == torch.int8:
        sdt = np.float16 if cache.k_scale.dtype == torch.float16 else np.float32
        for t, s in ((cache.k_cache, cache.k_scale), (cache.v_cache, cache.v_scale)):
            x = torch.randn(t.shape, generator=gen).half().float().numpy()
            q, sc = R.quantize(x)
            t.copy_(torch.from_numpy(q))
            s.copy_(torch.from_numpy(R.store_scale(sc, sdt)))
    else:
        for t in (cache.k_cache, cache.v_cache):
            t.copy_(torch.randn(t.shape, generator=gen).to(t.dtype))


def pool_of(cache) -> R.PagedPool:
    """numpy mirror of a device cache, compute dtype float32 (values exact)."""
    quant = cache.k_cache.dtype == torch.int8
    p = R.PagedPool(cache.num_blocks, cache.block_size, cache.n_kv_heads, cache.head_dim,
                    np.float32, quantized=quant,
                    scale_dtype=np.float16 if (quant and cache.k_scale.dtype == torch.float16) else np.float32)
    p.k = to_np(cache.k_cache)
    p.v = to_np(cache.v_cache)
    if quant:
        p.k_scale = to_np(cache.k_scale)
        p.v_scale = to_np(cache.v_scale)
    else:
        p.k = p.k.astype(np.float32)
        p.v = p.v.astype(np.float32)
    return p


def pool_dequantized(cache) -> R.PagedPool:
    """numpy mirror of an int8 cache as helios' gather hands it to attention:
    (q.float() * s.float()).to(compute dtype) (paged_attn.py:213-235), held
    as the float32 values those fp16 / bf16 numbers represent.  The MFMA
    prefill kernel attends over exactly these values."""
    out = {torch.float16: np.float16, torch.bfloat16: "bfloat16"}[cache.dtype]
    p = R.PagedPool(cache.num_blocks, cache.block_size, cache.n_kv_heads, cache.head_dim, np.float32)
    p.k = R.dequantize(to_np(cache.k_cache), to_np(cache.k_scale), out).astype(np.float32)
    p.v = R.dequantize(to_np(cache.v_cache), to_np(cache.v_scale), out).astype(np.float32)
    return p


def ragged_tables(gen: np.random.Generator, lens, block_size, num_blocks, shuffle=True):
    """Non-contiguous block tables from a (shuffled) pool."""
    need = [(c + block_size - 1) // block_size for c in lens]
    ids = np.arange(num_blocks)
    if shuffle:
        gen.shuffle(ids)
    assert sum(need) <= num_blocks
    out, o = [], 0
    for n in need:
        out.append([int(x) for x in ids[o:o + n]])
        o += n
    return out


def max_abs(a: np.ndarray, b: np.ndarray) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)))) if a.size else 0.0
