"""CPU checks of the Python surface that mirrors helios' paged_attn module:
names, attributes, byte accounting, host-side validation, and that there is
no CPU fallback (a CPU tensor is refused, never computed)."""

from __future__ import annotations

import inspect

import pytest
import torch

import helios_amd
from helios_amd import (
    PagedKVCache,
    QuantizedPagedKVCache,
    paged_attention_decode,
    paged_attention_decode_batched,
    paged_attention_prefill,
)

N_BLOCKS, BLOCK, HEADS, DIM = 8, 16, 2, 64


def _caches(dtype=torch.float32):
    kw = dict(num_blocks=N_BLOCKS, block_size=BLOCK, n_kv_heads=HEADS, head_dim=DIM,
              dtype=dtype, device="cpu")
    return PagedKVCache(**kw), QuantizedPagedKVCache(**kw)


def test_quantized_cache_is_a_drop_in_for_the_fp_cache():
    """reference tests/quant/test_kv_quant.py:38-45."""
    _fp, q = _caches()
    for name in ("write", "gather", "copy_block", "nbytes", "block_size", "n_kv_heads",
                 "head_dim", "num_blocks", "dtype", "k_cache", "v_cache", "k_scale",
                 "v_scale", "device"):
        assert hasattr(q, name), name
    assert isinstance(q, PagedKVCache)
    assert q.k_cache.dtype == torch.int8 and q.k_scale.dtype == torch.float16
    assert tuple(q.k_scale.shape) == (N_BLOCKS, HEADS, BLOCK)


def test_byte_accounting_matches_helios():
    """reference tests/quant/test_kv_quant.py:47-58."""
    fp, q = _caches()
    assert fp.nbytes / q.nbytes > 3.5
    fp16, q16 = _caches(torch.float16)
    assert 1.8 < fp16.nbytes / q16.nbytes < 2.0
    q32 = QuantizedPagedKVCache(N_BLOCKS, BLOCK, HEADS, DIM, torch.float16, "cpu",
                                scale_dtype=torch.float32)
    assert q32.nbytes == 2 * (N_BLOCKS * HEADS * BLOCK * DIM + N_BLOCKS * HEADS * BLOCK * 4)


def test_signatures_match_the_reference_api():
    """Positional names as in reference exec/paged_attn.py:264-270, :298-304, :368-375."""
    assert list(inspect.signature(paged_attention_decode).parameters) == [
        "query", "kv_cache", "block_ids", "context_len", "scale"]
    assert list(inspect.signature(paged_attention_decode_batched).parameters) == [
        "query", "kv_cache", "block_tables", "context_lens", "scale"]
    assert list(inspect.signature(paged_attention_prefill).parameters) == [
        "query", "kv_cache", "block_ids", "start_pos", "context_len", "scale"]
    assert list(inspect.signature(PagedKVCache.write).parameters) == [
        "self", "block_ids", "start_pos", "k", "v"]
    params = list(inspect.signature(helios_amd.paged_attention_decode_hip).parameters)
    assert params[:8] == ["query", "k_cache", "v_cache", "block_tables", "context_lens", "scale",
                          "k_scale", "v_scale"]


def test_gather_short_table_raises_index_error_before_any_gpu_work():
    """reference tests/parity/test_parity.py:145-148 (same message text)."""
    fp, q = _caches()
    for c in (fp, q):
        with pytest.raises(IndexError, match="context_len 99 needs 7 blocks, have 1"):
            c.gather([0], 99)


def test_write_past_the_table_raises_like_helios():
    """reference tests/quant/test_kv_quant.py:148-152."""
    _fp, q = _caches()
    k = torch.randn(BLOCK, HEADS, DIM)
    with pytest.raises(IndexError, match="logical block"):
        q.write([0], BLOCK * 2, k, k)


def test_block_ids_outside_the_pool_raise_index_error():
    fp, _q = _caches()
    with pytest.raises(IndexError, match="outside the pool"):
        paged_attention_decode(torch.randn(4, DIM), fp, [N_BLOCKS + 3], 5)


def test_empty_gather_and_empty_batch():
    fp, _q = _caches()
    k, v = fp.gather([], 0)
    assert k.shape == (0, HEADS, DIM) and v is k
    q = torch.randn(0, 4, DIM)
    assert paged_attention_decode_batched(q, fp, [], []) is q


def test_no_cpu_fallback():
    fp, _q = _caches()
    with pytest.raises(RuntimeError, match="GPU"):
        paged_attention_decode(torch.randn(4, DIM), fp, [0], 5)
    with pytest.raises(RuntimeError, match="GPU"):
        paged_attention_prefill(torch.randn(3, 4, DIM), fp, [0], 2, 5)
    with pytest.raises(RuntimeError, match="GPU"):
        fp.gather([0], 5)


def test_product_never_imports_the_oracle():
    import pathlib

    pkg = pathlib.Path(helios_amd.__file__).parent
    for src in pkg.rglob("*.py"):
        text = src.read_text()
        assert "oracle" not in text.replace("# oracle", ""), f"{src} mentions the oracle"
