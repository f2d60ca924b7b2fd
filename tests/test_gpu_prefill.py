"""GPU parity of the chunked-prefill / verify kernel (hpa_paged_prefill)
against the oracle.  Tolerances as in test_gpu_decode.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import (
    PagedKVCache,
    QuantizedPagedKVCache,
    paged_attention_prefill,
    paged_attention_varlen,
    paged_attention_verify_batched,
)
from oracle import paged_ref as R
from tests.gpu_util import dev, fill_cache, pool_dequantized, pool_of, ragged_tables, to_np
from tests.test_gpu_decode import _check

pytestmark = pytest.mark.gpu


def _setup(seed, ctxs, Hq, Hkv, D, bs, dtype, quant=False, scale_dtype=torch.float16):
    gen = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    nb = sum((c + bs - 1) // bs for c in ctxs) + 2
    cache = (QuantizedPagedKVCache(nb, bs, Hkv, D, dtype=dtype, device="cuda", scale_dtype=scale_dtype)
             if quant else PagedKVCache(nb, bs, Hkv, D, dtype=dtype, device="cuda"))
    fill_cache(cache, gen)
    return cache, ragged_tables(rng, ctxs, bs, nb), gen


@pytest.mark.parametrize("n_tokens", [1, 7, 11, 16, 33])
def test_prefill_matches_dense_reference_shapes(n_tokens):
    """reference tests/parity/test_parity.py:89-108 shapes (bs 4, D 8,
    Hkv 2, Hq 4, blocks (7i+3) % 32), fp32."""
    torch.manual_seed(0)
    bs, n_kv, hd, n_q = 4, 2, 8, 4
    cache = PagedKVCache(32, bs, n_kv, hd, dtype=torch.float32, device="cuda")
    blocks = [(7 * i + 3) % 32 for i in range((n_tokens + bs - 1) // bs)]
    k = torch.randn(n_tokens, n_kv, hd, device="cuda")
    v = torch.randn(n_tokens, n_kv, hd, device="cuda")
    q = torch.randn(n_tokens, n_q, hd, device="cuda")
    cache.write(blocks, 0, k, v)
    got = paged_attention_prefill(q, cache, blocks, 0, n_tokens)
    want = R.dense_causal_attention(to_np(q), to_np(k), to_np(v), n_q // n_kv)
    np.testing.assert_allclose(to_np(got), want, atol=2e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [16, 64, 128])
def test_varlen_matches_oracle(dtype, D):
    qlens = [1, 5, 64, 200, 33]
    starts = [0, 40, 100, 0, 1000]
    ctxs = [s + n for s, n in zip(starts, qlens)]
    cache, tables, gen = _setup(D, ctxs, 8, 2, D, 16, dtype)
    q = torch.randn(sum(qlens), 8, D, generator=gen).to(dtype).to(dev())
    got = paged_attention_varlen(q, cache, tables, qlens, starts, ctxs)
    want = R.paged_varlen(to_np(q).astype(np.float32), pool_of(cache), tables, qlens, starts, ctxs)
    _check(got, want, dtype, f"varlen D={D}")


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_varlen_int8(scale_dtype):
    qlens = [17, 128, 3]
    starts = [500, 0, 70]
    ctxs = [s + n for s, n in zip(starts, qlens)]
    cache, tables, gen = _setup(5, ctxs, 32, 8, 128, 16, torch.float16, quant=True,
                                scale_dtype=scale_dtype)
    q = torch.randn(sum(qlens), 32, 128, generator=gen).half().to(dev())
    got = paged_attention_varlen(q, cache, tables, qlens, starts, ctxs)
    # the MFMA kernel attends over helios' fp16 gather of the int8 pool
    want = R.paged_varlen(to_np(q).astype(np.float32), pool_dequantized(cache), tables, qlens, starts, ctxs)
    _check(got, want, torch.float16)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D,bs", [(128, 16), (64, 32)])
def test_mfma_prefill_int8(dtype, scale_dtype, D, bs):
    """INT8 pools on the MFMA kernel: ragged chunks, partial last blocks,
    contexts shorter than a step, several steps per row tile."""
    qlens = [1, 37, 130, 9, 64]
    starts = [3, 0, 250, 64, 700]
    ctxs = [s + n for s, n in zip(starts, qlens)]
    cache, tables, gen = _setup(D + bs, ctxs, 16, 4, D, bs, dtype, quant=True, scale_dtype=scale_dtype)
    q = torch.randn(sum(qlens), 16, D, generator=gen).to(dtype).to(dev())
    got = paged_attention_varlen(q, cache, tables, qlens, starts, ctxs)
    want = R.paged_varlen(to_np(q).astype(np.float32), pool_dequantized(cache), tables, qlens, starts, ctxs)
    _check(got, want, dtype, f"int8 {dtype} scales {scale_dtype} D={D} bs={bs}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_mfma_int8_dequantisation_is_helios_gather(dtype, scale_dtype):
    """With one key in context every query row's output is that key's V row
    (p = 1), so the kernel's dequantisation shows bit for bit: it must equal
    (q.float() * s.float()).to(dtype), helios' gather (paged_attn.py:228-233),
    for every int8 value and scales across the fp16 range."""
    H, D, bs = 2, 128, 16
    cache = QuantizedPagedKVCache(4, bs, H, D, dtype=dtype, device="cuda", scale_dtype=scale_dtype)
    gen = torch.Generator().manual_seed(1)
    cache.k_cache.copy_(torch.randint(-127, 128, cache.k_cache.shape, generator=gen, dtype=torch.int8))
    v = torch.randint(-127, 128, cache.v_cache.shape, generator=gen, dtype=torch.int8)
    v[2, 0, 0, :] = torch.arange(-127, 1, dtype=torch.int8)[:D]      # every value appears
    v[2, 1, 0, :] = torch.arange(0, 128, dtype=torch.int8)[:D]
    cache.v_cache.copy_(v)
    # 2^-22 .. 2^8: products from fp16 subnormals up to 127 * 256, all finite
    scales = torch.exp2(torch.rand(cache.v_scale.shape, generator=gen) * 30 - 22)
    cache.k_scale.copy_(scales.to(scale_dtype))
    cache.v_scale.copy_(scales.flip(-1).to(scale_dtype))
    q = torch.randn(1, 8, D, generator=gen).to(dtype).to(dev())
    got = paged_attention_varlen(q, cache, [[2]], [1], [0], [1])
    want = (cache.v_cache[2, :, 0, :].float() * cache.v_scale[2, :, 0, None].float()).to(dtype)
    assert torch.equal(got[0].view(H, 4, D), want[:, None, :].expand(H, 4, D))


def test_chunked_prefill_equals_single_shot():
    """reference tests/parity/test_parity.py:154-186 at the attention level:
    chunks attending to their cached prefix reproduce single-shot prefill."""
    cache, tables, gen = _setup(9, [300], 8, 2, 64, 16, torch.float16)
    q = torch.randn(300, 8, 64, generator=gen).half().to(dev())
    single = paged_attention_prefill(q, cache, tables[0], 0, 300)
    parts = [paged_attention_prefill(q[s:s + 64], cache, tables[0], s, min(s + 64, 300))
             for s in range(0, 300, 64)]
    chunked = torch.cat(parts)
    assert (chunked.float() - single.float()).abs().max().item() <= 2e-3
    want = R.paged_prefill(to_np(q).astype(np.float32), pool_of(cache), tables[0], 0, 300)
    _check(single, want, torch.float16)


@pytest.mark.parametrize("quant", [False, True])
def test_prefix_shared_blocks_config4_shape(quant):
    """Config 4 in miniature: Llama-8B heads (32/8, D 128), 4 sequences each
    appending a 128-token chunk onto prior context; the first 16 blocks of
    every table are the same physical blocks (prefix-cache aliasing).  Also
    on an int8 pool (the MFMA kernel's fused dequantisation)."""
    rng = np.random.default_rng(4)
    gen = torch.Generator().manual_seed(4)
    bs, shared = 16, 16
    priors = [300, 0, 1024, 57]
    chunk = 128
    nb = 400
    cache = (QuantizedPagedKVCache(nb, bs, 8, 128, dtype=torch.float16, device="cuda") if quant
             else PagedKVCache(nb, bs, 8, 128, dtype=torch.float16, device="cuda"))
    fill_cache(cache, gen)
    ids = list(rng.permutation(nb))
    prefix = [int(x) for x in ids[:shared]]
    free = [int(x) for x in ids[shared:]]
    tables = []
    for p in priors:
        need = (p + chunk + bs - 1) // bs
        own = min(shared, p // bs)
        t = prefix[:own] + [free.pop() for _ in range(need - own)]
        tables.append(t)
    ctxs = [p + chunk for p in priors]
    q = torch.randn(chunk * len(priors), 32, 128, generator=gen).half().to(dev())
    got = paged_attention_varlen(q, cache, tables, [chunk] * 4, priors, ctxs)
    want = R.paged_varlen(to_np(q).astype(np.float32), pool_dequantized(cache) if quant else pool_of(cache),
                          tables, [chunk] * 4, priors, ctxs)
    _check(got, want, torch.float16)


def test_verify_kernels_agree():
    """The decode kernel's multi-token verify and the prefill kernel compute
    the same attention (both against the oracle too)."""
    lens = [40, 2049, 7]
    cache, tables, gen = _setup(11, lens, 32, 8, 128, 16, torch.float16, quant=True)
    q = torch.randn(9, 32, 128, generator=gen).half().to(dev())
    a = paged_attention_verify_batched(q, cache, tables, lens, 3)
    b = paged_attention_varlen(q, cache, tables, [3] * 3, [c - 3 for c in lens], lens)
    assert (a.float() - b.float()).abs().max().item() <= 2e-3
    # the decode kernel dequantises exactly in fp32; the MFMA prefill attends
    # over helios' fp16 gather of the same int8 pool
    want = R.paged_verify_batched(to_np(q).astype(np.float32), pool_of(cache), tables, lens, 3)
    _check(a, want, torch.float16)
    want_b = R.paged_verify_batched(to_np(q).astype(np.float32), pool_dequantized(cache), tables, lens, 3)
    _check(b, want_b, torch.float16)


def test_rows_without_keys_are_zero():
    cache, tables, gen = _setup(12, [10], 4, 2, 64, 16, torch.float16)
    q = torch.randn(3, 4, 64, generator=gen).half().to(dev())
    # context 0: nothing to attend
    got = paged_attention_varlen(q, cache, tables, [3], [0], [0])
    assert torch.count_nonzero(got) == 0


@pytest.mark.parametrize("Hq,Hkv,D,bs,dtype", [
    (14, 2, 64, 16, torch.float16),    # Qwen2.5-0.5B heads: group of 7 rows per token
    (14, 2, 64, 32, torch.bfloat16),
    (8, 8, 128, 64, torch.float16),    # group of 1
    (32, 4, 128, 16, torch.bfloat16),  # group of 8
])
def test_mfma_prefill_group_and_block_shapes(Hq, Hkv, D, bs, dtype):
    """The fp16/bf16 MFMA kernel packs the group's query heads into 128-row
    tiles; row tiles then end mid-token for groups that do not divide 128."""
    qlens = [1, 37, 130, 9]
    starts = [3, 0, 250, 64]
    ctxs = [s + n for s, n in zip(starts, qlens)]
    cache, tables, gen = _setup(Hq + bs, ctxs, Hq, Hkv, D, bs, dtype)
    q = torch.randn(sum(qlens), Hq, D, generator=gen).to(dtype).to(dev())
    got = paged_attention_varlen(q, cache, tables, qlens, starts, ctxs)
    want = R.paged_varlen(to_np(q).astype(np.float32), pool_of(cache), tables, qlens, starts, ctxs)
    _check(got, want, dtype, f"Hq={Hq} Hkv={Hkv} D={D} bs={bs}")


def test_mfma_prefill_context_shorter_than_chunk():
    """context_len below start + n caps every row's keys at the context
    (paged_attn.py:401-404 with the gather cut at context_len)."""
    qlens = [20, 6]
    starts = [40, 0]
    ctxs = [45, 3]
    cache, tables, gen = _setup(21, [60, 6], 16, 4, 128, 16, torch.float16)
    q = torch.randn(sum(qlens), 16, 128, generator=gen).half().to(dev())
    got = paged_attention_varlen(q, cache, tables, qlens, starts, ctxs)
    want = R.paged_varlen(to_np(q).astype(np.float32), pool_of(cache), tables, qlens, starts, ctxs)
    _check(got, want, torch.float16)


@pytest.mark.parametrize("n_seqs", [100, 520])
def test_mfma_prefill_many_small_sequences(n_seqs):
    """Many (sequence, KV head) items: 100 sequences keep the longest-first
    order of each XCD's items; 520 x 8 heads exceed the 512 items per XCD it
    ranks and run in dispatch order.  Every row is checked."""
    rng = np.random.default_rng(n_seqs)
    qlens = [int(x) for x in rng.integers(1, 5, size=n_seqs)]
    ctxs = [int(x) for x in rng.integers(1, 61, size=n_seqs)]
    starts = [max(c - n, 0) for c, n in zip(ctxs, qlens)]
    cache, tables, gen = _setup(n_seqs, ctxs, 32, 8, 128, 16, torch.float16)
    q = torch.randn(sum(qlens), 32, 128, generator=gen).half().to(dev())
    got = paged_attention_varlen(q, cache, tables, qlens, starts, ctxs)
    want = R.paged_varlen(to_np(q).astype(np.float32), pool_of(cache), tables, qlens, starts, ctxs)
    _check(got, want, torch.float16, f"{n_seqs} sequences")
