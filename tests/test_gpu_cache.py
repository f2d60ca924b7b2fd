"""GPU parity of the KV-cache kernels: quantize+scatter write (bit-exact int8
payload and scales), fp scatter, gather/dequant and batched block copies."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helios_amd import PagedKVCache, QuantizedPagedKVCache, copy_blocks, write_kv
from oracle import paged_ref as R
from tests.gpu_util import to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("in_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D", [16, 64, 128, 256])
def test_int8_write_is_bit_exact(in_dtype, scale_dtype, D):
    gen = torch.Generator().manual_seed(D)
    bs, H, nb = 16, 2, 20
    cache = QuantizedPagedKVCache(nb, bs, H, D, dtype=torch.float16, device="cuda",
                                  scale_dtype=scale_dtype)
    pool = R.PagedPool(nb, bs, H, D, np.float32, quantized=True,
                       scale_dtype=np.float16 if scale_dtype == torch.float16 else np.float32)
    blocks = [7, 3, 19, 0]
    # mixed magnitudes, exact zeros rows and .5 ties after scaling
    k = (torch.randn(50, H, D, generator=gen) * torch.rand(50, H, 1, generator=gen) * 10)
    v = torch.randn(50, H, D, generator=gen)
    k[3] = 0.0
    v[4, 0, :] = torch.arange(D, dtype=torch.float32) - D / 2
    k, v = k.to(in_dtype), v.to(in_dtype)
    cache.write(blocks, 5, k.cuda(), v.cuda())
    pool.write(blocks, 5, k.float().numpy(), v.float().numpy())
    assert np.array_equal(to_np(cache.k_cache), pool.k)
    assert np.array_equal(to_np(cache.v_cache), pool.v)
    assert np.array_equal(to_np(cache.k_scale).view(np.uint8), pool.k_scale.view(np.uint8))
    assert np.array_equal(to_np(cache.v_scale).view(np.uint8), pool.v_scale.view(np.uint8))


def test_config3_new_token_write_per_sequence():
    """Config 3's write: one new token per sequence for 64 sequences, at
    position ctx - 1 through each sequence's table, fp16 input."""
    rng = np.random.default_rng(3)
    gen = torch.Generator().manual_seed(3)
    B, H, D, bs = 64, 2, 64, 16
    lens = rng.integers(512, 4097, size=B)
    need = [(int(c) + bs - 1) // bs for c in lens]
    nb = sum(need)
    ids = rng.permutation(nb)
    tables, o = [], 0
    for n in need:
        tables.append([int(x) for x in ids[o:o + n]])
        o += n
    cache = QuantizedPagedKVCache(nb, bs, H, D, dtype=torch.float16, device="cuda")
    pool = R.PagedPool(nb, bs, H, D, np.float32, quantized=True)
    k = torch.randn(B, H, D, generator=gen).half()
    v = torch.randn(B, H, D, generator=gen).half()
    starts = [int(c) - 1 for c in lens]
    write_kv(cache, tables, starts, k.cuda(), v.cuda(), query_lens=[1] * B)
    for b in range(B):
        pool.write(tables[b], starts[b], k[b:b + 1].float().numpy(), v[b:b + 1].float().numpy())
    assert np.array_equal(to_np(cache.k_cache), pool.k)
    assert np.array_equal(to_np(cache.v_cache), pool.v)
    assert np.array_equal(to_np(cache.k_scale), pool.k_scale)
    assert np.array_equal(to_np(cache.v_scale), pool.v_scale)


def test_write_with_device_offsets_matches_list_lengths():
    """write_kv with int32 device offsets (cu_query_lens + max_query_len, no
    host work) writes exactly what the list form writes, ragged lengths and
    an empty sequence included."""
    gen = torch.Generator().manual_seed(5)
    H, D, bs, nb = 2, 64, 16, 48
    qlens = [3, 0, 5, 1, 17]
    starts = [13, 40, 0, 31, 2]
    perm = np.random.default_rng(5).permutation(nb)
    tables = [[int(x) for x in perm[8 * i:8 * i + 8]] for i in range(len(qlens))]
    k = torch.randn(sum(qlens), H, D, generator=gen).half().cuda()
    v = torch.randn(sum(qlens), H, D, generator=gen).half().cuda()
    a = QuantizedPagedKVCache(nb, bs, H, D, dtype=torch.float16, device="cuda")
    b = QuantizedPagedKVCache(nb, bs, H, D, dtype=torch.float16, device="cuda")
    write_kv(a, tables, starts, k, v, query_lens=qlens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(qlens)]), dtype=torch.int32, device="cuda")
    tab = torch.tensor(tables, dtype=torch.int32, device="cuda")
    st = torch.tensor(starts, dtype=torch.int32, device="cuda")
    write_kv(b, tab, st, k, v, cu_query_lens=cu, max_query_len=max(qlens))
    torch.cuda.synchronize()
    for x, y in ((a.k_cache, b.k_cache), (a.v_cache, b.v_cache), (a.k_scale, b.k_scale), (a.v_scale, b.v_scale)):
        assert torch.equal(x, y)
    with pytest.raises(ValueError):
        write_kv(b, tab, st, k, v, cu_query_lens=cu)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_fp_write_and_gather_round_trip(dtype):
    """reference tests/parity/test_parity.py:134-142 on the device."""
    cache = PagedKVCache(16, 4, 2, 8, dtype=dtype, device="cuda")
    blocks = [11, 2, 7]
    k = torch.randn(10, 2, 8, device="cuda").to(dtype)
    v = torch.randn(10, 2, 8, device="cuda").to(dtype)
    cache.write(blocks, 0, k, v)
    gk, gv = cache.gather(blocks, 10)
    assert torch.equal(gk, k) and torch.equal(gv, v)
    # input dtype differing from the pool's is rounded to the pool's
    k32 = torch.randn(3, 2, 8, device="cuda")
    cache.write(blocks, 4, k32, k32)
    gk, _ = cache.gather(blocks, 7)
    assert torch.equal(gk[4:7], k32.to(dtype))


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_int8_gather_dequantises_like_helios(scale_dtype, dtype):
    """(q.float() * s.float()).to(dtype), bit for bit: with fp32 scales the
    product is rounded to fp32 and then to the compute dtype, two roundings
    that must not be fused into one (300 sequences' worth of products, so
    the rare double-rounding cases occur)."""
    gen = torch.Generator().manual_seed(0)
    cache = QuantizedPagedKVCache(40, 16, 2, 64, dtype=dtype, device="cuda", scale_dtype=scale_dtype)
    pool = R.PagedPool(40, 16, 2, 64, np.float16 if dtype == torch.float16 else "bfloat16", quantized=True,
                       scale_dtype=np.float16 if scale_dtype == torch.float16 else np.float32)
    blocks = [int(x) for x in np.random.default_rng(0).permutation(40)]
    k = torch.randn(640, 2, 64, generator=gen) * torch.rand(640, 2, 1, generator=gen) * 7
    v = torch.randn(640, 2, 64, generator=gen)
    cache.write(blocks, 0, k.cuda(), v.cuda())
    pool.write(blocks, 0, k.numpy(), v.numpy())
    gk, gv = cache.gather(blocks, 640)
    wk, wv = pool.gather(blocks, 640)
    assert np.array_equal(to_np(gk.float()), np.asarray(wk, np.float32))
    assert np.array_equal(to_np(gv.float()), np.asarray(wv, np.float32))


def test_partial_block_write_and_out_of_range():
    """reference tests/quant/test_kv_quant.py:134-152."""
    cache = QuantizedPagedKVCache(8, 16, 2, 64, dtype=torch.float16, device="cuda")
    first = torch.randn(4, 2, 64, device="cuda")
    cache.write([0], 0, first, first)
    snap, _ = cache.gather([0], 4)
    cache.write([0], 4, first * 50, first * 50)
    again, _ = cache.gather([0], 4)
    assert torch.equal(snap, again)
    k = torch.randn(20, 2, 64, device="cuda")
    with pytest.raises(IndexError, match="position 16 needs logical block 1"):
        cache.write([1], 0, k, k)
    # helios writes the positions before the failing one
    got, _ = cache.gather([1], 16)
    ref = QuantizedPagedKVCache(8, 16, 2, 64, dtype=torch.float16, device="cuda")
    ref.write([1], 0, k[:16], k[:16])
    want, _ = ref.gather([1], 16)
    assert torch.equal(got, want)


def test_copy_block_moves_scales():
    """reference tests/quant/test_kv_quant.py:112-131."""
    cache = QuantizedPagedKVCache(8, 16, 2, 64, dtype=torch.float16, device="cuda")
    large = torch.randn(16, 2, 64, device="cuda") * 1000
    small = torch.randn(16, 2, 64, device="cuda") * 0.001
    cache.write([0], 0, large, large)
    cache.write([1], 0, small, small)
    cache.copy_block(0, 1)
    a, _ = cache.gather([0], 16)
    b, _ = cache.gather([1], 16)
    assert torch.equal(a, b) and b.abs().max().item() > 100


def test_copy_blocks_all_layers_one_launch():
    caches = [PagedKVCache(10, 16, 2, 32, dtype=torch.float16, device="cuda") for _ in range(3)]
    for c in caches:
        c.k_cache.normal_()
        c.v_cache.normal_()
    before = [(c.k_cache.clone(), c.v_cache.clone()) for c in caches]
    pairs = [(1, 4), (2, 5), (4, 9)]  # (4, 9) reads a block written earlier in the list
    copy_blocks(caches, pairs)
    for (k0, v0), c in zip(before, caches):
        kk, vv = k0.clone(), v0.clone()
        for s, d in pairs:  # sequential semantics
            kk[d] = kk[s]
            vv[d] = vv[s]
        assert torch.equal(c.k_cache, kk) and torch.equal(c.v_cache, vv)


def _rope_tables(max_pos, d, theta=10000.0):
    """helios' build_rope_cache (exec/model.py:117-132), evaluated by torch."""
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    freqs = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv)
    return freqs.cos(), freqs.sin()


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_rope_fused_int8_write_is_bit_exact(scale_dtype):
    """K rotated by its position and quantized in one pass equals helios'
    apply_rope followed by the quantizing write, bit for bit; V untouched."""
    gen = torch.Generator().manual_seed(7)
    H, D, bs, nb = 8, 128, 16, 64
    qlens, starts = [5, 19, 1], [0, 30, 200]
    perm = np.random.default_rng(7).permutation(nb)
    tables = [[int(x) for x in perm[16 * i:16 * i + 16]] for i in range(3)]
    cos, sin = _rope_tables(512, D)
    k = (torch.randn(sum(qlens), H, D, generator=gen) * 2).half()
    v = torch.randn(sum(qlens), H, D, generator=gen).half()
    cache = QuantizedPagedKVCache(nb, bs, H, D, dtype=torch.float16, device="cuda", scale_dtype=scale_dtype)
    write_kv(cache, tables, starts, k.cuda(), v.cuda(), query_lens=qlens, rope=(cos.cuda(), sin.cuda()))
    pool = R.PagedPool(nb, bs, H, D, np.float32, quantized=True,
                       scale_dtype=np.float16 if scale_dtype == torch.float16 else np.float32)
    lo = 0
    for t, n, s0 in zip(tables, qlens, starts):
        pos = np.arange(s0, s0 + n)
        kr = R.apply_rope(k[lo:lo + n].numpy(), cos.numpy(), sin.numpy(), pos)
        pool.write(t, s0, kr, v[lo:lo + n].float().numpy())
        lo += n
    torch.cuda.synchronize()
    assert np.array_equal(to_np(cache.k_cache), pool.k)
    assert np.array_equal(to_np(cache.k_scale), pool.k_scale)
    assert np.array_equal(to_np(cache.v_cache), pool.v)
    assert np.array_equal(to_np(cache.v_scale), pool.v_scale)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_rope_fused_fp_write_matches_oracle(dtype):
    gen = torch.Generator().manual_seed(8)
    H, D, bs, nb = 2, 64, 16, 16
    qlens, starts = [17, 3], [5, 60]
    tables = [[3, 9, 1], [7, 2, 11, 4, 0]]
    cos, sin = _rope_tables(128, D)
    k = torch.randn(sum(qlens), H, D, generator=gen).to(dtype)
    v = torch.randn(sum(qlens), H, D, generator=gen).to(dtype)
    cache = PagedKVCache(nb, bs, H, D, dtype=dtype, device="cuda")
    write_kv(cache, tables, starts, k.cuda(), v.cuda(), query_lens=qlens, rope=(cos.cuda(), sin.cuda()))
    lo = 0
    got_k, got_v = cache.k_cache.cpu(), cache.v_cache.cpu()
    for t, n, s0 in zip(tables, qlens, starts):
        kr = torch.from_numpy(R.apply_rope(k[lo:lo + n].float().numpy(), cos.numpy(), sin.numpy(),
                                           np.arange(s0, s0 + n))).to(dtype)
        for i in range(n):
            p = s0 + i
            blk, off = t[p // bs], p % bs
            assert torch.equal(got_k[blk, :, off, :], kr[i])
            assert torch.equal(got_v[blk, :, off, :], v[lo + i])
        lo += n


def test_rope_positions_past_the_table_are_skipped():
    H, D, bs = 1, 32, 16
    cos, sin = _rope_tables(20, D)            # rows for positions 0..19 only
    cache = PagedKVCache(4, bs, H, D, dtype=torch.float32, device="cuda")
    k = torch.ones(6, H, D, device="cuda")
    write_kv(cache, [[0, 1]], [16], k, k, rope=(cos.cuda(), sin.cuda()))   # positions 16..21
    got = cache.k_cache.cpu()
    assert torch.count_nonzero(got[1, 0, :4]) == 4 * D       # positions 16..19 written
    assert torch.count_nonzero(got[1, 0, 4:6]) == 0          # 20, 21 have no table row
    with pytest.raises(ValueError):
        write_kv(cache, [[0, 1]], [0], k, k, rope=(cos.cuda(), sin.cuda()[:, :3]))
