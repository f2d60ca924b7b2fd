"""GPU parity of the paged decode / verify kernel (hpa_paged_decode) against
the oracle, on seeded inputs.

Tolerances (stated by the build's target): fp16 output max-abs <= 2e-3 against
a float64 reference computed from the same rounded inputs (int8 values
dequantised with the stored scales); bf16 gets one bf16 half-ulp of the
reference (|ref| * 2^-8) on top, since rounding the output to bf16 alone
exceeds 2e-3 once |out| > 0.5; fp32 KV (the toy-model path) <= 2e-5.  Batch-order invariance is asserted bit-exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helios_amd import (
    PagedKVCache,
    QuantizedPagedKVCache,
    paged_attention_decode,
    paged_attention_decode_batched,
    paged_attention_decode_hip,
    paged_attention_varlen,
    paged_attention_verify_batched,
)
from oracle import paged_ref as R
from tests.gpu_util import dev, fill_cache, max_abs, pool_dequantized, pool_of, ragged_tables, to_np

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 2e-3, torch.float32: 2e-5}


def _tol(dtype, want):
    t = TOL[dtype]
    if dtype == torch.bfloat16:
        return t + np.abs(want) * 2.0 ** -8
    return t


def _check(got: torch.Tensor, want: np.ndarray, dtype, what=""):
    g = to_np(got).astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - want)
    bound = _tol(dtype, want)
    assert (err <= bound).all(), f"{what}: max-abs {err.max():.3e}"


def _case(seed, n_seqs, lens, Hq, Hkv, D, bs, dtype, quant=False, scale_dtype=torch.float16,
          q_per_seq=1, extra_blocks=3):
    gen = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    nb = sum((c + bs - 1) // bs for c in lens) + extra_blocks
    if quant:
        cache = QuantizedPagedKVCache(nb, bs, Hkv, D, dtype=dtype, device="cuda",
                                      scale_dtype=scale_dtype)
    else:
        cache = PagedKVCache(nb, bs, Hkv, D, dtype=dtype, device="cuda")
    fill_cache(cache, gen)
    tables = ragged_tables(rng, lens, bs, nb)
    q = torch.randn(n_seqs * q_per_seq, Hq, D, generator=gen).to(dtype).to(dev())
    return cache, tables, q


def _oracle_decode(cache, q, tables, lens, scale=None, q_per_seq=1):
    pool = pool_of(cache)
    qn = to_np(q).astype(np.float32)
    if q_per_seq == 1:
        return R.paged_decode_batched(qn, pool, tables, lens, scale)
    return R.paged_verify_batched(qn, pool, tables, lens, q_per_seq, scale)


@pytest.mark.parametrize("n_seqs", [1, 4, 17])
@pytest.mark.parametrize("block_size", [16, 32])
def test_decode_matches_oracle_reference_shapes(n_seqs, block_size):
    """Shapes of reference tests/parity/test_triton_parity.py:50-86: ragged
    contexts bs*(i%3+1) - (i%bs), Hq 8 / Hkv 2 / D 64, fp16, tables strided
    by 7 through a 256-block pool."""
    torch.manual_seed(0)
    n_kv, n_q, D, n_blocks = 2, 8, 64, 256
    cache = PagedKVCache(n_blocks, block_size, n_kv, D, dtype=torch.float16, device="cuda")
    cache.k_cache.normal_()
    cache.v_cache.normal_()
    lens, tables, used = [], [], 0
    for i in range(n_seqs):
        ctx = max(1, block_size * (i % 3 + 1) - (i % block_size))
        need = (ctx + block_size - 1) // block_size
        tables.append([(used + j * 7) % n_blocks for j in range(need)])
        used += need
        lens.append(ctx)
    q = torch.randn(n_seqs, n_q, D, dtype=torch.float16, device="cuda")
    got = paged_attention_decode_batched(q, cache, tables, lens, 1.0 / math.sqrt(D))
    _check(got, _oracle_decode(cache, q, tables, lens, 1.0 / math.sqrt(D)), torch.float16)
    raw = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tables, lens)
    assert torch.equal(raw, got)


def test_decode_is_order_invariant_bitwise():
    """reference tests/parity/test_triton_parity.py:89-112, but bit-exact."""
    torch.manual_seed(1)
    cache = PagedKVCache(64, 16, 2, 64, dtype=torch.float16, device="cuda")
    cache.k_cache.normal_()
    cache.v_cache.normal_()
    tables, lens = [[0, 1], [5, 2, 9], [3]], [20, 40, 7]
    q = torch.randn(3, 4, 64, dtype=torch.float16, device="cuda")
    fwd = paged_attention_decode_batched(q, cache, tables, lens)
    order = [2, 0, 1]
    rev = paged_attention_decode_batched(q[order], cache, [tables[i] for i in order],
                                         [lens[i] for i in order])
    assert torch.equal(rev, fwd[order])
    _check(fwd, _oracle_decode(cache, q, tables, lens), torch.float16)


def test_single_token_context():
    """reference tests/parity/test_triton_parity.py:115-124."""
    torch.manual_seed(2)
    cache = PagedKVCache(16, 16, 1, 64, dtype=torch.float16, device="cuda")
    cache.k_cache.normal_()
    cache.v_cache.normal_()
    q = torch.randn(1, 1, 64, dtype=torch.float16, device="cuda")
    got = paged_attention_decode_batched(q, cache, [[0]], [1])
    # one key: the output is that key's value row exactly
    assert torch.equal(got[0, 0], cache.v_cache[0, 0, 0])


def test_config1_toy_decode_fp32():
    """Config 1: fp32, batch 4, Hq 4 / Hkv 2, D 64, bs 16, ctx U[17,100],
    blocks a seeded permutation of a 64-block pool."""
    rng = np.random.default_rng(0)
    gen = torch.Generator().manual_seed(0)
    lens = [int(x) for x in rng.integers(17, 101, size=4)]
    cache = PagedKVCache(64, 16, 2, 64, dtype=torch.float32, device="cuda")
    fill_cache(cache, gen)
    tables = ragged_tables(rng, lens, 16, 64)
    q = torch.randn(4, 4, 64, generator=gen).to(dev())
    got = paged_attention_decode_batched(q, cache, tables, lens, 1.0 / 8)
    want = _oracle_decode(cache, q, tables, lens, 1.0 / 8)
    _check(got, want, torch.float32, "cfg1")
    # and the reference's own dense oracle per sequence
    for i, (t, c) in enumerate(zip(tables, lens)):
        k, v = pool_of(cache).gather(t, c)
        np.testing.assert_allclose(to_np(got[i]), R.attention_decode(to_np(q[i]), k, v, 1 / 8),
                                   atol=2e-5)


@pytest.mark.parametrize("D", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_head_dims_and_dtypes(D, dtype):
    lens = [1, 15, 16, 17, 33, 100, 257]
    cache, tables, q = _case(10 + D, len(lens), lens, 4, 2, D, 16, dtype)
    got = paged_attention_decode_batched(q, cache, tables, lens)
    _check(got, _oracle_decode(cache, q, tables, lens), dtype, f"D={D} {dtype}")


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("dtype,T", [(torch.float16, 1), (torch.bfloat16, 1), (torch.float16, 5),
                                     (torch.bfloat16, 12)])
def test_head_dim_256_split_k(dtype, T, quant):
    """head_dim 256 keeps one step of loads in flight and merges one piece
    per round trip; long contexts cut into many 128-token pieces exercise
    the merge, and 4 * T rows per KV head the one-, two- and four-tile
    forms (no other kernel takes head_dim 256)."""
    print(f"head_dim 256, {dtype}, q_per_seq {T}, int8 {quant}", flush=True)
    lens = [T, 40, 700, 2100, 4500]
    cache, tables, q = _case(260 + T, len(lens), lens, 8, 2, 256, 16, dtype, quant=quant, q_per_seq=T)
    ks, vs = cache._scales()
    got = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tables, lens, 1 / 16, ks, vs,
                                     q_per_seq=T, part_tokens=128)
    _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=T, scale=1 / 16), dtype, "D=256")


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_int8_kv(scale_dtype, D, dtype):
    lens = [3, 16, 31, 64, 200, 513]
    cache, tables, q = _case(20 + D, len(lens), lens, 8, 2, D, 16, dtype, quant=True,
                             scale_dtype=scale_dtype)
    got = paged_attention_decode_batched(q, cache, tables, lens)
    _check(got, _oracle_decode(cache, q, tables, lens), dtype, f"int8 D={D}")


@pytest.mark.parametrize("T,scale_dtype", [(1, torch.float16), (3, torch.float16), (5, torch.float16),
                                           (8, torch.float32), (12, torch.float16)])
def test_bf16_queries_over_int8_pools(T, scale_dtype):
    """bf16 queries over an int8 pool run the fp16 MFMA form: each query
    row enters fp16 scaled by the power of two that brings its largest
    element into [2^14, 2^15).  Rows of ordinary magnitude, rows of 2^14,
    rows with elements down to 2^-30 and rows of 2^-40 throughout (all below
    fp16's range unscaled) match the oracle; 4 * T rows per KV head cover the decode kernel's one- and
    two-tile forms and the wide verify kernel (20, 32 and 48 rows)."""
    print(f"bf16 queries over int8, q_per_seq {T}, scales {scale_dtype}", flush=True)
    lens = [T, 40, 300, 1100]
    cache, tables, q = _case(170 + T, len(lens), lens, 16, 4, 128, 16, torch.bfloat16, quant=True,
                             scale_dtype=scale_dtype, q_per_seq=T)
    q = q.float()
    q[0::3] *= 2.0 ** 17 / 8  # large rows: scores in the thousands, one key dominates
    q[1::3, :, ::2] *= 2.0 ** -28  # tiny elements next to ordinary ones
    q[2::3, ::2] *= 2.0 ** -40  # whole heads far below fp16's range
    q = q.to(torch.bfloat16)
    got = paged_attention_verify_batched(q, cache, tables, lens, T) if T > 1 else \
        paged_attention_decode_batched(q, cache, tables, lens)
    _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=T), torch.bfloat16, "bf16 over int8")


def _scale_range(cache, seed):
    """Key scales from 2^-14 to 2^4 and value scales from 2^-14 to 2^-6,
    drawn per block (the payload keeps its bytes)."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    for sc, top in ((cache.k_scale, 5), (cache.v_scale, -5)):
        e = torch.randint(-14, top, (sc.shape[0], 1, 1), generator=gen, device="cuda").float()
        sc.copy_((torch.rand(sc.shape, generator=gen, device="cuda") * 0.5 + 0.5) * torch.exp2(e))


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_int8_decode_few_keys_large_values(scale_dtype):
    """400 contexts of 1-5 keys with value scales doubled (values up to ~8):
    with so few keys no rounding of a single weight averages out, so fp16
    weights P * vs would leave up to 2^-11 |v| in the output.  Outputs below
    4 in magnitude (where rounding the output itself costs <= 2^-12 * 4)
    stay within 2e-3; larger ones within 2e-3 plus their own half-ulp."""
    print(f"int8 decode, 1-5 keys, scales {scale_dtype}", flush=True)
    rng = np.random.default_rng(7)
    lens = [int(x) for x in rng.integers(1, 6, size=400)]
    cache, tables, q = _case(9, len(lens), lens, 32, 8, 128, 16, torch.float16, quant=True,
                             scale_dtype=scale_dtype)
    cache.v_scale.mul_(2.0)
    got = to_np(paged_attention_decode_batched(q, cache, tables, lens)).astype(np.float64)
    want = _oracle_decode(cache, q, tables, lens)
    err = np.abs(got - want)
    small = np.abs(want) < 4
    assert err[small].max() <= 2e-3, f"|out| < 4: max-abs {err[small].max():.3e}"
    assert (err <= 2e-3 + np.abs(want) * 2.0 ** -11).all(), f"max-abs {err.max():.3e}"


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_int8_decode_scale_range(scale_dtype):
    """300 contexts up to 1500 keys with key scales up to 2^4: scores reach
    thousands, so an offset in the fp16 key operand that is large next to
    the key bytes would leave its fp32 rounding, times the scale, in the
    softmax weights."""
    print(f"int8 decode, scale range, scales {scale_dtype}", flush=True)
    rng = np.random.default_rng(150)
    lens = [int(x) for x in rng.integers(1, 1500, size=300)]
    cache, tables, q = _case(150, len(lens), lens, 32, 8, 128, 16, torch.float16, quant=True,
                             scale_dtype=scale_dtype)
    _scale_range(cache, 151)
    got = paged_attention_decode_batched(q, cache, tables, lens)
    _check(got, _oracle_decode(cache, q, tables, lens), torch.float16, "int8 decode, scale range")


@pytest.mark.parametrize("Hq,Hkv,T", [(32, 8, 3), (14, 2, 1), (14, 2, 3), (8, 1, 5), (16, 1, 4), (2, 2, 2)])
@pytest.mark.parametrize("quant", [False, True])
def test_verify_rows_and_gqa_groups(Hq, Hkv, T, quant):
    """Multi-token verify (q_per_seq = T, causal among the T tokens) over
    every row-tile width (G*T up to 64)."""
    lens = [T, T + 5, 40, 129, 300]
    cache, tables, q = _case(30 + Hq + T, len(lens), lens, Hq, Hkv, 128, 16, torch.float16,
                             quant=quant, q_per_seq=T)
    got = paged_attention_verify_batched(q, cache, tables, lens, T)
    want = _oracle_decode(cache, q, tables, lens, q_per_seq=T)
    _check(got, want, torch.float16, f"verify {Hq}/{Hkv}x{T}")


@pytest.mark.parametrize("Hq,Hkv,T,D,dtype", [(8, 2, 5, 128, torch.bfloat16), (16, 4, 8, 64, torch.float16),
                                              (14, 2, 3, 128, torch.float16)])
def test_verify_17_to_32_rows_on_fp_pools_runs_the_mfma_prefill_kernel(Hq, Hkv, T, D, dtype):
    """17-32 query rows per KV head over fp16 / bf16 pools also go to the
    MFMA prefill kernel (the decode kernel's two-row-tile instantiation
    spills registers): bit for bit the same tokens through
    paged_attention_varlen, and the oracle."""
    print(f"verify {Hq}/{Hkv}x{T} D {D} {dtype} on the MFMA kernel", flush=True)
    lens = [T, T + 5, 40, 129, 300, 1500]
    cache, tables, q = _case(90 + Hq + T, len(lens), lens, Hq, Hkv, D, 16, dtype, q_per_seq=T)
    got = paged_attention_verify_batched(q, cache, tables, lens, T)
    same = paged_attention_varlen(q, cache, tables, [T] * len(lens), [c - T for c in lens], lens)
    assert torch.equal(got, same)
    want = R.paged_verify_batched(to_np(q).astype(np.float32), pool_of(cache), tables, lens, T)
    _check(got, want, dtype, "17-32-row verify")


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("Hq,Hkv,T,D,dtype", [(32, 4, 8, 128, torch.float16), (16, 4, 9, 128, torch.float16),
                                              (8, 1, 5, 128, torch.float16), (8, 1, 6, 64, torch.bfloat16)])
def test_wide_verify_runs_the_mfma_prefill_kernel(Hq, Hkv, T, D, dtype, quant):
    """33-64 query rows per KV head go to the MFMA prefill kernel: the
    verify equals, bit for bit, the same tokens through paged_attention_varlen
    (start = context - T), and the oracle.  Queries over int8 pools take the
    register-dequantising verify kernel instead, which keeps the dequantised
    values in fp32 as the decode kernel does: it matches the exact oracle,
    and for fp16, to the bound, the oracle over the dequantised values rounded
    to the compute dtype as helios' gather hands them over
    (paged_attn.py:213-235).  Rounding those values to bf16 moves scores by
    more than the bound, so bf16 is held to the exact oracle alone."""
    print(f"wide verify {Hq}/{Hkv}x{T} D {D} {dtype} int8 {quant}", flush=True)
    lens = [T, T + 5, 40, 129, 300]
    cache, tables, q = _case(80 + Hq + T, len(lens), lens, Hq, Hkv, D, 16, dtype,
                             quant=quant, q_per_seq=T)
    got = paged_attention_verify_batched(q, cache, tables, lens, T)
    if quant:
        _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=T), dtype, "int8 wide verify")
        if dtype == torch.bfloat16:
            return
    else:
        same = paged_attention_varlen(q, cache, tables, [T] * len(lens), [c - T for c in lens], lens)
        assert torch.equal(got, same)
    pool = pool_dequantized(cache) if quant else pool_of(cache)
    want = R.paged_verify_batched(to_np(q).astype(np.float32), pool, tables, lens, T)
    _check(got, want, dtype, "wide verify")


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("Hq,Hkv,T,D", [(8, 1, 5, 128), (32, 4, 8, 128), (14, 2, 5, 64), (16, 2, 7, 64),
                                        (32, 8, 16, 128), (8, 1, 3, 128), (14, 2, 3, 64), (32, 8, 8, 128)])
def test_int8_wide_verify_dequantises_in_registers(Hq, Hkv, T, D, scale_dtype):
    """33-64 rows per KV head (17-32 in test_verify_rows_and_gqa_groups),
    fp16 queries over an int8 pool: the verify
    kernel that turns each wave's own int8 operands into fp16 in registers
    (1152 + x, offsets removed algebraically) against the oracle on the
    exactly dequantised values.  Contexts cover a context equal to the token
    count, steps ending mid-block and mid-step, one 16-key half of a step
    past the context, and tables longer than 128 blocks.  Two calls give
    the same bits."""
    print(f"int8 verify in registers: {Hq}/{Hkv} x {T}, D {D}, scales {scale_dtype}", flush=True)
    lens = [T, T + 1, 33, 48, 64 + T, 300, 2100 + T]
    cache, tables, q = _case(140 + Hq + T + D, len(lens), lens, Hq, Hkv, D, 16, torch.float16,
                             quant=True, scale_dtype=scale_dtype, q_per_seq=T)
    got = paged_attention_verify_batched(q, cache, tables, lens, T)
    torch.cuda.synchronize()
    _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=T), torch.float16, "int8 verify in registers")
    again = paged_attention_verify_batched(q, cache, tables, lens, T)
    assert torch.equal(got, again)


def test_int8_wide_verify_cuts_long_units():
    """A few long contexts: the verify kernel cuts units longer than their
    XCD's steps per resident workgroup in two, and the piece that finishes
    second merges both in piece order.  The result matches the oracle, two
    calls give the same bits, and the arrival counters are back at zero
    afterwards: a decode on the same workspace, whose own split-K counts on
    them, still matches the oracle."""
    print("int8 verify, cut units", flush=True)
    T = 12
    lens = [T, 900, 4000, 7003, 2500]
    cache, tables, q = _case(160, len(lens), lens, 32, 8, 128, 16, torch.float16, quant=True, q_per_seq=T)
    got = paged_attention_verify_batched(q, cache, tables, lens, T)
    _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=T), torch.float16, "cut units")
    again = paged_attention_verify_batched(q, cache, tables, lens, T)
    assert torch.equal(got, again)
    qd = q[T - 1::T].contiguous()
    dec = paged_attention_decode_batched(qd, cache, tables, lens)
    _check(dec, _oracle_decode(cache, qd, tables, lens), torch.float16, "decode after cut verify")


def test_int8_wide_verify_many_sequences_and_scale_range():
    """Config 5's head shape with 12 speculative tokens (48 rows per KV
    head) over 300 sequences, so workgroups run longest-first over several
    rounds, with key scales from 2^-14 to 2^4 and value scales from 2^-14
    to 2^-6 on different blocks (values stay below 2, where fp16 rounds the
    output within the bound)."""
    print("int8 verify in registers: 300 sequences", flush=True)
    rng = np.random.default_rng(150)
    T = 12
    lens = [int(x) for x in rng.integers(T, 1500, size=300)]
    cache, tables, q = _case(150, len(lens), lens, 32, 8, 128, 16, torch.float16, quant=True, q_per_seq=T)
    _scale_range(cache, 151)
    got = paged_attention_verify_batched(q, cache, tables, lens, T)
    _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=T), torch.float16, "int8 verify, 300 sequences")


@pytest.mark.parametrize("D,bs,dtype", [(128, 8, torch.float16), (32, 16, torch.float16),
                                        (64, 16, torch.float32)])
def test_wide_verify_on_shapes_the_mfma_kernel_does_not_take(D, bs, dtype):
    """33-64 rows per KV head with block size 8, head_dim 32 or fp32 queries
    stay on the decode kernel (four row tiles)."""
    print(f"wide verify on the decode kernel: D {D}, block {bs}, {dtype}", flush=True)
    T, lens = 5, [5, 12, 40, 129, 300]
    cache, tables, q = _case(90 + D + bs, len(lens), lens, 8, 1, D, bs, dtype, q_per_seq=T)
    got = paged_attention_verify_batched(q, cache, tables, lens, T)
    _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=T), dtype, f"decode-kernel verify D={D}")


@pytest.mark.parametrize("part", [128, 256, 512])
def test_split_k_long_contexts(part):
    """Contexts spanning many partitions (split-K + merge), including
    lengths that end mid-step and mid-partition."""
    lens = [1, 127, 128, 129, 1000, 4096, 5001]
    cache, tables, q = _case(40 + part, len(lens), lens, 14, 2, 64, 16, torch.float16)
    k, v = cache.k_cache, cache.v_cache
    got = paged_attention_decode_hip(q, k, v, tables, lens, part_tokens=part)
    _check(got, _oracle_decode(cache, q, tables, lens), torch.float16, f"part {part}")
    # the partition size changes the summation order only
    other = paged_attention_decode_hip(q, k, v, tables, lens, part_tokens=1024)
    assert max_abs(to_np(got), to_np(other)) <= 2e-3


def test_split_k_int8_verify():
    lens = [2000, 3, 4500, 777]
    cache, tables, q = _case(50, len(lens), lens, 32, 8, 128, 16, torch.float16, quant=True,
                             q_per_seq=3)
    got = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tables, lens,
                                     k_scale=cache.k_scale, v_scale=cache.v_scale, q_per_seq=3,
                                     part_tokens=256)
    _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=3), torch.float16)


def test_block_size_4_and_non_contiguous_tables():
    """reference tests/parity/test_parity.py uses 4-token blocks."""
    lens = [1, 4, 5, 11, 33, 70]
    cache, tables, q = _case(60, len(lens), lens, 4, 2, 32, 4, torch.float32)
    got = paged_attention_decode_batched(q, cache, tables, lens)
    _check(got, _oracle_decode(cache, q, tables, lens), torch.float32)


def test_single_sequence_api_and_empty_context():
    cache, tables, q = _case(70, 1, [45], 4, 2, 64, 16, torch.float16)
    got = paged_attention_decode(q[0], cache, tables[0], 45)
    _check(got[None], _oracle_decode(cache, q, tables, [45]), torch.float16)
    # an empty context is defined as zeros (helios would give NaN)
    z = paged_attention_decode_batched(q, cache, tables, [0])
    assert torch.count_nonzero(z) == 0


def test_device_tensor_tables_match_list_tables():
    lens = [50, 700, 3]
    cache, tables, q = _case(80, 3, lens, 8, 2, 64, 16, torch.float16)
    width = max(len(t) for t in tables)
    tt = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.int32, device="cuda")
    lt = torch.tensor(lens, dtype=torch.int32, device="cuda")
    a = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tables, lens)
    b = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tt, lt, max_context_len=700)
    assert torch.equal(a, b)


@pytest.mark.parametrize("quant", [False, True])
def test_stream_k_many_pieces_and_empty_units(quant):
    """A 32-token slice floor cuts the long units into hundreds of pieces
    (more than the merge keeps in LDS) and puts empty contexts between cut
    units; empty contexts give zeros, the rest match the oracle."""
    lens = [0, 5000, 0, 1, 33, 2049, 0]
    cache, tables, q = _case(90, len(lens), lens, 8, 2, 64, 16, torch.float16, quant=quant)
    ks = cache.k_scale if quant else None
    vs = cache.v_scale if quant else None
    got = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tables, lens,
                                     k_scale=ks, v_scale=vs, part_tokens=32)
    live = [i for i, c in enumerate(lens) if c > 0]
    want = _oracle_decode(cache, q[live], [tables[i] for i in live], [lens[i] for i in live])
    _check(got[live], want, torch.float16, "stream-K pieces")
    dead = [i for i, c in enumerate(lens) if c == 0]
    assert torch.count_nonzero(got[dead]) == 0
    # the slice floor only reorders the summation
    other = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tables, lens,
                                       k_scale=ks, v_scale=vs)
    assert max_abs(to_np(got), to_np(other)) <= 2e-3


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("Hq,Hkv,T,D,dtype", [(14, 2, 13, 64, torch.float16), (32, 8, 20, 128, torch.float16),
                                              (8, 1, 17, 128, torch.bfloat16)])
def test_verify_beyond_64_rows_per_kv_head(Hq, Hkv, T, D, dtype, quant):
    """Any gamma verifies, as helios' runner does (exec/runner.py:330-362):
    Qwen's G = 7 with gamma = 12 (91 rows per KV head), G = 4 with 20 tokens
    (80 rows) and G = 8 with 17 (136 rows, more than one 128-row tile) run on
    the MFMA prefill kernel and equal paged_attention_varlen over the same
    tokens bit for bit, and the oracle."""
    print(f"verify > 64 rows: {Hq}/{Hkv} x {T}, D {D}, {dtype}, int8 {quant}", flush=True)
    lens = [T, T + 3, 64, 300, 1100]
    cache, tables, q = _case(110 + Hq + T, len(lens), lens, Hq, Hkv, D, 16, dtype, quant=quant, q_per_seq=T)
    got = paged_attention_verify_batched(q, cache, tables, lens, T)
    same = paged_attention_varlen(q, cache, tables, [T] * len(lens), [c - T for c in lens], lens)
    assert torch.equal(got, same)
    pool = pool_dequantized(cache) if quant else pool_of(cache)
    want = R.paged_verify_batched(to_np(q).astype(np.float32), pool, tables, lens, T)
    _check(got, want, dtype, "verify > 64 rows")


@pytest.mark.parametrize("D,bs,dtype", [(32, 16, torch.float16), (128, 8, torch.float16), (64, 16, torch.float32)])
def test_verify_beyond_64_rows_on_the_generic_prefill_kernel(D, bs, dtype):
    """More than 64 rows on shapes the MFMA kernel does not take (head_dim 32,
    block size 8, fp32) run on the generic prefill kernel's verify mode."""
    print(f"verify > 64 rows, generic kernel: D {D}, block {bs}, {dtype}", flush=True)
    T, lens = 9, [9, 20, 77, 300]
    cache, tables, q = _case(120 + D + bs, len(lens), lens, 16, 2, D, bs, dtype, q_per_seq=T)
    got = paged_attention_verify_batched(q, cache, tables, lens, T)
    _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=T), dtype, f"generic verify D={D}")
    same = paged_attention_varlen(q, cache, tables, [T] * len(lens), [c - T for c in lens], lens)
    assert torch.equal(got, same)


def test_permuted_query_layouts_give_row_major_results():
    """A dense but permuted query ([T, Hq, D] made by transposing [Hq, T, D])
    is attended as its values say, and the result is a row-major tensor, for
    decode, verify and the ragged prefill alike."""
    lens = [40, 77, 300]
    cache, tables, q = _case(130, len(lens), lens, 8, 2, 64, 16, torch.float16, q_per_seq=3)
    qp = q.permute(1, 0, 2).contiguous().permute(1, 0, 2)  # same values, strides (D, rows*D, 1)
    assert not qp.is_contiguous() and torch.equal(qp, q)
    v1 = paged_attention_verify_batched(qp, cache, tables, lens, 3)
    assert v1.is_contiguous() and torch.equal(v1, paged_attention_verify_batched(q, cache, tables, lens, 3))
    q1 = q[::3]
    q1p = q1.permute(1, 0, 2).contiguous().permute(1, 0, 2)
    d1 = paged_attention_decode_batched(q1p, cache, tables, lens)
    assert d1.is_contiguous() and torch.equal(d1, paged_attention_decode_batched(q1.contiguous(), cache, tables, lens))
    p1 = paged_attention_varlen(qp, cache, tables, [3] * 3, [c - 3 for c in lens], lens)
    p0 = paged_attention_varlen(q, cache, tables, [3] * 3, [c - 3 for c in lens], lens)
    assert p1.is_contiguous() and torch.equal(p1, p0)
    _check(p1, _oracle_decode(cache, q, tables, lens, q_per_seq=3), torch.float16, "permuted varlen")


def test_context_above_the_launch_bound_is_honoured():
    """max_context_len only sizes the launch: a device-tensor context above
    it is attended in full (the result equals the call with the right bound),
    and list contexts reject a bound below their largest one."""
    lens = [50, 700, 3]
    cache, tables, q = _case(140, 3, lens, 8, 2, 64, 16, torch.float16)
    width = max(len(t) for t in tables)
    tt = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.int32, device="cuda")
    lt = torch.tensor(lens, dtype=torch.int32, device="cuda")
    right = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tt, lt, max_context_len=700)
    stale = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tt, lt, max_context_len=64)
    _check(stale, _oracle_decode(cache, q, tables, lens), torch.float16, "stale bound")
    assert max_abs(to_np(right), to_np(stale)) <= 2e-3
    with pytest.raises(ValueError, match="below a context"):
        paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tables, lens, max_context_len=64)


def test_metadata_tensors_are_validated():
    """int64, non-contiguous or misplaced metadata tensors are refused rather
    than read as int32 words."""
    lens = [50, 70]
    cache, tables, q = _case(150, 2, lens, 8, 2, 64, 16, torch.float16)
    width = max(len(t) for t in tables)
    tt = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.int32, device="cuda")
    lt = torch.tensor(lens, dtype=torch.int32, device="cuda")
    k, v = cache.k_cache, cache.v_cache
    with pytest.raises(ValueError, match="int32"):
        paged_attention_decode_hip(q, k, v, tt.long(), lt, max_context_len=70)
    with pytest.raises(ValueError, match="int32"):
        paged_attention_decode_hip(q, k, v, tt, lt.long(), max_context_len=70)
    with pytest.raises(ValueError, match="contiguous"):
        paged_attention_decode_hip(q, k, v, tt.t().contiguous().t(), lt, max_context_len=70)
    with pytest.raises(ValueError, match="is on cpu"):
        paged_attention_decode_hip(q, k, v, tt.cpu(), lt, max_context_len=70)
    with pytest.raises(ValueError, match="out must be contiguous"):
        paged_attention_decode_hip(q, k, v, tt, lt, max_context_len=70,
                                   out=torch.empty(8, 2, 64, dtype=torch.float16, device="cuda").transpose(0, 1))
    with pytest.raises(ValueError, match="sum to"):
        paged_attention_varlen(q, cache, tt, torch.tensor([1, 2], dtype=torch.int32), lt - 1, lt)


_F16, _B16, _F32 = torch.float16, torch.bfloat16, torch.float32
# (query dtype, int8 pool, scale dtype, head_dim, Hkv, G, tokens, part_tokens):
# every route of hpa_paged_decode at least once
_ROUTES = [
    (_F16, True, _F16, 128, 4, 4, 2, 0),      # int8 decode kernel, 8 rows
    (_B16, True, _F32, 64, 2, 4, 4, 64),      # bf16 over int8, 16 rows
    (_F16, True, _F16, 128, 2, 4, 5, 64),     # int8 verify kernel, 20 rows
    (_B16, True, _F32, 128, 1, 7, 4, 0),      # int8 verify kernel (bf16), 28 rows
    (_F16, True, _F32, 64, 2, 8, 6, 128),     # int8 verify kernel, 48 rows
    (_B16, True, _F16, 128, 4, 4, 16, 64),    # int8 verify kernel (bf16), 64 rows
    (_B16, True, _F32, 64, 2, 4, 6, 64),      # int8 verify kernel (bf16), head_dim 64, 24 rows
    (_F16, True, _F16, 128, 2, 7, 12, 0),     # int8, 84 rows: MFMA prefill verify
    (_B16, True, _F16, 256, 2, 4, 5, 64),     # int8 head_dim 256, two tiles
    (_F16, False, None, 128, 4, 4, 3, 64),    # fp16 decode kernel, 12 rows
    (_B16, False, None, 128, 2, 7, 4, 0),     # bf16 pool, 28 rows: MFMA prefill
    (_F16, False, None, 64, 1, 8, 8, 128),    # 64 rows: MFMA prefill
    (_F16, False, None, 128, 2, 8, 20, 64),   # 160 rows: MFMA prefill, two tiles
    (_F16, False, None, 256, 2, 2, 12, 64),   # head_dim 256, 24 rows: decode kernel
    (_B16, False, None, 256, 1, 7, 1, 0),     # head_dim 256 decode
]


@pytest.mark.parametrize("case", range(len(_ROUTES)))
def test_every_route_on_random_contexts(case):
    """Every route of hpa_paged_decode -- the decode kernel's one-, two- and
    four-tile forms, the int8 verify kernel, the MFMA prefill kernel's
    verify mode -- on seeded random contexts up to 2 500 keys, cut into
    pieces by a small part_tokens where given.  Int8 verifies above 64 rows
    run over the dequantised values rounded to the compute dtype (helios'
    gather), so they are held to that oracle; everything else to the exact
    one."""
    dtype, quant, scale_dtype, D, Hkv, G, T, part = _ROUTES[case]
    rng = np.random.default_rng(1000 + case)
    n = int(rng.integers(2, 7))
    lens = sorted(int(x) for x in rng.integers(T, 2500, size=n))
    rows = G * T
    print(f"case {case}: {dtype} int8 {quant} ({scale_dtype}) D {D} Hkv {Hkv} G {G} T {T} rows {rows} "
          f"lens {lens} part {part}", flush=True)
    cache, tables, q = _case(2000 + case, n, lens, G * Hkv, Hkv, D, 16, dtype, quant=quant,
                             scale_dtype=scale_dtype or torch.float16, q_per_seq=T)
    ks, vs = cache._scales()
    got = paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tables, lens, 1 / math.sqrt(D), ks, vs,
                                     q_per_seq=T, part_tokens=part)
    pool = pool_dequantized(cache) if quant and rows > 64 else pool_of(cache)
    qn = to_np(q).astype(np.float32)
    want = (R.paged_decode_batched(qn, pool, tables, lens, 1 / math.sqrt(D)) if T == 1 else
            R.paged_verify_batched(qn, pool, tables, lens, T, 1 / math.sqrt(D)))
    _check(got, want, dtype, f"route case {case}")
