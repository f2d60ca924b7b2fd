"""Pins the CPU oracle (oracle/paged_ref.py) before it is trusted as the
checker of the GPU kernels.

Every check here is independent of the formula it checks: hand-derived
integer answers, an exact float64 division, brute-force loops in pure Python,
and the reference's own test cases (reference tests/parity/test_parity.py,
tests/quant/test_kv_quant.py).  The last section plants plausible mistakes
in copies of the oracle and shows that these checks catch them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_ref as R

RNG = np.random.default_rng


# ------------------------------------------------------------------ quantize


def test_quantize_round_half_even_ties():
    # absmax 127 makes s exactly 1.0, so x / s = x and every .5 is a tie.
    x = np.array([[127.0, 2.5, -2.5, 3.5, -3.5, 0.5, -0.5, 1.5, 126.5, -126.5, 0.49999997]], np.float32)
    q, s = R.quantize(x)
    assert s.dtype == np.float32 and s[0] == 1.0
    assert q.tolist() == [[127, 2, -2, 4, -4, 0, 0, 2, 126, -126, 0]]


def test_quantize_zero_row_uses_the_clamp():
    q, s = R.quantize(np.zeros((1, 8), np.float32))
    assert (q == 0).all()
    assert s[0] == np.float32(np.float32(1e-8) / np.float32(127.0))
    # stored as fp16 this underflows to zero (helios stores fp16 scales)
    assert R.store_scale(s)[0] == 0


def test_quantize_extremes_hit_plus_minus_127():
    x = RNG(0).standard_normal((64, 4, 32)).astype(np.float32)
    q, s = R.quantize(x)
    am = np.abs(x).argmax(-1)
    top = np.take_along_axis(q, am[..., None], -1)[..., 0]
    assert (np.abs(top) == 127).all()
    assert q.min() >= -127 and q.max() <= 127


def test_quantize_uses_true_division_not_reciprocal():
    """Find inputs where fp32 x * (1/s) and x / s round to different integers;
    the oracle must follow the division (torch's `x / scale`), checked against
    an exact float64 quotient rounded once to fp32."""
    rng = RNG(1)
    hits = 0
    for _ in range(200):
        x = (rng.standard_normal((256, 64)) * rng.uniform(0.1, 10)).astype(np.float32)
        q, s = R.quantize(x)
        exact = (x.astype(np.float64) / s.astype(np.float64)[:, None]).astype(np.float32)
        want = np.clip(np.rint(exact), -127, 127).astype(np.int8)
        assert np.array_equal(q, want)
        recip = np.clip(np.rint(x * (np.float32(1) / s)[:, None]), -127, 127).astype(np.int8)
        hits += int((recip != want).sum())
    assert hits > 0, "no reciprocal/division disagreement found; the check would be vacuous"


def test_fp16_scale_storage_rounds_to_nearest_even():
    one = np.float32(1.0)
    tie_down = one + np.float32(2.0 ** -11)        # halfway 1 and 1+2^-10 -> 1 (even)
    tie_up = one + np.float32(3 * 2.0 ** -11)      # halfway 1+2^-10 and 1+2^-9 -> 1+2^-9
    got = R.store_scale(np.array([tie_down, tie_up], np.float32)).astype(np.float64)
    assert got.tolist() == [1.0, 1.0 + 2.0 ** -9]


def test_round_trip_bound_of_the_reference():
    """tests/quant/test_kv_quant.py:61-90: |err| <= s/2 + |q| |s - fp16(s)|."""
    rng = RNG(0)
    pool = R.PagedPool(8, 16, 2, 64, np.float32, quantized=True)
    k = rng.standard_normal((16, 2, 64)).astype(np.float32)
    v = rng.standard_normal((16, 2, 64)).astype(np.float32)
    pool.write([0], 0, k, v)
    gk, gv = pool.gather([0], 16)
    for got, want in ((gk, k), (gv, v)):
        s = np.abs(want).max(-1, keepdims=True) / np.float32(127.0)
        qi = np.abs(np.clip(np.rint(want / s), -127, 127))
        serr = np.abs(s - s.astype(np.float16).astype(np.float32))
        assert (np.abs(got - want) <= s / 2 + qi * serr + 1e-7).all()


# -------------------------------------------------------- pool / indexing


def test_write_gather_round_trip_through_scattered_blocks():
    """tests/parity/test_parity.py:134-142."""
    rng = RNG(2)
    pool = R.PagedPool(16, 4, 2, 8)
    k = rng.standard_normal((10, 2, 8)).astype(np.float32)
    v = rng.standard_normal((10, 2, 8)).astype(np.float32)
    pool.write([11, 2, 7], 0, k, v)
    gk, gv = pool.gather([11, 2, 7], 10)
    assert np.array_equal(gk, k) and np.array_equal(gv, v)
    # closed form: position p lives at block table[p // bs], offset p % bs
    for p in range(10):
        assert np.array_equal(pool.k[[11, 2, 7][p // 4], :, p % 4], k[p])


def test_gather_rejects_short_table():
    """tests/parity/test_parity.py:145-148."""
    pool = R.PagedPool(16, 4, 2, 8)
    with pytest.raises(IndexError, match="context_len 99 needs 25 blocks, have 1"):
        pool.gather([0], 99)


def test_write_out_of_range_raises_after_writing_the_prefix():
    """tests/quant/test_kv_quant.py:148-152, and helios writes positions
    before the failing one (paged_attn.py:74-85)."""
    pool = R.PagedPool(8, 16, 2, 64, quantized=True)
    k = RNG(3).standard_normal((20, 2, 64)).astype(np.float32)
    with pytest.raises(IndexError, match="position 16 needs logical block 1 but the sequence has only 1 blocks"):
        pool.write([0], 0, k, k)
    assert (pool.k[0] != 0).any()


def test_partial_block_write_leaves_neighbours():
    """tests/quant/test_kv_quant.py:134-145."""
    rng = RNG(0)
    pool = R.PagedPool(8, 16, 2, 64, quantized=True)
    first = rng.standard_normal((4, 2, 64)).astype(np.float32)
    pool.write([0], 0, first, first)
    snap, _ = pool.gather([0], 4)
    pool.write([0], 4, 50 * first, 50 * first)
    again, _ = pool.gather([0], 4)
    assert np.array_equal(snap, again)


def test_copy_block_moves_scales():
    """tests/quant/test_kv_quant.py:112-131."""
    rng = RNG(0)
    pool = R.PagedPool(8, 16, 2, 64, quantized=True)
    large = (rng.standard_normal((16, 2, 64)) * 1000).astype(np.float32)
    small = (rng.standard_normal((16, 2, 64)) * 0.001).astype(np.float32)
    pool.write([0], 0, large, large)
    pool.write([1], 0, small, small)
    pool.copy_block(0, 1)
    a, _ = pool.gather([0], 16)
    b, _ = pool.gather([1], 16)
    assert np.array_equal(a, b) and np.abs(b).max() > 100


# --------------------------------------------------------------- attention


def _tiny(seed, T, ctx, Hq, Hkv, D):
    rng = RNG(seed)
    return (rng.standard_normal((T, Hq, D)), rng.standard_normal((ctx, Hkv, D)),
            rng.standard_normal((ctx, Hkv, D)))


@pytest.mark.parametrize("T,ctx,start", [(1, 5, 4), (3, 7, 4), (4, 4, 0), (2, 9, 3)])
def test_attention_matches_brute_force(T, ctx, start):
    q, k, v = _tiny(T * 10 + ctx, T, ctx, 4, 2, 3)
    pos = start + np.arange(T)
    got = R.attention(q, k, v, pos, 0.7)
    want = np.array(R.brute_force_attention(q, k, v, pos, 0.7))
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_empty_rows_are_nan_like_torch():
    q, k, v = _tiny(0, 2, 3, 2, 1, 4)
    got = R.attention(q, k, v, np.array([-1, 0]), 1.0)
    assert np.isnan(got[0]).all() and np.isfinite(got[1]).all()


@pytest.mark.parametrize("n_tokens", [1, 7, 11, 16, 33])
def test_paged_prefill_matches_dense_reference(n_tokens):
    """tests/parity/test_parity.py:89-108."""
    rng = RNG(n_tokens)
    bs, n_kv, hd, n_q = 4, 2, 8, 4
    pool = R.PagedPool(32, bs, n_kv, hd)
    blocks = [(7 * i + 3) % 32 for i in range((n_tokens + bs - 1) // bs)]
    k = rng.standard_normal((n_tokens, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((n_tokens, n_kv, hd)).astype(np.float32)
    q = rng.standard_normal((n_tokens, n_q, hd)).astype(np.float32)
    pool.write(blocks, 0, k, v)
    got = R.paged_prefill(q, pool, blocks, 0, n_tokens)
    np.testing.assert_allclose(got, R.dense_causal_attention(q, k, v, n_q // n_kv), atol=1e-12)
    small = np.array(R.brute_force_attention(q[:3], k, v, np.arange(3), 1 / math.sqrt(hd)))
    np.testing.assert_allclose(got[:3], small, atol=1e-12)


def test_paged_decode_matches_dense_reference():
    """tests/parity/test_parity.py:111-131."""
    rng = RNG(1)
    bs, n_kv, hd, n_q, T = 4, 2, 8, 4, 11
    pool = R.PagedPool(32, bs, n_kv, hd)
    blocks = [5, 1, 9]
    k = rng.standard_normal((T + 1, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((T + 1, n_kv, hd)).astype(np.float32)
    pool.write(blocks, 0, k[:T], v[:T])
    pool.write(blocks, T, k[T:], v[T:])
    qn = rng.standard_normal((n_q, hd)).astype(np.float32)
    got = R.paged_decode(qn, pool, blocks, T + 1)
    want = np.array(R.brute_force_attention(qn[None], k, v, [T], 1 / math.sqrt(hd)))[0]
    np.testing.assert_allclose(got, want, atol=1e-12)


def test_chunked_prefill_equals_single_shot():
    rng = RNG(4)
    pool = R.PagedPool(16, 4, 2, 8)
    blocks = [3, 9, 0, 12]
    k = rng.standard_normal((13, 2, 8)).astype(np.float32)
    v = rng.standard_normal((13, 2, 8)).astype(np.float32)
    q = rng.standard_normal((13, 4, 8)).astype(np.float32)
    pool.write(blocks, 0, k, v)
    single = R.paged_prefill(q, pool, blocks, 0, 13)
    parts = [R.paged_prefill(q[s:s + 5], pool, blocks, s, min(s + 5, 13)) for s in range(0, 13, 5)]
    np.testing.assert_allclose(np.concatenate(parts), single, atol=1e-12)


def test_verify_equals_per_sequence_prefill_and_decode():
    rng = RNG(5)
    pool = R.PagedPool(32, 4, 2, 8)
    tables = [[1, 5, 9], [2, 30, 7, 4]]
    lens = [10, 15]
    for t, c in zip(tables, lens):
        pool.write(t, 0, rng.standard_normal((c, 2, 8)), rng.standard_normal((c, 2, 8)))
    q = rng.standard_normal((6, 4, 8))
    got = R.paged_verify_batched(q, pool, tables, lens, 3)
    # last verify token == a plain decode at that context
    for i, (t, c) in enumerate(zip(tables, lens)):
        np.testing.assert_allclose(got[3 * i + 2], R.paged_decode(q[3 * i + 2], pool, t, c), atol=1e-12)
        np.testing.assert_allclose(got[3 * i], R.paged_decode(q[3 * i], pool, t, c - 2), atol=1e-12)


def test_batched_decode_is_order_invariant():
    """tests/parity/test_triton_parity.py:89-112 at the oracle level."""
    rng = RNG(6)
    pool = R.PagedPool(64, 16, 2, 16)
    tables, lens = [[0, 1], [5, 2, 9], [3]], [20, 40, 7]
    for t, c in zip(tables, lens):
        pool.write(t, 0, rng.standard_normal((c, 2, 16)), rng.standard_normal((c, 2, 16)))
    q = rng.standard_normal((3, 4, 16))
    fwd = R.paged_decode_batched(q, pool, tables, lens)
    order = [2, 0, 1]
    rev = R.paged_decode_batched(q[order], pool, [tables[i] for i in order], [lens[i] for i in order])
    np.testing.assert_array_equal(rev, fwd[order])


def test_helios_cpu_routes_agree_with_the_oracle():
    rng = RNG(7)
    pool = R.PagedPool(64, 16, 2, 32, quantized=True)
    tables = [[4, 8, 15], [16, 23, 42, 7], [1]]
    lens = [40, 60, 9]
    for t, c in zip(tables, lens):
        pool.write(t, 0, rng.standard_normal((c, 2, 32)), rng.standard_normal((c, 2, 32)))
    q = rng.standard_normal((3, 6, 32)).astype(np.float32)
    want = R.paged_decode_batched(q, pool, tables, lens)
    got = R.helios_cpu_decode_batched_fp32(q, pool, tables, lens)
    np.testing.assert_allclose(got, want, atol=2e-6)
    qp = rng.standard_normal((5, 6, 32)).astype(np.float32)
    np.testing.assert_allclose(R.helios_cpu_prefill_fp32(qp, pool, tables[1], 55, 60),
                               R.paged_prefill(qp, pool, tables[1], 55, 60), atol=2e-6)


def _ragged_case(seed):
    """Three sequences written through scattered blocks of one pool: token
    counts (3, 0, 4) -- the middle chunk empty -- at start positions (2, 5, 0)
    with contexts (5, 5, 3), the last one shorter than its chunk's reach."""
    rng = RNG(seed)
    bs, Hkv, Hq, D = 2, 2, 4, 3
    pool = R.PagedPool(16, bs, Hkv, D)
    tables = [[7, 2, 11], [4, 0, 9], [13, 5]]
    ctxs, starts, qlens = [5, 5, 3], [2, 5, 0], [3, 0, 4]
    dense = []
    for t, c in zip(tables, ctxs):
        k = rng.standard_normal((c, Hkv, D)).astype(np.float32)  # the pool's storage dtype
        v = rng.standard_normal((c, Hkv, D)).astype(np.float32)
        pool.write(t, 0, k, v)
        dense.append((k, v))
    q = rng.standard_normal((sum(qlens), Hq, D))
    return pool, tables, ctxs, starts, qlens, dense, q


def _varlen_brute_force(q, dense, ctxs, starts, qlens, scale):
    """Row by row in pure Python: token i of sequence b (row offset by the
    earlier chunks) attends the first min(start + i + 1, ctx) keys of that
    sequence's own dense K/V."""
    rows, lo = [], 0
    for (k, v), c, s, n in zip(dense, ctxs, starts, qlens):
        for i in range(n):
            rows.append(R.brute_force_attention(q[lo + i:lo + i + 1], k[:c], v[:c], [s + i], scale)[0])
        lo += n
    return np.array(rows)


def test_varlen_matches_brute_force_on_a_ragged_batch():
    """paged_varlen (BatchedAttention.run's prefill branch, reference
    exec/model.py:303-317) against per-token brute force on the dense K/V:
    row offsets across sequences, an empty chunk, per-sequence start
    positions and a context that cuts a chunk's causal reach."""
    pool, tables, ctxs, starts, qlens, dense, q = _ragged_case(21)
    got = R.paged_varlen(q, pool, tables, qlens, starts, ctxs, 0.6)
    assert got.shape == q.shape
    np.testing.assert_allclose(got, _varlen_brute_force(q, dense, ctxs, starts, qlens, 0.6), atol=1e-12)


def test_varlen_default_scale_and_empty_batch():
    pool, tables, ctxs, starts, qlens, dense, q = _ragged_case(22)
    got = R.paged_varlen(q, pool, tables, qlens, starts, ctxs)
    np.testing.assert_allclose(got, _varlen_brute_force(q, dense, ctxs, starts, qlens, 1 / math.sqrt(3)),
                               atol=1e-12)
    empty = R.paged_varlen(q[:0], pool, [], [], [], [])
    assert empty.shape == (0, 4, 3)


def _varlen_no_offset(q, pool, tables, qlens, starts, ctxs, scale):
    """Planted mistake: every sequence reads its queries from row 0."""
    return np.concatenate([R.paged_prefill(q[:n], pool, t, s, c, scale)
                           for t, n, s, c in zip(tables, qlens, starts, ctxs)])


def _varlen_start_zero(q, pool, tables, qlens, starts, ctxs, scale):
    """Planted mistake: chunks treated as starting at position 0."""
    return R.paged_varlen(q, pool, tables, qlens, [0] * len(starts), ctxs, scale)


def _varlen_swapped_tables(q, pool, tables, qlens, starts, ctxs, scale):
    """Planted mistake: sequence b attends through the next sequence's table."""
    return R.paged_varlen(q, pool, tables[1:] + tables[:1], qlens, starts, ctxs, scale)


@pytest.mark.parametrize("bad", [_varlen_no_offset, _varlen_start_zero, _varlen_swapped_tables])
def test_varlen_brute_force_catches_planted_mistakes(bad):
    pool, tables, ctxs, starts, qlens, dense, q = _ragged_case(23)
    want = _varlen_brute_force(q, dense, ctxs, starts, qlens, 0.6)
    try:
        got = bad(q, pool, tables, qlens, starts, ctxs, 0.6)
    except (IndexError, ValueError):
        return  # a planted mistake that fails loudly is caught too
    assert got.shape != want.shape or not np.allclose(got, want, atol=1e-6)


# ------------------------------------------------- planted mistakes get caught


def _wrong_gqa_attention(q, k, v, q_positions, scale):
    """Planted mistake: query head h reads KV head h % Hkv instead of h // rep."""
    Hq, Hkv = q.shape[1], k.shape[1]
    idx = np.arange(Hq) % Hkv
    kk, vv = k[:, idx], v[:, idx]
    return R.attention(q, kk, vv, q_positions, scale)


def _wrong_mask_attention(q, k, v, q_positions, scale):
    """Planted mistake: off-by-one causal mask (k_pos >= q_pos masked)."""
    return R.attention(q, k, v, np.asarray(q_positions) - 1, scale)


@pytest.mark.parametrize("bad", [_wrong_gqa_attention, _wrong_mask_attention])
def test_brute_force_catches_planted_attention_mistakes(bad):
    q, k, v = _tiny(9, 3, 6, 4, 2, 3)
    pos = 3 + np.arange(3)
    want = np.array(R.brute_force_attention(q, k, v, pos, 0.5))
    with np.errstate(invalid="ignore"):
        got = bad(q, k, v, pos, 0.5)
    assert not np.allclose(got, want, atol=1e-6, equal_nan=True)


def test_tie_vectors_catch_round_half_away():
    x = np.array([[127.0, 2.5, -2.5, 0.5]], np.float32)
    s = np.float32(1.0)
    away = np.sign(x / s) * np.floor(np.abs(x / s) + 0.5)
    q, _ = R.quantize(x)
    assert not np.array_equal(away.astype(np.int8), q)


# ------------------------------------------------------------------ rotary

def _helios_rope_tables(max_pos, d, theta=10000.0):
    """helios' own table recipe (exec/model.py:117-132), evaluated by torch."""
    import torch

    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    freqs = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv)
    return freqs.cos().numpy(), freqs.sin().numpy()


def test_rope_position_zero_is_identity():
    cos, sin = _helios_rope_tables(8, 16)
    x = np.random.default_rng(0).standard_normal((3, 2, 16)).astype(np.float32)
    out = R.apply_rope(x, cos, sin, np.zeros(3, dtype=np.int64))
    assert np.array_equal(out, x)


def test_rope_hand_computed_rotation():
    # c = 0.5, s = 0.75 are exact in binary, so every product and sum is exact
    cos = np.array([[1.0, 1.0], [0.5, 0.5]], np.float32)
    sin = np.array([[0.0, 0.0], [0.75, 0.75]], np.float32)
    x = np.array([[[1.0, -2.0, 2.0, 4.0]]], np.float32)   # x1 = (1, -2), x2 = (2, 4)
    out = R.apply_rope(x, cos, sin, np.array([1]))
    # (x1 c - x2 s, x2 c + x1 s)
    assert out.tolist() == [[[0.5 - 1.5, -1.0 - 3.0, 1.0 + 0.75, 2.0 - 1.5]]]


def test_rope_matches_torch_elementwise_bit_for_bit():
    """helios evaluates x1 * c - x2 * s with torch elementwise ops on fp16 or
    fp32 inputs promoted to fp32; the oracle's float32 NumPy ops round the
    same way, so the rotated values (and everything quantized from them)
    agree bit for bit."""
    import torch

    cos, sin = _helios_rope_tables(512, 128)
    rng = np.random.default_rng(1)
    for dt in (np.float16, np.float32):
        x = (rng.standard_normal((40, 8, 128)) * 3).astype(dt)
        pos = rng.integers(0, 512, size=40)
        xt = torch.from_numpy(x)
        c = torch.from_numpy(cos)[torch.from_numpy(pos)].unsqueeze(1)
        s = torch.from_numpy(sin)[torch.from_numpy(pos)].unsqueeze(1)
        x1, x2 = xt.chunk(2, dim=-1)
        want = torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1).numpy()
        got = R.apply_rope(x, cos, sin, pos)
        assert got.dtype == np.float32 and np.array_equal(got, want)


def test_rope_planted_sign_mistake_is_caught():
    cos = np.array([[0.5, 0.5]], np.float32)
    sin = np.array([[0.75, 0.75]], np.float32)
    x = np.array([[[1.0, -2.0, 2.0, 4.0]]], np.float32)
    good = R.apply_rope(x, cos, sin, np.array([0]))
    x1, x2 = x[..., :2], x[..., 2:]
    wrong = np.concatenate((x1 * 0.5 + x2 * 0.75, x2 * 0.5 - x1 * 0.75), axis=-1)
    assert not np.array_equal(good, wrong)


def test_rope_table_restatement_close_to_helios():
    cos, sin = _helios_rope_tables(256, 64)
    c2, s2 = R.build_rope_cache(256, 64)
    assert np.abs(cos - c2).max() < 1e-4 and np.abs(sin - s2).max() < 1e-4


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-8, 8, 10000),
                        # exact ties (low half 0x8000) with even and odd kept bits, and a carry
                        np.array([0x3F808000, 0x3F818000, 0x3F7FFFFF, 0x7F7F8000 - 0x10000], np.uint32).view(np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(R.round_bf16(x), want)
    # hand example: 1 + 2^-8 is a tie between 1 and 1 + 2^-7, even (1) wins
    assert R.round_bf16(np.float32(1 + 2 ** -8)) == 1.0
