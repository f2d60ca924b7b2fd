"""Parity at BASELINE.json's five configs, at their full sizes.

Each test builds exactly the seeded inputs bench.py times (its workload
builders are imported, not retyped), runs one step of the HIP path through
the C-ABI and compares every output row with the oracle:

  config 1  fp32 toy decode                       max-abs <= 2e-5 (float64 oracle)
  config 2  Qwen-0.5B fp16 decode, batch 64        max-abs <= 2e-3
  config 3  the same over int8 KV: the quantize+scatter write of one new
            token per sequence (payload and scales bit-exact, every other
            slot untouched), then the decode     max-abs <= 2e-3
  config 4  Llama-8B fp16 chunked prefill, 8 x 512 tokens on priors up to
            3584 with 64 shared prefix blocks   max-abs <= 2e-3
            (and the same shape over an int8 pool)
  config 5  Llama-8B int8 decode + verify, batch 256, lognormal contexts
                                                 max-abs <= 2e-3

The fp16 checkers are the oracle's fp32 restatements of helios' CPU routes
(helios_cpu_prefill_fp32, one paged_attention_prefill per sequence, the
decode being its one-token case), which tests/test_oracle.py pins to the
float64 oracle within 2e-6; the inputs are the exact values the kernels read
(fp16 pools upcast, int8 pools dequantised with the stored scales, or, for
the MFMA prefill over int8, the dequantised values rounded to fp16 as
helios' gather hands them to attention, paged_attn.py:213-235).  Reference
tests restated at these sizes: tests/parity/test_parity.py:89-148 and
tests/parity/test_triton_parity.py:50-86.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from oracle import paged_ref as R
from tests.gpu_util import max_abs, pool_dequantized, pool_of, to_np

pytestmark = pytest.mark.gpu


def _dev():
    return torch.device("cuda:0")


def _oracle_rows(q: np.ndarray, pool, tables, starts, ctxs, qlens, scale) -> np.ndarray:
    """helios' CPU route, one paged_attention_prefill per sequence."""
    outs, lo = [], 0
    for t, s, c, n in zip(tables, starts, ctxs, qlens):
        outs.append(R.helios_cpu_prefill_fp32(q[lo:lo + n], pool, t, s, c, scale))
        lo += n
    return np.concatenate(outs, axis=0)


def _tables_of(wl):
    return [[int(x) for x in row[:(c + bench.BLOCK - 1) // bench.BLOCK]]
            for row, c in zip(wl.tables_np, wl.lens)]


def _decode_check(wl, got: torch.Tensor, tol: float, what: str):
    pool = pool_of(wl.caches[0])
    q = to_np(wl.q).astype(np.float32)
    T = wl.Tq
    want = _oracle_rows(q, pool, _tables_of(wl), [c - T for c in wl.lens], wl.lens, [T] * wl.B, wl.scale)
    g = to_np(got).astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = max_abs(g, want)
    print(f"{what}: max-abs {err:.3e} over {g.shape[0]} rows", flush=True)
    assert err <= tol, f"{what}: max-abs {err:.3e} > {tol}"


def test_config1_toy_fp32_decode():
    print("config 1: toy fp32 decode", flush=True)
    wl = bench.DecodeWorkload(1, _dev(), 0)
    got = wl.step()
    torch.cuda.synchronize()
    pool = pool_of(wl.caches[0])
    want = R.paged_decode_batched(to_np(wl.q), pool, _tables_of(wl), wl.lens, wl.scale)
    err = max_abs(to_np(got), want)
    print(f"config 1: max-abs {err:.3e}", flush=True)
    assert err <= 2e-5


def test_config2_qwen_fp16_decode_batch64():
    print("config 2: Qwen-0.5B fp16 decode, batch 64", flush=True)
    wl = bench.DecodeWorkload(2, _dev(), 1)
    assert wl.B == 64 and min(wl.lens) >= 512 and max(wl.lens) <= 4096
    got = wl.step()
    torch.cuda.synchronize()
    _decode_check(wl, got, 2e-3, "config 2")


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.float32])
def test_config3_int8_write_then_decode(scale_dtype):
    print(f"config 3: int8 write + decode, scales {scale_dtype}", flush=True)
    wl = bench.DecodeWorkload(3, _dev(), 2, scale_dtype=scale_dtype)
    c = wl.caches[0]
    before = [to_np(t).copy() for t in (c.k_cache, c.v_cache, c.k_scale, c.v_scale)]
    got = wl.step()  # write one new token per sequence at ctx - 1, then decode
    torch.cuda.synchronize()
    after = [to_np(t) for t in (c.k_cache, c.v_cache, c.k_scale, c.v_scale)]
    # the write: exactly the new slots change, to the oracle's quantisation
    sdt = np.float16 if scale_dtype == torch.float16 else np.float32
    tabs = _tables_of(wl)
    want = [x.copy() for x in before]
    for src, (pay, sc) in ((wl.new_k, (0, 2)), (wl.new_v, (1, 3))):
        qv, s = R.quantize(to_np(src).astype(np.float32))
        for b, ctx in enumerate(wl.lens):
            p = ctx - 1
            blk, off = tabs[b][p // bench.BLOCK], p % bench.BLOCK
            want[pay][blk, :, off, :] = qv[b]
            want[sc][blk, :, off] = R.store_scale(s[b], sdt)
    for name, a, w in zip(("k", "v", "k_scale", "v_scale"), after, want):
        assert a.dtype == w.dtype and np.array_equal(a, w), f"config 3 write: {name} differs"
    _decode_check(wl, got, 2e-3, f"config 3 ({'fp16' if sdt == np.float16 else 'fp32'} scales)")


@pytest.mark.parametrize("kv_int8", [False, True])
def test_config4_llama8b_chunked_prefill(kv_int8):
    print(f"config 4: Llama-8B chunked prefill 8 x 512, int8 pool {kv_int8}", flush=True)
    wl = bench.PrefillWorkload(_dev(), 3, kv_int8=kv_int8)
    assert wl.B == 8 and wl.T == 512 and max(wl.priors) <= 3584
    # the prefix blocks really are shared wherever a prior covers them
    full = [p // bench.BLOCK for p in wl.priors]
    shared = [t[:min(64, f)] for t, f in zip(wl.tabs, full)]
    longest = max(shared, key=len)
    assert all(s == longest[:len(s)] for s in shared) and len(longest) == min(64, max(full))
    got = wl.step()
    torch.cuda.synchronize()
    pool = pool_dequantized(wl.cache) if kv_int8 else pool_of(wl.cache)
    want = _oracle_rows(to_np(wl.q).astype(np.float32), pool, wl.tabs, wl.priors, wl.ctxs,
                        [wl.T] * wl.B, wl.scale)
    g = to_np(got).astype(np.float64)
    assert np.isfinite(g).all()
    err = max_abs(g, want)
    print(f"config 4 (int8 {kv_int8}): max-abs {err:.3e} over {g.shape[0]} rows", flush=True)
    assert err <= 2e-3


def test_config5_llama8b_int8_decode_verify_batch256():
    print("config 5: Llama-8B int8 decode + verify, batch 256", flush=True)
    wl = bench.DecodeWorkload(5, _dev(), 4)
    assert wl.B == 256 and wl.Tq == 3 and min(wl.lens) >= 64 and max(wl.lens) <= 32768
    first = wl.step().clone()
    torch.cuda.synchronize()
    _decode_check(wl, first, 2e-3, "config 5")
    # a second call on the same workspace (its counters back at zero) is
    # bit-identical: the split-K merge order is fixed
    again = wl.step()
    torch.cuda.synchronize()
    assert torch.equal(again, first)


def test_bf16_error_reported_as_max_abs_and_ulps():
    """Config 2's shape in bf16: the error against the float64 oracle on the
    same rounded inputs, reported as max-abs and in units of the output's
    bf16 ulp.  Rounding the output to bf16 alone costs up to half an ulp
    (2^-9 ~ 1.95e-3 for |out| in [0.5, 1)), so the bound is 2e-3 plus half an
    ulp of the reference, and the ulp-normalised error where |out| >= 1/8
    stays within one ulp."""
    from helios_amd import PagedKVCache, paged_attention_decode_hip
    from tests.gpu_util import fill_cache

    gen = torch.Generator().manual_seed(11)
    rng = np.random.default_rng(11)
    B, Hq, Hkv, D = 64, 14, 2, 64
    lens = [int(x) for x in rng.integers(512, 4097, size=B)]
    need = [(c + 15) // 16 for c in lens]
    cache = PagedKVCache(sum(need), 16, Hkv, D, dtype=torch.bfloat16, device="cuda")
    fill_cache(cache, gen)
    ids = rng.permutation(sum(need))
    tabs, o = [], 0
    for n in need:
        tabs.append([int(x) for x in ids[o:o + n]])
        o += n
    q = torch.randn(B, Hq, D, generator=gen).to(torch.bfloat16).cuda()
    got = to_np(paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tabs, lens)).astype(np.float64)
    want = R.paged_decode_batched(to_np(q), pool_of(cache), tabs, lens)
    err = np.abs(got - want)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
    big = np.abs(want) >= 0.125
    ulps = float((err[big] / ulp[big]).max()) if big.any() else 0.0
    print(f"bf16 decode: max-abs {err.max():.3e}, max {ulps:.3f} bf16 ulps where |out| >= 1/8", flush=True)
    assert (err <= 2e-3 + np.abs(want) * 2.0 ** -8).all()
    assert ulps <= 1.0
