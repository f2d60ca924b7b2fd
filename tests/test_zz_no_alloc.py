"""The decode entry point that allocates nothing (hpa_paged_decode_noalloc).

It runs the same kernels as hpa_paged_decode with its split-K workspace in
the library's static per-GPU scratch instead of caller memory, so called
through the C-ABI on the same inputs it must give the same bits.  Two calls
in a row, the second on a smaller batch, check that what the first call left
in the shared scratch does not leak into the second.  Shapes whose workspace
exceeds the scratch are refused with HPA_ERR_WORKSPACE before anything runs.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from helios_amd import _lib
from helios_amd._lib import DTYPE_CODE, stream_ptr
from tests.test_gpu_decode import _case, _check, _oracle_decode

pytestmark = pytest.mark.gpu


def _padded(tables, dev):
    width = max(len(t) for t in tables)
    return torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.int32, device=dev)


def _args(q, out, cache, tt, lt, q_per_seq, max_ctx, part):
    ks, vs = cache._scales()
    quant = cache.k_cache.dtype == torch.int8
    Hkv, bs, D = cache.n_kv_heads, cache.block_size, cache.head_dim
    return [q.data_ptr(), out.data_ptr(), DTYPE_CODE[q.dtype], cache.k_cache.data_ptr(), cache.v_cache.data_ptr(),
            DTYPE_CODE[cache.k_cache.dtype], ks.data_ptr() if quant else None, vs.data_ptr() if quant else None,
            DTYPE_CODE[ks.dtype] if quant else 0, tt.data_ptr(), tt.shape[1], lt.data_ptr(), lt.numel(),
            q_per_seq, q.shape[1], Hkv, D, bs, cache.num_blocks, max_ctx, ctypes.c_float(D ** -0.5), part]


@pytest.mark.parametrize("quant", [False, True])
def test_noalloc_decode_equals_the_workspace_entry_point(quant):
    lib = _lib.lib()
    dev = torch.device("cuda:0")
    runs = [  # (seed, lens, q_per_seq, part_tokens): a wide split-K batch, then a smaller one
        (201, [3000, 17, 4500, 777, 4, 2100, 64, 3333], 3, 256),
        (202, [900, 5, 1200], 1, 128),
    ]
    for seed, lens, T, part in runs:
        print(f"noalloc decode: int8 {quant}, {len(lens)} sequences x {T}, part {part}", flush=True)
        cache, tables, q = _case(seed, len(lens), lens, 32, 8, 128, 16, torch.float16, quant=quant,
                                 q_per_seq=T)
        tt, lt = _padded(tables, dev), torch.tensor(lens, dtype=torch.int32, device=dev)
        max_ctx = max(lens)
        need = lib.hpa_decode_workspace_size(len(lens), T, 32, 8, 128, max_ctx, part)
        assert 0 < need <= _lib.HPA_NOALLOC_SCRATCH_BYTES
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        want = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        st = lib.hpa_paged_decode(*_args(q, want, cache, tt, lt, T, max_ctx, part), ws.data_ptr(), need,
                                  stream_ptr(dev))
        _lib.check(st, "hpa_paged_decode")
        st = lib.hpa_paged_decode_noalloc(*_args(q, got, cache, tt, lt, T, max_ctx, part), stream_ptr(dev))
        _lib.check(st, "hpa_paged_decode_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got, want), "noalloc differs from the workspace entry point"
        _check(got, _oracle_decode(cache, q, tables, lens, q_per_seq=T), torch.float16, "noalloc")


def test_noalloc_refuses_shapes_beyond_its_scratch():
    lib = _lib.lib()
    dev = torch.device("cuda:0")
    # 64 rows per KV head at head_dim 256 over long contexts: ~541 MB of workspace
    need = lib.hpa_decode_workspace_size(256, 4, 16, 1, 256, 32768, 0)
    assert need > _lib.HPA_NOALLOC_SCRATCH_BYTES
    x = torch.zeros(16, dtype=torch.int32, device=dev)
    p = x.data_ptr()
    st = lib.hpa_paged_decode_noalloc(p, p, _lib.HPA_F16, p, p, _lib.HPA_F16, None, None, 0, p, 1, p, 256, 4,
                                      16, 1, 256, 16, 1, 32768, ctypes.c_float(0.0625), 0, stream_ptr(dev))
    assert st == _lib.HPA_ERR_WORKSPACE
    assert b"static scratch" in lib.hpa_last_error()


def test_noalloc_at_config5_full_size():
    """Config 5's own batch (256 sequences x 3 tokens, Llama-8B int8 pool, the
    wave cap's workspace, ~50 MiB of the 64 MiB scratch): the no-alloc entry
    point equals hpa_paged_decode with a caller workspace bit for bit, twice
    in a row (the scratch keeps the counters at zero between calls)."""
    import bench

    lib = _lib.lib()
    dev = torch.device("cuda:0")
    print("noalloc decode at config 5's full size", flush=True)
    wl = bench.DecodeWorkload(5, dev, 4)
    cache = wl.caches[0]
    need = lib.hpa_decode_workspace_size(wl.B, wl.Tq, wl.Hq, wl.Hkv, wl.D, wl.max_ctx, 0)
    assert 0 < need <= _lib.HPA_NOALLOC_SCRATCH_BYTES
    want = wl.step().clone()
    for _ in range(2):
        got = torch.full_like(wl.q, float("nan"))
        st = lib.hpa_paged_decode_noalloc(*_args(wl.q, got, cache, wl.tables_t, wl.lens_t, wl.Tq, wl.max_ctx, 0),
                                          stream_ptr(dev))
        _lib.check(st, "hpa_paged_decode_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got, want), "noalloc differs from the workspace entry point at config 5"
