"""GPU parity of the device-resident step metadata: hpa_step_tables against
the oracle's restatement of helios' per-step BatchedAttnMeta over a long run
of scheduler steps, and attention driven by it equal, bit for bit, to the
same kernels driven by helios' Python lists."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import helios_amd as H
from oracle import paged_ref as R
from oracle import step_meta_ref as M
from tests.test_step_meta import Sim

pytestmark = pytest.mark.gpu


def _check_meta(meta, ref):
    want = M.padded_tables(ref.block_tables)
    got = meta.block_tables.cpu().numpy()
    w = want.shape[1]
    assert got.shape[0] == want.shape[0]
    np.testing.assert_array_equal(got[:, :w], want)
    assert not got[:, w:].any()
    np.testing.assert_array_equal(meta.context_lens.cpu().numpy(), ref.context_lens)
    np.testing.assert_array_equal(meta.start_positions.cpu().numpy(), ref.start_positions)
    cu = meta.cu_query_lens.cpu().numpy()
    assert [(int(cu[b]), int(cu[b + 1])) for b in range(len(cu) - 1)] == ref.token_slices
    assert meta.token_slices == ref.token_slices
    assert meta.is_decode == ref.is_decode


@pytest.mark.parametrize("max_seqs,release", [(64, True), (12, False)])
def test_step_tables_match_the_oracle_over_many_steps(max_seqs, release):
    print(f"step tables: max_seqs {max_seqs}, release {release}", flush=True)
    sim = Sim(seed=100 + max_seqs, bs=4)
    tabs = H.DeviceBlockTables(max_seqs, 64, "cuda", block_size=4, num_blocks=sim.pool)
    for _ in range(300):
        step, finished, preempted = sim.step(max_batch=min(max_seqs, 10))
        if release:
            for sid in finished + preempted:
                tabs.release(sid)
        pre, dec = tabs.prepare_step(step)
        assert (pre is None) == (not step.prefills) and (dec is None) == (not step.decodes)
        if pre is not None:
            _check_meta(pre, M.prefill_meta(step.prefills))
        if dec is not None:
            _check_meta(dec, M.decode_meta(step.decodes))
        res = tabs.resident.cpu().numpy()
        for it in list(step.prefills) + list(step.decodes):
            np.testing.assert_array_equal(res[tabs.host.row[it.seq_id], : len(it.block_ids)], it.block_ids)


def test_wide_rows_and_many_sequences():
    """Rows wider than one 256-thread group and the full row count."""
    rng = np.random.default_rng(1)
    n, width = 300, 700
    tabs = H.DeviceBlockTables(n, width, "cuda")
    tables = [[int(x) for x in rng.integers(0, 1 << 20, size=rng.integers(0, width + 1))] for _ in range(n)]
    lens = [len(t) * 16 for t in tables]
    meta = tabs.prepare(list(range(n)), tables, lens, [max(c - 1, 0) for c in lens], [1] * n, True)
    _check_meta(meta, M.Meta([(i, i + 1) for i in range(n)], tables, lens,
                             [max(c - 1, 0) for c in lens], True))
    # grow every table by one block, shrink a few, replace one in the middle
    for i, t in enumerate(tables):
        if i % 7 == 0 and t:
            del t[len(t) // 2:]
        elif len(t) < width:
            t.append(i)
        if i % 11 == 0 and len(t) > 3:
            t[1] = 123456
    lens = [len(t) * 16 for t in tables]
    meta = tabs.prepare(list(range(n)), tables, lens, [max(c - 1, 0) for c in lens], [1] * n, True)
    _check_meta(meta, M.Meta([(i, i + 1) for i in range(n)], tables, lens,
                             [max(c - 1, 0) for c in lens], True))


@pytest.mark.parametrize("pool_dtype", [torch.float16, torch.int8])
def test_attention_on_device_metadata_equals_list_driven_calls(pool_dtype):
    """A scheduler run writing and attending through DeviceBlockTables gives
    the same pools and outputs, bit for bit, as the same kernels fed the
    runner's Python lists (exec/runner.py:203-268, model.py:236-247)."""
    print(f"device metadata end-to-end: {pool_dtype}", flush=True)
    gen = torch.Generator().manual_seed(7)
    bs, Hq, Hkv, D, nb = 16, 8, 2, 64, 640
    sim = Sim(seed=9, bs=bs, pool=nb, unique=True)

    def make():
        if pool_dtype == torch.int8:
            return H.QuantizedPagedKVCache(nb, bs, Hkv, D, dtype=torch.float16, device="cuda")
        return H.PagedKVCache(nb, bs, Hkv, D, dtype=torch.float16, device="cuda")

    a, b = make(), make()
    for x, y in ((a.k_cache, b.k_cache), (a.v_cache, b.v_cache)):
        init = torch.randn(x.shape, generator=gen).to(x.dtype) if pool_dtype != torch.int8 else \
            torch.randint(-127, 128, x.shape, generator=gen, dtype=torch.int8)
        x.copy_(init)
        y.copy_(init)
    if pool_dtype == torch.int8:
        for x, y in ((a.k_scale, b.k_scale), (a.v_scale, b.v_scale)):
            s = (torch.rand(x.shape, generator=gen) * 0.02 + 1e-3).to(x.dtype)
            x.copy_(s)
            y.copy_(s)
    cos, sin = (torch.from_numpy(t).cuda() for t in R.build_rope_cache(2048, D, 10000.0))
    tabs = H.DeviceBlockTables.for_cache(a, 16, 64)
    steps = 0
    for _ in range(60):
        step, finished, preempted = sim.step(max_batch=10)
        for sid in finished + preempted:
            tabs.release(sid)
        pre_m, dec_m = tabs.prepare_step(step)
        for items, meta, ref in ((step.prefills, pre_m, M.prefill_meta(step.prefills)),
                                 (step.decodes, dec_m, M.decode_meta(step.decodes))):
            if not items:
                continue
            n_tok = ref.token_slices[-1][1]
            k = torch.randn(n_tok, Hkv, D, generator=gen).half().cuda()
            v = torch.randn(n_tok, Hkv, D, generator=gen).half().cuda()
            q = torch.randn(n_tok, Hq, D, generator=gen).half().cuda()
            H.write_kv_batched(a, meta, k, v, rope=(cos, sin))
            out_a = H.batched_attention(q, a, meta, 0.125)
            qlens = [hi - lo for lo, hi in ref.token_slices]
            H.write_kv(b, ref.block_tables, ref.start_positions, k, v, query_lens=qlens, rope=(cos, sin))
            if ref.is_decode:
                out_b = H.paged_attention_decode_batched(q, b, ref.block_tables, ref.context_lens, 0.125)
            else:
                out_b = H.paged_attention_varlen(q, b, ref.block_tables, qlens, ref.start_positions,
                                                 ref.context_lens, 0.125)
            assert torch.equal(out_a, out_b)
            steps += 1
    assert steps > 40
    for x, y in ((a.k_cache, b.k_cache), (a.v_cache, b.v_cache)):
        assert torch.equal(x, y)
    if pool_dtype == torch.int8:
        assert torch.equal(a.k_scale, b.k_scale) and torch.equal(a.v_scale, b.v_scale)


def test_a_step_on_device_metadata_does_not_synchronise():
    """After the first steps have sized the buffers, prepare + write +
    attention for every layer issue no synchronising call."""
    bs, Hq, Hkv, D, nb, layers = 16, 8, 2, 64, 256, 4
    sim = Sim(seed=3, bs=bs, pool=nb, unique=True)
    caches = [H.PagedKVCache(nb, bs, Hkv, D, dtype=torch.float16, device="cuda") for _ in range(layers)]
    tabs = H.DeviceBlockTables.for_cache(caches[0], 16, 32)
    gen = torch.Generator(device="cuda").manual_seed(0)

    def run(step):
        for meta in tabs.prepare_step(step):
            if meta is None:
                continue
            for c in caches:
                k = torch.randn(meta.n_tokens, Hkv, D, device="cuda", dtype=torch.float16, generator=gen)
                q = torch.randn(meta.n_tokens, Hq, D, device="cuda", dtype=torch.float16, generator=gen)
                H.write_kv_batched(c, meta, k, k)
                H.batched_attention(q, c, meta, 0.125)

    for _ in range(6):
        run(sim.step(max_batch=10)[0])
    torch.cuda.synchronize()
    prev = torch.cuda.get_sync_debug_mode()
    torch.cuda.set_sync_debug_mode("error")
    try:
        for _ in range(6):
            run(sim.step(max_batch=10)[0])
        # the detector does see the list-to-device conversion these calls avoid
        q = torch.zeros(2, Hq, D, device="cuda", dtype=torch.float16)
        with pytest.raises(RuntimeError):
            H.paged_attention_decode_batched(q, caches[0], [[3], [4, 5]], [9, 20], 0.125)
    finally:
        torch.cuda.set_sync_debug_mode(prev)
    torch.cuda.synchronize()


def test_step_tables_c_abi_contract():
    """hpa_step_tables called directly: a replaced suffix lands in the
    resident row and the step row, entries past n_blocks read 0, and a row
    outside the resident array gives an all-zero step row (and writes
    nothing)."""
    from helios_amd import _lib

    L = _lib.load_library()
    resident = torch.arange(4 * 6, dtype=torch.int32, device="cuda").view(4, 6).contiguous()
    before = resident.clone()
    # (row, n_blocks, upd_first, upd_count, upd_offset)
    entries = torch.tensor([[2, 5, 3, 2, 0], [7, 4, 0, 1, 2], [0, 2, 0, 0, 3]], dtype=torch.int32, device="cuda")
    new_ids = torch.tensor([100, 101, 555], dtype=torch.int32, device="cuda")
    step = torch.full((3, 6), -1, dtype=torch.int32, device="cuda")
    st = L.hpa_step_tables(entries.data_ptr(), 3, new_ids.data_ptr(), 3, resident.data_ptr(), 4, 6,
                           step.data_ptr(), 6, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    want_res = before.clone()
    want_res[2, 3:5] = torch.tensor([100, 101], dtype=torch.int32)
    assert torch.equal(resident, want_res)
    assert step[0].tolist() == [12, 13, 14, 100, 101, 0]
    assert step[1].tolist() == [0] * 6   # row 7 is outside the 4 resident rows
    assert step[2].tolist() == [0, 1, 0, 0, 0, 0]
