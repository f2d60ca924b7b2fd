"""A multi-layer decode / verify step captured in a HIP graph.

With the step's metadata on the device (DeviceBlockTables) and the outputs
and a decode workspace owned by the caller, every layer's write_kv_batched +
batched_attention is launches only -- no host work, no synchronisation, no
allocation (the capture is checked to allocate nothing) -- so the whole step
can be captured and replayed.  The decode kernel's split-K counters are returned to zero by
the kernel itself, so a replay needs no memset node.  Each replay here runs
after eager work and a synchronisation, with new inputs copied into the
captured tensors, and must equal the same calls made eagerly on twin caches,
bit for bit.  Nine query tokens per sequence (36 rows per KV head) run the
verify on the MFMA prefill kernel."""

from __future__ import annotations

import pytest
import torch

import helios_amd as H
from tests.test_step_meta import Sim

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("quant,q_per_seq", [(False, 1), (True, 1), (True, 3), (False, 9), (True, 9)])
def test_captured_step_replays_equal_eager(quant, q_per_seq):
    print(f"graph replay: int8 {quant}, q_per_seq {q_per_seq}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(5)
    bs, Hq, Hkv, D, nb, layers = 16, 16, 4, 128, 512, 3
    sim = Sim(seed=8, bs=bs, pool=nb, unique=True)
    for _ in range(30):  # a populated batch: prompts in, some decodes running
        step = sim.step(max_batch=12)[0]
    tables = [s["blocks"] for s in sim.seqs.values() if s["ctx"] > 0]
    ctx = [s["ctx"] for s in sim.seqs.values() if s["ctx"] > 0]
    # room for the q_per_seq tokens written by this step
    for t, c in zip(tables, ctx):
        while len(t) * bs < c + q_per_seq:
            t.append(sim._blocks(1)[0])
    B = len(tables)

    def make():
        if quant:
            return H.QuantizedPagedKVCache(nb, bs, Hkv, D, dtype=torch.float16, device="cuda")
        return H.PagedKVCache(nb, bs, Hkv, D, dtype=torch.float16, device="cuda")

    graph_caches, eager_caches = [make() for _ in range(layers)], [make() for _ in range(layers)]
    for gc, ec in zip(graph_caches, eager_caches):
        for x, y in ((gc.k_cache, ec.k_cache), (gc.v_cache, ec.v_cache)):
            init = torch.randint(-127, 128, x.shape, generator=gen, device="cuda", dtype=torch.int8) if quant \
                else torch.randn(x.shape, generator=gen, device="cuda", dtype=torch.float16)
            x.copy_(init)
            y.copy_(init)
        if quant:
            for x, y in ((gc.k_scale, ec.k_scale), (gc.v_scale, ec.v_scale)):
                s = torch.rand(x.shape, generator=gen, device="cuda") * 0.02 + 1e-3
                x.copy_(s)
                y.copy_(s)
    tabs = H.DeviceBlockTables.for_cache(graph_caches[0], 32, 16)
    base = tabs.prepare(range(B), tables, [c + 1 for c in ctx], ctx, [1] * B, True)
    meta = base.verify(q_per_seq) if q_per_seq > 1 else base
    n_tok = B * q_per_seq
    q = torch.empty(layers, n_tok, Hq, D, device="cuda", dtype=torch.float16)
    k = torch.empty(layers, n_tok, Hkv, D, device="cuda", dtype=torch.float16)
    v = torch.empty_like(k)

    def fill():
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=gen, device="cuda").half())

    def owned():
        return ([torch.empty(n_tok, Hq, D, device="cuda", dtype=torch.float16) for _ in range(layers)],
                H.decode_workspace(B, q_per_seq, Hq, Hkv, D, meta.max_context_len, "cuda"))

    graph_owned, eager_owned = owned(), owned()

    def step(caches, own):
        outs, ws = own
        for li, c in enumerate(caches):
            H.write_kv_batched(c, meta, k[li], v[li])
            H.batched_attention(q[li], c, meta, 0.125, out=outs[li], workspace=ws)
        return outs

    fill()
    step(graph_caches, graph_owned)  # warm: launch configuration cached
    step(eager_caches, eager_owned)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        # counted inside the capture: torch's own capture set-up is not ours
        allocs = torch.cuda.memory_stats()["allocation.all.allocated"]
        graph_out = step(graph_caches, graph_owned)
        allocs = torch.cuda.memory_stats()["allocation.all.allocated"] - allocs
    torch.cuda.synchronize()
    assert allocs == 0, f"the captured step allocated {allocs} times"
    for rep in range(4):
        fill()
        want = step(eager_caches, eager_owned)  # eager work between the replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for li in range(layers):
            assert torch.equal(graph_out[li], want[li]), f"replay {rep} layer {li}"
    for gc, ec in zip(graph_caches, eager_caches):
        assert torch.equal(gc.k_cache, ec.k_cache) and torch.equal(gc.v_cache, ec.v_cache)
        if quant:
            assert torch.equal(gc.k_scale, ec.k_scale) and torch.equal(gc.v_scale, ec.v_scale)
