#!/usr/bin/env python3
"""Benchmark of helios' paged-attention hot path on one MI355X.

One "step" is one call of the hot path over one batch of seeded synthetic
input already resident in HBM.  The default workload is config 5 of
BASELINE.json -- Llama-3-8B-shape INT8-KV decode + speculative verify
(Hq 32 / Hkv 8, D 128, batch 256, 3 query tokens per sequence, contexts
lognormal(median 2048, sigma 0.5) clipped to [64, 32768], block size 16),
the shape the build's >= 70%-of-HBM target is stated on.  ``--config N``
measures the other configs the same way.

Prints ONE JSON line (the driver's contract) with a ``roofline`` object for
the dominant kernel and a ``cpu_baseline`` object: the oracle's restatement of
helios' own CPU route, timed on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, 8 TB/s
MFMA_F16_PEAK_TFS = 2500.0  # MI355X dense fp16/bf16 MFMA, 2.5 PFLOP/s
BLOCK = 16


def _ctx_lognormal(rng, n, median, sigma, lo, hi):
    import numpy as np

    x = np.exp(rng.normal(math.log(median), sigma, size=n))
    return [int(v) for v in np.clip(np.rint(x), lo, hi)]


class Workload:
    """A seeded config: device tensors, the step to time, and its work."""

    name = ""
    bound = "hbm"

    def step(self):  # pragma: no cover - overridden
        raise NotImplementedError


def _shuffled_tables(rng, lens, device):
    import numpy as np
    import torch

    need = [(c + BLOCK - 1) // BLOCK for c in lens]
    nb = int(sum(need))
    perm = rng.permutation(nb).astype(np.int32)
    width = max(need)
    tab = np.zeros((len(lens), width), np.int32)
    o = 0
    for i, n in enumerate(need):
        tab[i, :n] = perm[o:o + n]
        o += n
    return nb, torch.from_numpy(tab).to(device), tab


def _fill_by_writes(cache, lens, tables_t, gen, device, chunk_tokens=1 << 19):
    """Fill every (sequence, position) of the pool with N(0,1) fp16 K/V through
    the library's own write kernel (for int8 pools: quantize + scatter, the
    configs' 'quantized N(0,1) fp16' recipe)."""
    import torch

    from helios_amd import write_kv

    H, D = cache.n_kv_heads, cache.head_dim
    i = 0
    while i < len(lens):
        j, tok = i, 0
        while j < len(lens) and (tok == 0 or tok + lens[j] <= chunk_tokens):
            tok += lens[j]
            j += 1
        vdt = torch.bfloat16 if cache.dtype == torch.bfloat16 else torch.float16
        k = torch.randn(tok, H, D, generator=gen, device=device, dtype=vdt)
        v = torch.randn(tok, H, D, generator=gen, device=device, dtype=vdt)
        write_kv(cache, tables_t[i:j], [0] * (j - i), k, v, query_lens=lens[i:j])
        i = j
    torch.cuda.synchronize()


class DecodeWorkload(Workload):
    """Configs 2, 3 and 5: batched decode (q_per_seq 1) or verify (3)."""

    def __init__(self, cfg, device, seed, part_tokens=0, copies=1, scale_dtype=None, qdtype=None):
        import numpy as np
        import torch

        import helios_amd as H

        self.cfg = cfg
        rng = np.random.default_rng(seed)
        gen = torch.Generator(device=device).manual_seed(seed)
        if cfg == 5:
            self.name = "llama3-8b-int8-decode-verify (config 5)"
            B, Hq, Hkv, D, Tq, quant = 256, 32, 8, 128, 3, True
            lens = _ctx_lognormal(rng, B, 2048, 0.5, 64, 32768)
        elif cfg in (2, 3):
            quant = cfg == 3
            self.name = ("qwen2.5-0.5b-int8-decode+write (config 3)" if quant
                         else "qwen2.5-0.5b-fp16-decode (config 2)")
            B, Hq, Hkv, D, Tq = 64, 14, 2, 64, 1
            lens = [int(x) for x in rng.integers(512, 4097, size=B)]
        else:
            self.name = "toy-fp32-decode (config 1)"
            B, Hq, Hkv, D, Tq, quant = 4, 4, 2, 64, 1, False
            lens = [int(x) for x in rng.integers(17, 101, size=B)]
        dtype = torch.float32 if cfg == 1 else (qdtype or torch.float16)
        if dtype == torch.bfloat16:
            self.name += ", bf16 queries"
        self.B, self.Hq, self.Hkv, self.D, self.Tq, self.quant = B, Hq, Hkv, D, Tq, quant
        self.lens = lens
        nb, self.tables_t, self.tables_np = _shuffled_tables(rng, lens, device)
        self.lens_t = torch.tensor(lens, dtype=torch.int32, device=device)
        self.max_ctx = max(lens)
        self.scale = 1.0 / math.sqrt(D)
        self.part_tokens = part_tokens
        # Configs 2/3 fit in the 256 MB Infinity Cache: rotate over enough
        # pool copies that every step reads from HBM.
        self.caches = []
        self.scale_dtype = scale_dtype or torch.float16
        for _ in range(copies):
            if quant:
                c = H.QuantizedPagedKVCache(nb, BLOCK, Hkv, D, dtype=dtype, device=device,
                                            scale_dtype=self.scale_dtype)
            else:
                c = H.PagedKVCache(nb, BLOCK, Hkv, D, dtype=dtype, device=device)
            _fill_by_writes(c, lens, self.tables_t, gen, device)
            self.caches.append(c)
        self.q = torch.randn(B * Tq, Hq, D, generator=gen, device=device, dtype=dtype)
        self.out = torch.empty_like(self.q)
        ws = H.decode_workspace_bytes(B, Tq, Hq, Hkv, D, self.max_ctx, part_tokens)
        self.ws = torch.zeros(max(ws, 1), dtype=torch.uint8, device=device)
        if cfg == 3:  # one new token per sequence, written at position ctx - 1
            self.new_k = torch.randn(B, Hkv, D, generator=gen, device=device, dtype=dtype)
            self.new_v = torch.randn(B, Hkv, D, generator=gen, device=device, dtype=dtype)
            self.new_pos = torch.tensor([c - 1 for c in lens], dtype=torch.int32, device=device)
            self.new_cu = torch.arange(0, B + 1, dtype=torch.int32, device=device)
        self.i = 0
        sb = 4 if self.scale_dtype == torch.float32 else 2
        kvb = D * (1 if quant else (4 if cfg == 1 else 2)) + (sb if quant else 0)
        elt = 4 if cfg == 1 else 2
        sum_ctx = sum(lens)
        n_tab = sum((c + BLOCK - 1) // BLOCK for c in lens)
        self.kv_bytes = sum_ctx * 2 * Hkv * kvb
        self.alg_bytes = self.kv_bytes + 2 * B * Tq * Hq * D * elt + 4 * n_tab + 4 * B
        if cfg == 3:  # the write: read K,V fp16, write int8 + scale
            self.alg_bytes += B * 2 * Hkv * (D * 2 + D + sb)
        self.flops = 4 * D * Hq * sum(sum(min(c, c - Tq + t + 1) for t in range(Tq)) for c in lens)
        self.tokens = B * Tq

    def step(self):
        import helios_amd as H

        c = self.caches[self.i % len(self.caches)]
        self.i += 1
        if self.cfg == 3:
            H.write_kv(c, self.tables_t, self.new_pos, self.new_k, self.new_v,
                       cu_query_lens=self.new_cu, max_query_len=1)
        ks, vs = c._scales()
        return H.paged_attention_decode_hip(
            self.q, c.k_cache, c.v_cache, self.tables_t, self.lens_t, self.scale, ks, vs,
            q_per_seq=self.Tq, max_context_len=self.max_ctx, part_tokens=self.part_tokens,
            out=self.out, workspace=self.ws,
        )

    def config(self):
        import torch

        return {"workload": self.name, "batch": self.B, "q_per_seq": self.Tq,
                "n_q_heads": self.Hq, "n_kv_heads": self.Hkv, "head_dim": self.D,
                "block_size": BLOCK, "q_dtype": str(self.q.dtype).replace("torch.", ""),
                "kv_dtype": "int8" if self.quant else
                ("fp32" if self.cfg == 1 else ("bf16" if self.q.dtype == torch.bfloat16 else "fp16")),
                "scale_dtype": ("fp32" if self.scale_dtype == torch.float32 else "fp16") if self.quant else None,
                "context": {"mean": round(sum(self.lens) / len(self.lens), 1),
                            "max": self.max_ctx, "min": min(self.lens)},
                "pool_copies": len(self.caches), "part_tokens": self.part_tokens or "auto"}

    def cpu_baseline(self, budget_s):
        """helios' CPU route (fp32, reference engine.py:135-138) on a bounded
        sample: decode -> paged_attention_decode_batched; verify -> one
        paged_attention_prefill per sequence (reference runner.py:354-362)."""
        import numpy as np

        from oracle import paged_ref as R

        c = self.caches[0]
        pool = R.PagedPool(c.num_blocks, BLOCK, self.Hkv, self.D, np.float32, quantized=self.quant)
        if self.quant:
            pool.k = c.k_cache.cpu().numpy()
            pool.v = c.v_cache.cpu().numpy()
            pool.k_scale = c.k_scale.cpu().numpy()
            pool.v_scale = c.v_scale.cpu().numpy()
        else:  # (numpy has no bf16: through fp32, which holds every value)
            pool.k = c.k_cache.float().cpu().numpy()
            pool.v = c.v_cache.float().cpu().numpy()
        q = self.q.float().cpu().numpy()
        tabs = [list(self.tables_np[i, :(n + BLOCK - 1) // BLOCK]) for i, n in enumerate(self.lens)]
        done, t0 = 0, time.perf_counter()
        if self.Tq == 1:
            chunk = 8
            while done < self.B and time.perf_counter() - t0 < budget_s:
                sl = slice(done, min(self.B, done + chunk))
                R.helios_cpu_decode_batched_fp32(q[sl], pool, tabs[sl], self.lens[sl], self.scale)
                done = sl.stop
        else:
            T = self.Tq
            while done < self.B and time.perf_counter() - t0 < budget_s:
                c_ = self.lens[done]
                R.helios_cpu_prefill_fp32(q[done * T:(done + 1) * T], pool, tabs[done], c_ - T, c_,
                                          self.scale)
                done += 1
        dt = time.perf_counter() - t0
        return done * self.Tq, dt, f"{done} of {self.B} sequences ({done * self.Tq} query tokens)"


class PrefillWorkload(Workload):
    """Config 4: 8 sequences each appending a 512-token chunk onto prior
    context U[0, 3584]; the first 64 blocks (1024 tokens) of every table are
    the same physical blocks wherever the prior context covers them."""

    bound = "mfma"

    def __init__(self, device, seed, kv_int8=False):
        import numpy as np
        import torch

        import helios_amd as H

        self.kv_int8 = kv_int8
        self.name = ("llama3-8b-int8-kv-chunked-prefill (config 4 shape, int8 pool)" if kv_int8
                     else "llama3-8b-fp16-chunked-prefill (config 4)")
        rng = np.random.default_rng(seed)
        gen = torch.Generator(device=device).manual_seed(seed)
        B, Hq, Hkv, D, T = 8, 32, 8, 128, 512
        self.B, self.Hq, self.Hkv, self.D, self.T = B, Hq, Hkv, D, T
        priors = [int(x) for x in rng.integers(0, 3585, size=B)]
        ctxs = [p + T for p in priors]
        shared = 64
        need = [(c + BLOCK - 1) // BLOCK for c in ctxs]
        own_shared = [min(shared, p // BLOCK) for p in priors]  # only full prior blocks alias
        nb = shared + sum(n - s for n, s in zip(need, own_shared))
        perm = [int(x) for x in rng.permutation(nb)]
        prefix, rest = perm[:shared], perm[shared:]
        tabs, o = [], 0
        for n, s in zip(need, own_shared):
            tabs.append(prefix[:s] + rest[o:o + n - s])
            o += n - s
        width = max(need)
        tab = np.zeros((B, width), np.int32)
        for i, t in enumerate(tabs):
            tab[i, :len(t)] = t
        self.tables_t = torch.from_numpy(tab).to(device)
        self.tabs = tabs
        self.priors, self.ctxs = priors, ctxs
        self.cache = H.PagedKVCache(nb, BLOCK, Hkv, D, dtype=torch.float16, device=device)
        for t in (self.cache.k_cache, self.cache.v_cache):
            t.normal_(generator=gen)
        if kv_int8:
            # the same values quantized by the library's write kernel, every
            # block written as one run of nb x 16 tokens
            fp = self.cache
            self.cache = H.QuantizedPagedKVCache(nb, BLOCK, Hkv, D, dtype=torch.float16, device=device,
                                                 scale_dtype=torch.float16)
            flat = [t.permute(0, 2, 1, 3).reshape(nb * BLOCK, Hkv, D) for t in (fp.k_cache, fp.v_cache)]
            H.write_kv(self.cache, [list(range(nb))], [0], flat[0], flat[1])
            del fp, flat
            torch.cuda.synchronize()
        self.q = torch.randn(B * T, Hq, D, generator=gen, device=device, dtype=torch.float16)
        self.qlens = torch.full((B,), T, dtype=torch.int32, device=device)
        self.cu = torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=device)
        self.pos_t = torch.tensor(priors, dtype=torch.int32, device=device)
        self.ctx_t = torch.tensor(ctxs, dtype=torch.int32, device=device)
        self.scale = 1.0 / math.sqrt(D)
        self.flops = 4 * D * Hq * sum(sum(p + i + 1 for i in range(T)) for p in priors)
        n_tab = sum(need)
        kvb = D + 2 if kv_int8 else 2 * D
        self.alg_bytes = sum(ctxs) * 2 * Hkv * kvb + 2 * B * T * Hq * D * 2 + 4 * n_tab
        self.tokens = B * T
        self.out = torch.empty_like(self.q)

    def step(self):
        import helios_amd as H

        return H.paged_attention_varlen(self.q, self.cache, self.tables_t, self.qlens, self.pos_t,
                                        self.ctx_t, self.scale, max_query_len=self.T,
                                        cu_query_lens=self.cu, out=self.out)

    def config(self):
        return {"workload": self.name, "sequences": self.B, "chunk": self.T,
                "n_q_heads": self.Hq, "n_kv_heads": self.Hkv, "head_dim": self.D,
                "block_size": BLOCK, "kv_dtype": "int8" if self.kv_int8 else "fp16",
                "prior_context": self.priors,
                "shared_prefix_blocks": 64}

    def cpu_baseline(self, budget_s):
        import numpy as np

        from oracle import paged_ref as R

        if self.kv_int8:
            pool = R.PagedPool(self.cache.num_blocks, BLOCK, self.Hkv, self.D, np.float32, quantized=True,
                               scale_dtype=np.float16)
            pool.k, pool.v = self.cache.k_cache.cpu().numpy(), self.cache.v_cache.cpu().numpy()
            pool.k_scale, pool.v_scale = self.cache.k_scale.cpu().numpy(), self.cache.v_scale.cpu().numpy()
        else:
            pool = R.PagedPool(self.cache.num_blocks, BLOCK, self.Hkv, self.D, np.float32)
            pool.k = self.cache.k_cache.float().cpu().numpy()
            pool.v = self.cache.v_cache.float().cpu().numpy()
        q = self.q.float().cpu().numpy()
        done, t0 = 0, time.perf_counter()
        while done < self.B and time.perf_counter() - t0 < budget_s:
            R.helios_cpu_prefill_fp32(q[done * self.T:(done + 1) * self.T], pool, self.tabs[done],
                                      self.priors[done], self.ctxs[done], self.scale)
            done += 1
        dt = time.perf_counter() - t0
        return done * self.T, dt, f"{done} of {self.B} sequences ({done * self.T} query tokens)"


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(wl, budget_s):
    """The oracle's restatement of helios' CPU route on a bounded sample,
    with every core this process may run on (n = len(sched_getaffinity))
    given to the BLAS pool."""
    n = len(os.sched_getaffinity(0))
    try:
        from threadpoolctl import threadpool_limits

        with threadpool_limits(limits=n, user_api="blas"):
            tokens, secs, sample = wl.cpu_baseline(budget_s)
    except ImportError:
        tokens, secs, sample = wl.cpu_baseline(budget_s)
    return {"value": round(tokens / secs, 1) if secs > 0 else None, "unit": "tokens/s",
            "cores": n, "cpu_model": _cpu_model(), "kind": "port", "sample": sample,
            "seconds": round(secs, 2)}


def time_steps(wl, steps, warmup, warmup_s, chunk=10):
    """`warmup` untimed steps, continued until at least `warmup_s` seconds
    have passed (the GPU clock needs tens of milliseconds of sustained work
    to ramp up), then exactly `steps` timed steps with a synchronisation on
    both sides.  The steps are timed in chunks of `chunk`, each between its
    own pair of HIP events on the stream the kernels run on (torch's current
    stream), and the result is the median over the chunks.  An event record
    between every two steps costs GPU time of its own (config 4 reads ~8%
    slower with one around every step).  The host enqueues faster than the
    GPU runs even config 2's 25 us steps, so the steps run back to back.
    (Holding the stream with a spin kernel while the host enqueued them let
    the clock drop: config 4 read 8% slower.)  Returns (median over the
    chunks of ms per step, ms per step from the first start to the last end,
    warmup steps run, seconds of the timed region by the host clock)."""
    import torch

    stream = torch.cuda.current_stream()
    done, t0 = 0, time.perf_counter()
    while done < warmup or time.perf_counter() - t0 < warmup_s:
        wl.step()
        done += 1
        if done % 50 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    sizes = [min(chunk, steps - i) for i in range(0, steps, chunk)]
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in sizes]
    t_wall = time.perf_counter()
    for (e0, e1), n in zip(ev, sizes):
        e0.record(stream)
        for _ in range(n):
            wl.step()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    per = sorted(e0.elapsed_time(e1) / n for (e0, e1), n in zip(ev, sizes))
    med = per[len(per) // 2] if len(per) % 2 else 0.5 * (per[len(per) // 2 - 1] + per[len(per) // 2])
    return med, ev[0][0].elapsed_time(ev[-1][1]) / steps, done, wall


def roofline(wl, ms, key):
    if wl.bound == "hbm":
        achieved = wl.alg_bytes / (ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": _traffic(key), "algorithmic_bytes": int(wl.alg_bytes)}
    else:
        achieved = wl.flops / (ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_F16_PEAK_TFS,
                "unit": "TFLOP/s", "frac": round(achieved / MFMA_F16_PEAK_TFS, 4),
                "traffic": _traffic(key), "algorithmic_flops": int(wl.flops)}
    roof["kernel"] = "decode_kernel" if wl.bound == "hbm" else "prefill_mfma_kernel"
    return roof


def _traffic(workload_key):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload_key}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def meta_bench(device, layers, steps, warmup, seed=4):
    """Wall time of one decode-verify step of config 5's batch over ``layers``
    layers, with the step's attention metadata (a) handed to every layer's
    call as the runner's Python lists (helios' pattern: exec/runner.py:261-268
    builds them, each layer's call converts them, triton_attn.py:156-165) and
    (b) prepared once per step in device-resident tables (DeviceBlockTables)
    and passed to every layer as device tensors.  Contexts grow by one token
    per step; a table gains a block when its context crosses a block
    boundary.  One pool serves every layer (the per-layer kernels are the
    same; only the metadata path differs)."""
    import numpy as np
    import torch

    import helios_amd as H

    wl = DecodeWorkload(5, device, seed)
    rng = np.random.default_rng(seed + 1)
    cache = wl.caches[0]
    nb = cache.num_blocks
    tables = [[int(x) for x in row[: (c + BLOCK - 1) // BLOCK]] for row, c in zip(wl.tables_np, wl.lens)]
    lens = list(wl.lens)
    Tq = wl.Tq
    width = max(len(t) for t in tables) + (steps + warmup + 10) // BLOCK + 2
    tabs = H.DeviceBlockTables.for_cache(cache, wl.B, width)
    q = wl.q

    def advance():
        for i in range(len(lens)):
            lens[i] += 1
            if (lens[i] + BLOCK - 1) // BLOCK > len(tables[i]):
                tables[i].append(int(rng.integers(nb)))

    def step_lists():
        advance()
        for _ in range(layers):
            H.paged_attention_verify_batched(q, cache, tables, lens, Tq, wl.scale)

    prep = []

    def step_device():
        advance()
        t0 = time.perf_counter()
        meta = tabs.prepare(range(len(lens)), tables, lens, [c - Tq for c in lens], [Tq] * len(lens), True)
        prep.append(time.perf_counter() - t0)
        for _ in range(layers):
            H.batched_attention(q, cache, meta, wl.scale)

    res = {}
    for name, fn in (("lists", step_lists), ("device", step_device)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        prep.clear()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record()
        for _ in range(steps):
            fn()
        ev1.record()
        torch.cuda.synchronize()
        res[name] = ((time.perf_counter() - t0) * 1e3 / steps, ev0.elapsed_time(ev1) / steps)
        print(f"{name}: {res[name][0]:.3f} ms/step wall", file=sys.stderr, flush=True)
    # prepare's own host cost, with the GPU idle (in the loop above it also
    # waits whenever the host runs two steps ahead of the GPU)
    idle = []
    for _ in range(10):
        advance()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        meta = tabs.prepare(range(len(lens)), tables, lens, [c - Tq for c in lens], [Tq] * len(lens), True)
        idle.append(time.perf_counter() - t0)
    torch.cuda.synchronize()
    # the layers' kernels alone, metadata already on the device
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        for _ in range(layers):
            H.batched_attention(q, cache, meta, wl.scale)
    ev1.record()
    torch.cuda.synchronize()
    kernels_ms = ev0.elapsed_time(ev1) / steps
    print(json.dumps({
        "metric": f"decode-verify step wall time over {layers} layers (config 5 batch): "
                  "device-resident step metadata vs per-layer Python lists",
        "value": round(res["device"][0], 3), "unit": "ms/step", "higher_is_better": False,
        "lists_ms_per_step": round(res["lists"][0], 3),
        "kernels_only_ms_per_step": round(kernels_ms, 3),
        "prepare_us_median_in_loop": round(float(np.median(prep)) * 1e6, 1),
        "prepare_us_median_gpu_idle": round(float(np.median(idle)) * 1e6, 1),
        "steps": steps, "warmup": warmup, "layers": layers,
        "config": {"workload": wl.name, "batch": wl.B, "q_per_seq": Tq},
    }))


def graph_bench(device, cfg, layers, steps, warmup):
    """One decode step of config `cfg`'s batch through `layers` layers (each
    with its own pool copy, metadata on the device): launched eagerly, layer
    by layer, and replayed as one captured HIP graph.  Small batches are
    where the per-launch cost shows."""
    import torch

    import helios_amd as H

    wl = DecodeWorkload(cfg, device, cfg - 1, 0, layers)
    tabs = H.DeviceBlockTables.for_cache(wl.caches[0], wl.B, wl.tables_np.shape[1])
    tables = [[int(x) for x in row[: (c + BLOCK - 1) // BLOCK]] for row, c in zip(wl.tables_np, wl.lens)]
    meta = tabs.prepare(range(wl.B), tables, wl.lens, [c - wl.Tq for c in wl.lens], [wl.Tq] * wl.B, True)
    outs = [torch.empty_like(wl.q) for _ in range(layers)]
    ks = [c._scales() for c in wl.caches]

    def step():
        for li, c in enumerate(wl.caches):
            H.paged_attention_decode_hip(wl.q, c.k_cache, c.v_cache, meta.block_tables, meta.context_lens,
                                         wl.scale, ks[li][0], ks[li][1], q_per_seq=wl.Tq,
                                         max_context_len=meta.max_context_len, out=outs[li])

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    res = {}
    for name, fn in (("eager", step), ("graph", g.replay)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name] = e0.elapsed_time(e1) / steps
        print(f"{name}: {res[name] * 1e3 / layers:.2f} us per layer", file=sys.stderr, flush=True)
    print(json.dumps({
        "metric": f"decode step over {layers} layers ({wl.name}): eager launches vs one captured HIP graph",
        "value": round(res["graph"], 4), "unit": "ms/step", "higher_is_better": False,
        "eager_ms_per_step": round(res["eager"], 4),
        "graph_us_per_layer": round(res["graph"] * 1e3 / layers, 2),
        "eager_us_per_layer": round(res["eager"] * 1e3 / layers, 2),
        "hbm_gbs_graph": round(wl.alg_bytes * layers / (res["graph"] * 1e-3) / 1e9, 1),
        "steps": steps, "warmup": warmup, "layers": layers,
        "config": {"workload": wl.name, "batch": wl.B, "q_per_seq": wl.Tq},
    }))


def spec_bench(device, gamma, steps, warmup, seed=4, qdtype=None):
    """Attention work of one speculative step for config 5's batch, one
    layer: gamma draft decodes over an int8 KV shadow (each writing its
    token), the verify pass (gamma tokens per sequence written to and
    attended over the int8 target cache) and the shadow's re-sync (gamma
    tokens written and attended).  Batched: 2 gamma + 4 launches for the
    whole batch (DeviceAttnMeta.advanced / .verify).  Per sequence, as
    helios runs speculation (exec/runner.py:131-133, :302-406): the same
    calls once per sequence."""
    import numpy as np
    import torch

    import helios_amd as H

    wl = DecodeWorkload(5, device, seed, qdtype=qdtype)
    dt = wl.q.dtype
    target = wl.caches[0]
    shadow = H.QuantizedPagedKVCache(target.num_blocks, BLOCK, wl.Hkv, wl.D, dtype=dt,
                                     device=device, scale_dtype=torch.float16)
    for a, b in ((shadow.k_cache, target.k_cache), (shadow.v_cache, target.v_cache),
                 (shadow.k_scale, target.k_scale), (shadow.v_scale, target.v_scale)):
        a.copy_(b)
    B, Hq, Hkv, D = wl.B, wl.Hq, wl.Hkv, wl.D
    # contexts leave room for the gamma speculative positions inside the last block
    lens = [max(1, c - gamma) for c in wl.lens]
    tables = [[int(x) for x in row[: (c + BLOCK - 1) // BLOCK]] for row, c in zip(wl.tables_np, wl.lens)]
    tabs = H.DeviceBlockTables.for_cache(target, B, max(len(t) for t in tables))
    gen = torch.Generator(device=device).manual_seed(seed)
    q1 = torch.randn(B, Hq, D, generator=gen, device=device, dtype=dt)
    k1 = torch.randn(B, Hkv, D, generator=gen, device=device, dtype=dt)
    qg = torch.randn(B * gamma, Hq, D, generator=gen, device=device, dtype=dt)
    kg = torch.randn(B * gamma, Hkv, D, generator=gen, device=device, dtype=dt)
    base = tabs.prepare(range(B), tables, lens, [c - 1 for c in lens], [1] * B, True)
    drafts = [base.advanced(j) for j in range(gamma)]
    vm = base.verify(gamma)
    sc = wl.scale

    def batched():
        for m in drafts:
            H.write_kv_batched(shadow, m, k1, k1)
            H.batched_attention(q1, shadow, m, sc)
        H.write_kv_batched(target, vm, kg, kg)
        H.batched_attention(qg, target, vm, sc)
        H.write_kv_batched(shadow, vm, kg, kg)
        H.batched_attention(qg, shadow, vm, sc)

    def per_sequence():
        for b in range(B):
            t, c = tables[b], lens[b]
            for j in range(gamma):
                shadow.write(t, c - 1 + j, k1[b:b + 1], k1[b:b + 1])
                H.paged_attention_decode(q1[b], shadow, t, c + j, sc)
            qb, kb = qg[b * gamma:(b + 1) * gamma], kg[b * gamma:(b + 1) * gamma]
            target.write(t, c - 1, kb, kb)
            H.paged_attention_prefill(qb, target, t, c - 1, c + gamma - 1, sc)
            shadow.write(t, c - 1, kb, kb)
            H.paged_attention_prefill(qb, shadow, t, c - 1, c + gamma - 1, sc)

    res = {}
    for name, fn, n, w in (("batched", batched, steps, warmup), ("per_sequence", per_sequence, 2, 1)):
        for _ in range(w):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        res[name] = (time.perf_counter() - t0) * 1e3 / n
        print(f"{name}: {res[name]:.3f} ms per layer-step", file=sys.stderr, flush=True)
    # K/V bytes read (int8 payload + fp16 scale per token, head and tensor):
    # draft j attends context + j, verify and re-sync attend context + gamma - 1
    row = 2 * Hkv * (D + 2)
    kv_read = sum(lens) * row
    alg = gamma * kv_read + B * (gamma * (gamma - 1) // 2) * row + 2 * (kv_read + B * (gamma - 1) * row)
    print(json.dumps({
        "metric": f"speculative step attention (gamma {gamma}, int8 target + int8 draft shadow, "
                  "config 5 batch, one layer): batched vs per sequence",
        "value": round(res["batched"], 3), "unit": "ms per layer-step", "higher_is_better": False,
        "per_sequence_ms": round(res["per_sequence"], 3),
        "launches_batched": 2 * (gamma + 2), "launches_per_sequence": 2 * (gamma + 2) * B,
        "hbm_gbs_batched": round(alg / (res["batched"] * 1e-3) / 1e9, 1),
        "algorithmic_bytes": int(alg),
        "config": {"workload": wl.name, "batch": B, "gamma": gamma, "q_dtype": str(dt).replace("torch.", "")},
    }))


def helios_shape_bench(device, steps, warmup):
    """helios' only published measurement of this path
    (tests/parity/test_triton_parity.py:125-175; numbers in
    exec/triton_attn.py:3-7): fp16 paged decode of 32 sequences x 512
    context, Hq 32 / Hkv 8, head_dim 128, block 16, sequence i on blocks
    [32 i, 32 i + 32), pool and queries drawn after torch.manual_seed(3).
    Timed two ways:
    - the kernel alone: median over chunks of 10 calls between HIP event
      pairs, with int32 device tables and lengths;
    - helios' own protocol: wall clock over 20 calls after 5 warmups,
      synchronised before and after, through paged_attention_decode_hip with
      Python lists (converted per call, as helios' wrapper does).
    helios measured 2.676 ms (Triton) and 14.089 ms (PyTorch path) on a
    Tesla T4; that is other hardware, so no ratio is reported as a
    baseline.  The 67 MB pool fits in the 256 MB Infinity Cache and, as in
    helios' protocol, every call reads the same pool, so repeated calls are
    served largely from that cache rather than HBM."""
    import torch

    import helios_amd as H

    torch.manual_seed(3)
    bs, hkv, hq, d, n, ctx = 16, 8, 32, 128, 32, 512
    need = ctx // bs
    cache = H.PagedKVCache(n * need + 8, bs, hkv, d, dtype=torch.float16, device=device)
    cache.k_cache.normal_()
    cache.v_cache.normal_()
    tables = [[i * need + j for j in range(need)] for i in range(n)]
    lens = [ctx] * n
    q = torch.randn(n, hq, d, dtype=torch.float16, device=device)
    tt = torch.tensor(tables, dtype=torch.int32, device=device)
    lt = torch.tensor(lens, dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    ws = H.decode_workspace(n, 1, hq, hkv, d, ctx, device=device)

    def call():
        H.paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tt, lt, max_context_len=ctx, out=out,
                                     workspace=ws)

    stream = torch.cuda.current_stream(device)
    for _ in range(max(warmup, 5)):
        call()
    torch.cuda.synchronize()
    chunks = max(1, steps // 10)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(chunks)]
    for a, b in ev:
        a.record(stream)
        for _ in range(10):
            call()
        b.record(stream)
    torch.cuda.synchronize()
    ms = sorted(a.elapsed_time(b) / 10 for a, b in ev)
    kernel_ms = ms[len(ms) // 2]

    def helios_protocol():
        return H.paged_attention_decode_hip(q, cache.k_cache, cache.v_cache, tables, lens)

    for _ in range(5):
        helios_protocol()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        helios_protocol()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / 20
    kv_bytes = n * ctx * 2 * hkv * d * 2
    print(json.dumps({
        "metric": "paged decode at helios' published shape (32 seqs x 512 ctx, Hq 32 / Hkv 8, D 128, fp16, "
                  "block 16)",
        "value": round(kernel_ms, 4), "unit": "ms per call", "higher_is_better": False,
        "kernel_ms": round(kernel_ms, 4),
        "helios_protocol_wall_ms": round(wall_ms, 4),
        "kv_gbs_kernel": round(kv_bytes / (kernel_ms * 1e-3) / 1e9, 1),
        "kv_bytes": kv_bytes,
        "reference_published": {"hardware": "Tesla T4", "triton_ms": 2.676, "pytorch_ms": 14.089,
                                "source": "exec/triton_attn.py:3-7"},
        "vs_baseline": None,
        "dtype": "f16", "data": "synthetic (torch.manual_seed(3), N(0,1) pool and queries)",
    }))


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=5, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--dtype", choices=["fp16", "bf16"], default="fp16",
                    help="query (and fp pool) dtype of the decode configs 2, 3, 5 and --spec-gamma")
    ap.add_argument("--kv-int8", action="store_true",
                    help="config 4 on an int8 pool (the same values quantized by the write kernel)")
    ap.add_argument("--part-tokens", type=int, default=0,
                    help="split-K partition size for decode (0 = library default)")
    ap.add_argument("--copies", type=int, default=None,
                    help="pool copies rotated per step (default: enough to exceed 256 MB)")
    ap.add_argument("--warmup-s", type=float, default=1.0,
                    help="untimed warmup continues until this many seconds have passed")
    ap.add_argument("--cpu-budget", type=float, default=15.0,
                    help="seconds of CPU baseline work (0 disables it)")
    ap.add_argument("--no-prefill", action="store_true",
                    help="config 5 only: skip the config-4 prefill measured beside it")
    ap.add_argument("--meta-layers", type=int, default=0, metavar="L",
                    help="only time a decode-verify step over L layers with device-resident "
                         "vs per-layer list metadata, print its own JSON line, and exit")
    ap.add_argument("--graph-layers", type=int, default=0, metavar="L",
                    help="only time --config's decode step over L layers, eager vs one captured "
                         "HIP graph, print its own JSON line, and exit")
    ap.add_argument("--spec-gamma", type=int, default=0, metavar="G",
                    help="only time one speculative step's attention (gamma G, config 5 batch) "
                         "batched vs per sequence, print its own JSON line, and exit")
    ap.add_argument("--helios-shape", action="store_true",
                    help="time the decode at helios' only published shape (32 seqs x 512 ctx, fp16) instead")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (the known-size kernel "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and exit")
    args = ap.parse_args()

    if args.calibrate_copy:
        import torch

        n = args.calibrate_copy << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n, "copies": 5}))
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the paged-attention path "
                                   "has no multi-GPU mode (sequences and KV heads shard "
                                   "without exchange; one GPU's share is what is measured)",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    import helios_amd  # noqa: F401

    qdt = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    device = torch.device("cuda:0")
    if args.graph_layers:
        graph_bench(device, args.config, args.graph_layers, min(args.steps, 100), min(args.warmup, 20))
        return
    if args.spec_gamma:
        spec_bench(device, args.spec_gamma, min(args.steps, 50), min(args.warmup, 20), qdtype=qdt)
        return
    if args.helios_shape:
        helios_shape_bench(device, args.steps, args.warmup)
        return
    if args.meta_layers:
        meta_bench(device, args.meta_layers, min(args.steps, 20), min(args.warmup, 5))
        return
    seed = args.config - 1 if args.seed is None else args.seed

    if args.config == 4:
        wl = PrefillWorkload(device, seed, kv_int8=args.kv_int8)
    else:
        copies = args.copies
        if copies is None:
            copies = 1 if args.config in (1, 5) else 5
        wl = DecodeWorkload(args.config, device, seed, args.part_tokens, copies,
                            qdtype=qdt if args.config in (2, 3, 5) else None)

    print(f"bench: {wl.name} built; timing {args.steps} steps", file=sys.stderr, flush=True)
    ms_step, ms_run, warm_done, wall = time_steps(wl, args.steps, args.warmup, args.warmup_s)
    print(f"bench: {ms_step * 1e3:.1f} us per step; CPU baseline next", file=sys.stderr, flush=True)
    key = f"config{args.config}" + ("_int8" if args.kv_int8 else "")
    value = wl.tokens / (ms_step * 1e-3)
    cpu = cpu_baseline(wl, args.cpu_budget) if args.cpu_budget > 0 else None

    line = {
        "metric": "paged-attn decode tokens/s + achieved HBM GB/s (% peak) on 1 MI355X"
        if wl.bound == "hbm" else "paged-attn chunked-prefill tokens/s + MFMA TFLOP/s (% peak) on 1 MI355X",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_s": args.warmup_s,
        "warmup_steps_run": warm_done,
        "ms_per_step": round(ms_step, 5),
        "ms_per_step_run": round(ms_run, 5),
        "timing": "median over chunks of 10 steps, each chunk between its own HIP event pair on the kernels' "
                  "stream; ms_per_step_run = first start to last end / steps",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("int8-kv/" + ("bf16" if qdt == torch.bfloat16 and args.config != 4 else "fp16"))
        if (getattr(wl, "quant", False) or getattr(wl, "kv_int8", False)) else
        ("f32" if args.config == 1 else ("bf16" if qdt == torch.bfloat16 and args.config != 4 else "f16")),
        "data": "synthetic (seeded N(0,1); int8 KV quantized on the GPU by the library's write kernel)",
        "config": wl.config(),
        "roofline": roofline(wl, ms_step, key),
        "cpu_baseline": cpu,
        "wall_s_timed_region": round(wall, 4),
    }
    if args.config == 5 and not args.no_prefill:
        # config 4 (the MFMA-bound chunked prefill) measured in the same run
        pw = PrefillWorkload(device, 3)
        print(f"bench: {pw.name} built; timing {args.steps} steps", file=sys.stderr, flush=True)
        pms, pms_run, pwarm, _ = time_steps(pw, args.steps, args.warmup, args.warmup_s)
        print(f"bench: {pms * 1e3:.1f} us per step; CPU baseline next", file=sys.stderr, flush=True)
        line["prefill"] = {
            "metric": "paged-attn chunked-prefill tokens/s + MFMA TFLOP/s (% peak) on 1 MI355X",
            "value": round(pw.tokens / (pms * 1e-3), 1), "unit": "tokens/s",
            "ms_per_step": round(pms, 5), "ms_per_step_run": round(pms_run, 5),
            "warmup_steps_run": pwarm, "dtype": "f16", "config": pw.config(),
            "roofline": roofline(pw, pms, "config4"),
            "cpu_baseline": cpu_baseline(pw, args.cpu_budget) if args.cpu_budget > 0 else None,
        }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
