"""Token-identical greedy decode on helios' toy model.

tests/golden/toy_greedy.json holds helios' own greedy tokens for its toy model
(TOY_CONFIG, seed 0; reference tests/parity/test_parity.py:36-53, :273-304),
written by tests/golden/make_toy_greedy.py.  The toy model is restated in
tests/toy_model.py; its weights are pinned by helios' per-parameter checksums.
The CPU test drives it with the NumPy oracle's paged attention, the GPU test
with libheliosattn.so (fp32 pool, as helios' CPU engine runs it, engine.py:135-138),
both over a shuffled, non-contiguous block table.  Every step's top-1 / top-2
logit margin in the fixture is >= 6e-4, far above fp32 attention's rounding
differences, so the tokens must match exactly.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import paged_ref as R
from tests.toy_model import TOY, AttentionBackend, ToyModel, checksums, greedy, toy_weights

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "toy_greedy.json")
BS, NUM_BLOCKS = 16, 64


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def weights():
    return toy_weights(TOY, seed=0)


def _table(n_tokens: int, seed: int):
    need = (n_tokens + BS - 1) // BS
    return [int(b) for b in np.random.default_rng(seed).permutation(NUM_BLOCKS)[:need]]


class OracleAttention(AttentionBackend):
    def __init__(self, n_kv_heads, head_dim):
        self.nkv, self.hd = n_kv_heads, head_dim

    def new_cache(self, layer):
        return R.PagedPool(NUM_BLOCKS, BS, self.nkv, self.hd, np.float32)

    def write(self, cache, block_ids, start_pos, k, v):
        cache.write(block_ids, start_pos, k.numpy(), v.numpy())

    def decode(self, q, cache, block_ids, context_len, scale):
        return torch.from_numpy(R.paged_decode(q.double().numpy(), cache, block_ids, context_len, scale)).float()

    def prefill(self, q, cache, block_ids, start_pos, context_len, scale):
        out = R.paged_prefill(q.double().numpy(), cache, block_ids, start_pos, context_len, scale)
        return torch.from_numpy(out).float()


def test_restated_weights_match_helios_checksums(golden, weights):
    ref = golden["weights"]
    got = checksums(weights)
    assert set(ref) == set(got)
    for name, (s, ss) in got.items():
        assert list(weights[name].shape) == ref[name]["shape"], name
        assert s == pytest.approx(ref[name]["sum"], rel=1e-9, abs=1e-9), name
        assert ss == pytest.approx(ref[name]["sumsq"], rel=1e-9), name


def test_golden_margins_leave_headroom(golden):
    for case in golden["cases"]:
        assert min(case["margins"]) > 5e-4
        assert len(case["tokens"]) == case["n_new"]


def test_toy_greedy_with_oracle_attention_matches_helios(golden, weights):
    model = ToyModel(weights, "cpu")
    attn = OracleAttention(TOY["num_key_value_heads"], model.hd)
    for i, case in enumerate(golden["cases"]):
        table = _table(len(case["prompt"]) + case["n_new"], seed=10 + i)
        with torch.inference_mode():
            toks = greedy(model, attn, case["prompt"], case["n_new"], table)
        assert toks == case["tokens"], f"case {i}"


class HipAttention(AttentionBackend):
    def __init__(self, n_kv_heads, head_dim):
        import helios_amd as H

        self.H, self.nkv, self.hd = H, n_kv_heads, head_dim

    def new_cache(self, layer):
        return self.H.PagedKVCache(NUM_BLOCKS, BS, self.nkv, self.hd, dtype=torch.float32, device="cuda")

    def write(self, cache, block_ids, start_pos, k, v):
        cache.write(block_ids, start_pos, k, v)

    def decode(self, q, cache, block_ids, context_len, scale):
        return self.H.paged_attention_decode(q, cache, block_ids, context_len, scale)

    def prefill(self, q, cache, block_ids, start_pos, context_len, scale):
        return self.H.paged_attention_prefill(q, cache, block_ids, start_pos, context_len, scale)


@pytest.mark.gpu
def test_toy_greedy_with_hip_attention_matches_helios(golden, weights):
    model = ToyModel(weights, "cuda")
    attn = HipAttention(TOY["num_key_value_heads"], model.hd)
    for i, case in enumerate(golden["cases"]):
        print(f"toy greedy case {i}: prompt {len(case['prompt'])} tokens, {case['n_new']} new", flush=True)
        table = _table(len(case["prompt"]) + case["n_new"], seed=10 + i)
        with torch.inference_mode():
            toks = greedy(model, attn, case["prompt"], case["n_new"], table)
        torch.cuda.synchronize()
        assert toks == case["tokens"], f"case {i}"


class HipAttentionFusedRope(HipAttention):
    """K rotated inside the cache write (write_kv with the model's tables)."""

    fused_rope = True

    def __init__(self, n_kv_heads, head_dim, cos, sin):
        super().__init__(n_kv_heads, head_dim)
        self.cos, self.sin = cos.contiguous(), sin.contiguous()

    def write(self, cache, block_ids, start_pos, k, v):
        self.H.write_kv(cache, [list(block_ids)], [start_pos], k, v, rope=(self.cos, self.sin))


@pytest.mark.gpu
def test_toy_greedy_with_fused_rope_write_matches_helios(golden, weights):
    model = ToyModel(weights, "cuda")
    attn = HipAttentionFusedRope(TOY["num_key_value_heads"], model.hd, model.cos, model.sin)
    for i, case in enumerate(golden["cases"]):
        print(f"toy greedy (fused rope write) case {i}", flush=True)
        table = _table(len(case["prompt"]) + case["n_new"], seed=20 + i)
        with torch.inference_mode():
            toks = greedy(model, attn, case["prompt"], case["n_new"], table)
        torch.cuda.synchronize()
        assert toks == case["tokens"], f"case {i}"
