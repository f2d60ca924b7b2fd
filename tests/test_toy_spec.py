"""Batched speculative decoding on helios' toy model, on the device-resident
step metadata and the int8 draft-KV shadow.

helios speculates one sequence at a time (exec/runner.py:302-406): gamma
draft decodes, one verify pass over [last] + drafted[:-1], greedy accept of
the matching prefix plus a bonus token, then a re-sync of the draft's KV
shadow (a QuantizedPagedKVCache per layer, runner.py:76-94) over the
committed tokens.  Here every sequence of the batch speculates together:
each draft step is one decode launch over the shadow (DeviceAttnMeta.advanced),
the verify is one launch with gamma query tokens per sequence
(DeviceAttnMeta.verify), and the re-sync reuses the verify metadata on the
shadow.  The committed tokens must equal helios' own greedy tokens
(tests/golden/toy_greedy.json) exactly, in both of helios' modes
(tests/parity/test_parity.py:231-253, tests/quant/test_qassd.py:147-193):

  symmetric   draft = target model, writing the target's fp32 caches; every
              draft is accepted
  asymmetric  draft = int4-rounded weights (tests/toy_model.py
              int4_draft_weights), writing an int8 KV shadow; some drafts
              are rejected, and the output still equals the target's
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from tests.toy_model import TOY, ToyModel, int4_draft_weights, toy_weights

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "toy_greedy.json")
BS, NUM_BLOCKS = 16, 64


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def _attend(meta, scale):
    import helios_amd as H

    def attend(cache, q, k, v):
        H.write_kv_batched(cache, meta, k, v)
        return H.batched_attention(q, cache, meta, scale)

    return attend


def speculate(target, draft, tcaches, dcaches, cases, gamma, resync):
    """Greedy generation of every case at once; returns the tokens per case
    and (drafted, accepted) counts."""
    import helios_amd as H

    rng = np.random.default_rng(gamma)
    perm = [int(b) for b in rng.permutation(NUM_BLOCKS)]
    tables, o = [], 0
    for c in cases:
        need = (len(c["prompt"]) + c["n_new"] + gamma + 2 + BS - 1) // BS
        tables.append(perm[o:o + need])
        o += need
    tabs = H.DeviceBlockTables.for_cache(tcaches[0], len(cases), 8)
    scale = target.scale

    # prefill every prompt in one ragged batch, target and draft
    ids = list(range(len(cases)))
    plens = [len(c["prompt"]) for c in cases]
    meta = tabs.prepare(ids, tables, plens, [0] * len(cases), plens, False)
    toks = [t for c in cases for t in c["prompt"]]
    pos = [p for n in plens for p in range(n)]
    logits = target.forward_tokens(toks, pos, tcaches, _attend(meta, scale))
    if resync:
        draft.forward_tokens(toks, pos, dcaches, _attend(meta, scale))
    last_rows = np.cumsum(plens) - 1
    committed = [[int(torch.argmax(logits[r]))] for r in last_rows]
    ctx = [n + 1 for n in plens]
    drafted_n = accepted_n = 0

    while True:
        act = [b for b in ids if len(committed[b]) < cases[b]["n_new"]]
        if not act:
            break
        base = tabs.prepare(act, [tables[b] for b in act], [ctx[b] for b in act],
                            [ctx[b] - 1 for b in act], [1] * len(act), True)
        # draft: gamma one-token steps over the draft's KV
        cur = [committed[b][-1] for b in act]
        drafted = [[] for _ in act]
        for j in range(gamma):
            lg = draft.forward_tokens(cur, [ctx[b] - 1 + j for b in act], dcaches,
                                      _attend(base.advanced(j), scale))
            cur = torch.argmax(lg, dim=-1).tolist()
            for i, t in enumerate(cur):
                drafted[i].append(t)
        # verify: gamma tokens per sequence in one pass over the target's KV
        vm = base.verify(gamma)
        vt = [t for i, b in enumerate(act) for t in [committed[b][-1]] + drafted[i][:-1]]
        vp = [ctx[b] - 1 + t for b in act for t in range(gamma)]
        vl = target.forward_tokens(vt, vp, tcaches, _attend(vm, scale)).view(len(act), gamma, -1)
        best = torch.argmax(vl, dim=-1).tolist()
        new = []
        for i, b in enumerate(act):
            n_acc = 0
            while n_acc < gamma and best[i][n_acc] == drafted[i][n_acc]:
                n_acc += 1
            nt = drafted[i][:n_acc] + ([best[i][n_acc]] if n_acc < gamma else [])
            drafted_n += gamma
            accepted_n += n_acc
            new.append(nt)
        # re-sync the draft's shadow over the committed tokens (padded to gamma)
        if resync:
            rt = [t for i, b in enumerate(act) for t in ([committed[b][-1]] + new[i][:-1] + [0] * gamma)[:gamma]]
            draft.forward_tokens(rt, vp, dcaches, _attend(vm, scale))
        for i, b in enumerate(act):
            committed[b].extend(new[i])
            ctx[b] += len(new[i])
    torch.cuda.synchronize()
    return [c[: cases[b]["n_new"]] for b, c in enumerate(committed)], drafted_n, accepted_n


@pytest.mark.parametrize("gamma", [1, 2, 4])
def test_symmetric_speculation_matches_greedy(golden, gamma):
    import helios_amd as H

    print(f"symmetric speculation gamma {gamma}", flush=True)
    model = ToyModel(toy_weights(TOY, seed=0), "cuda")
    caches = [H.PagedKVCache(NUM_BLOCKS, BS, TOY["num_key_value_heads"], model.hd, dtype=torch.float32,
                             device="cuda") for _ in range(TOY["num_hidden_layers"])]
    with torch.inference_mode():
        toks, drafted, accepted = speculate(model, model, caches, caches, golden["cases"], gamma, False)
    for b, case in enumerate(golden["cases"]):
        assert toks[b] == case["tokens"], f"case {b}"
    assert drafted > 0 and accepted == drafted


@pytest.mark.parametrize("gamma", [2, 4])
def test_asymmetric_speculation_with_int8_shadow_matches_greedy(golden, gamma):
    import helios_amd as H

    print(f"asymmetric speculation (int8 shadow) gamma {gamma}", flush=True)
    w = toy_weights(TOY, seed=0)
    target = ToyModel(w, "cuda")
    draft = ToyModel(int4_draft_weights(w), "cuda")
    L, Hkv, D = TOY["num_hidden_layers"], TOY["num_key_value_heads"], target.hd
    tcaches = [H.PagedKVCache(NUM_BLOCKS, BS, Hkv, D, dtype=torch.float32, device="cuda") for _ in range(L)]
    shadow = [H.QuantizedPagedKVCache(NUM_BLOCKS, BS, Hkv, D, dtype=torch.float32, device="cuda")
              for _ in range(L)]
    with torch.inference_mode():
        toks, drafted, accepted = speculate(target, draft, tcaches, shadow, golden["cases"], gamma, True)
    for b, case in enumerate(golden["cases"]):
        assert toks[b] == case["tokens"], f"case {b}"
    print(f"  acceptance {accepted}/{drafted}", flush=True)
    assert drafted > 0 and 0 < accepted < drafted
