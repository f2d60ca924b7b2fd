"""Step metadata kept on the device: the oracle's restatement of helios'
per-step BatchedAttnMeta, and the host half of DeviceBlockTables (row
residency, changed-suffix deltas, packing), checked on the CPU against a
NumPy model of hpa_step_tables."""

from __future__ import annotations

import random

import numpy as np
import pytest

import torch

from helios_amd.step_meta import DeviceAttnMeta, TableResidency, make_group, step_groups
from oracle import step_meta_ref as M

ENTRY = 5


# ------------------------------------------------------------------ oracle


def test_prefill_meta_hand_example():
    items = [M.PrefillItem(7, [1, 2, 3], 0, [4, 9]), M.PrefillItem(3, [5, 6], 16, [2, 8])]
    m = M.prefill_meta(items)
    assert m.token_slices == [(0, 3), (3, 5)]
    assert m.block_tables == [[4, 9], [2, 8]]
    assert m.context_lens == [3, 18]
    assert m.start_positions == [0, 16]
    assert m.is_decode is False


def test_decode_meta_hand_example():
    items = [M.DecodeItem(1, 42, 16, [3, 5], 17), M.DecodeItem(2, 43, 0, [6], 1)]
    m = M.decode_meta(items)
    assert m.token_slices == [(0, 1), (1, 2)]
    assert m.block_tables == [[3, 5], [6]]
    assert m.context_lens == [17, 1]
    assert m.start_positions == [16, 0]
    assert m.is_decode is True


def test_padded_tables_hand_examples():
    np.testing.assert_array_equal(M.padded_tables([[3, 1], [7], []]), [[3, 1], [7, 0], [0, 0]])
    assert M.padded_tables([]).shape == (0, 1)
    assert M.padded_tables([[], []]).shape == (2, 0)


def test_runner_invariants():
    rng = random.Random(5)
    items = [M.PrefillItem(i, [0] * rng.randint(1, 40), rng.randint(0, 300), [0] * 30) for i in range(9)]
    m = M.prefill_meta(items)
    assert m.token_slices[0][0] == 0
    for (a, b), (c, d) in zip(m.token_slices, m.token_slices[1:]):
        assert b == c
    for (lo, hi), it, c, s in zip(m.token_slices, items, m.context_lens, m.start_positions):
        assert hi - lo == it.num_tokens and c == s + it.num_tokens


# --------------------------------------------- host planner vs the oracle


def apply_plan(plan, resident: np.ndarray) -> np.ndarray:
    """hpa_step_tables as include/helios_attn.h states it: write each entry's
    replaced suffix into its resident row, then gather the row (entries >=
    n_blocks as 0) into [n, width]."""
    p = plan.packed
    ent = p[: ENTRY * plan.n_entries].reshape(plan.n_entries, ENTRY)
    new = p[plan.new_ids_offset: plan.new_ids_offset + plan.n_new_ids]
    out = np.zeros((plan.n_entries, plan.width), dtype=np.int32)
    for e, (row, nb, first, count, off) in enumerate(ent):
        resident[row, first: first + count] = new[off: off + count]
        nb = min(nb, resident.shape[1], plan.width)
        out[e, :nb] = resident[row, :nb]
    return out


def check_against_oracle(plan, step_tables, metas_ref):
    for (e0, n, off, g), ref in zip(plan.groups, metas_ref):
        p = plan.packed
        got = step_tables[e0: e0 + n]
        want = M.padded_tables(ref.block_tables)
        w = want.shape[1]
        np.testing.assert_array_equal(got[:, :w], want)
        assert not got[:, w:].any()
        np.testing.assert_array_equal(p[off: off + n], ref.context_lens)
        np.testing.assert_array_equal(p[off + n: off + 2 * n], ref.start_positions)
        cu = p[off + 2 * n: off + 3 * n + 1]
        assert [(int(cu[b]), int(cu[b + 1])) for b in range(n)] == ref.token_slices


class Sim:
    """A toy scheduler: sequences arrive with a prompt, prefill in chunks,
    decode token by token, take copy-on-write replacements, get preempted
    (blocks freed, later re-admitted with new blocks) and finish."""

    def __init__(self, seed, bs=4, pool=4096, unique=False):
        self.rng = random.Random(seed)
        self.bs, self.pool = bs, pool
        self.seqs = {}
        self.next_id = 0
        # unique: blocks come from a free list (no two live sequences share
        # one), as helios' allocator hands them out; else ids are random
        self.unique = unique
        self.free = list(range(pool))
        self.rng.shuffle(self.free)

    def _blocks(self, n):
        if self.unique:
            out, self.free = self.free[:n], self.free[n:]
            assert len(out) == n, "pool exhausted"
            return out
        return [self.rng.randrange(self.pool) for _ in range(n)]

    def _free(self, blocks):
        if self.unique:
            self.free.extend(blocks)

    def step(self, max_batch):
        r = self.rng
        while len(self.seqs) < max_batch and r.random() < 0.5:
            plen = r.randint(1, 60)
            self.seqs[self.next_id] = dict(prompt=plen, done=0, ctx=0, blocks=[], preempted=False)
            self.next_id += 1
        pre, dec, finished, preempted = [], [], [], []
        for sid, s in list(self.seqs.items()):
            x = r.random()
            if x < 0.03:
                finished.append(sid)
                self._free(s["blocks"])
                del self.seqs[sid]
                continue
            if x < 0.05:
                preempted.append(sid)
                self._free(s["blocks"])
                s.update(done=0, ctx=0, blocks=[])
                continue
            if x < 0.15:
                continue  # not scheduled this step
            if s["blocks"] and r.random() < 0.05:
                i = r.randrange(len(s["blocks"]))  # copy-on-write
                self._free([s["blocks"][i]])
                s["blocks"][i] = self._blocks(1)[0]
            if s["done"] < s["prompt"]:
                n = min(r.randint(1, 24), s["prompt"] - s["done"])
                start = s["done"]
                s["done"] += n
                need = -(-s["done"] // self.bs)
                s["blocks"] += self._blocks(need - len(s["blocks"]))
                pre.append(M.PrefillItem(sid, [0] * n, start, list(s["blocks"])))
                s["ctx"] = s["done"]
            else:
                s["ctx"] += 1
                need = -(-s["ctx"] // self.bs)
                s["blocks"] += self._blocks(need - len(s["blocks"]))
                dec.append(M.DecodeItem(sid, 0, s["ctx"] - 1, list(s["blocks"]), s["ctx"]))
        step = type("Step", (), {})()
        step.prefills, step.decodes = pre, dec
        return step, finished, preempted


@pytest.mark.parametrize("max_seqs,release", [(64, True), (12, False)])
def test_planner_tracks_a_scheduler_over_many_steps(max_seqs, release):
    sim = Sim(seed=max_seqs, bs=4)
    width = 64
    res = TableResidency(max_seqs, width, block_size=4, num_blocks=sim.pool)
    resident = np.zeros((max_seqs, width), dtype=np.int32)
    uploaded = full = 0
    for _ in range(400):
        step, finished, preempted = sim.step(max_batch=min(max_seqs, 10))
        for sid in finished + preempted:
            if release:
                res.release(sid)
        groups, which = step_groups(step)
        if not groups:
            continue
        plan = res.plan(groups)
        tables = apply_plan(plan, resident)
        refs = [M.prefill_meta(step.prefills) if w == 0 else M.decode_meta(step.decodes) for w in which]
        check_against_oracle(plan, tables, refs)
        for e0, n, off, g in plan.groups:
            for sid, t in zip(g.seq_ids, g.tables):
                np.testing.assert_array_equal(resident[res.row[sid], : len(t)], t)
        uploaded += plan.n_new_ids
        full += sum(len(t) for g in groups for t in g.tables)
    assert uploaded < full / 4  # deltas, not whole tables


def test_steady_decode_uploads_only_appended_blocks():
    bs = 16
    res = TableResidency(8, 32, block_size=bs, num_blocks=1000)
    tables = {i: [10 * i + j for j in range(3)] for i in range(8)}
    ctx = {i: 3 * bs - 8 + i for i in range(8)}

    def group():
        return make_group(list(tables), list(tables.values()), list(ctx.values()),
                          [c - 1 for c in ctx.values()], [1] * 8, True)

    assert res.plan([group()]).n_new_ids == 24
    for step in range(12):
        crossing = 0
        for i in tables:
            ctx[i] += 1
            if (ctx[i] - 1) % bs == 0:
                tables[i].append(500 + 8 * step + i)
                crossing += 1
        plan = res.plan([group()])
        assert plan.n_new_ids == crossing


def test_errors_leave_residency_unchanged():
    res = TableResidency(2, 4, block_size=4, num_blocks=10)
    res.plan([make_group([1], [[1, 2]], [8], [7], [1], True)])
    before = (dict(res.row), [list(m) for m in res.mirror], list(res.free), res.tick)
    with pytest.raises(IndexError, match="context_len 9 needs 3 blocks, have 2"):
        res.plan([make_group([1], [[1, 2]], [9], [8], [1], True)])
    with pytest.raises(IndexError, match="block id 10 is outside the pool of 10 blocks"):
        res.plan([make_group([1, 2], [[1, 2, 3], [10]], [9, 1], [8, 0], [1, 1], True)])
    with pytest.raises(ValueError, match="appears twice"):
        res.plan([make_group([1, 1], [[1, 2], [1, 2]], [8, 8], [7, 7], [1, 1], True)])
    with pytest.raises(ValueError, match="rows hold 4"):
        res.plan([make_group([3], [[1, 2, 3, 4, 5]], [1], [0], [1], True)])
    with pytest.raises(ValueError, match="the tables hold 2"):
        res.plan([make_group([3, 4, 5], [[1], [1], [1]], [1, 1, 1], [0, 0, 0], [1, 1, 1], True)])
    with pytest.raises(ValueError, match="same number of query tokens"):
        res.plan([make_group([3, 4], [[1], [1]], [1, 2], [0, 0], [1, 2], True)])
    assert before == (dict(res.row), [list(m) for m in res.mirror], list(res.free), res.tick)


def test_lru_reuses_the_oldest_row_not_in_the_step():
    res = TableResidency(2, 4)
    res.plan([make_group(["a"], [[1]], [1], [0], [1], True)])
    res.plan([make_group(["b"], [[2]], [1], [0], [1], True)])
    res.plan([make_group(["a"], [[1]], [2], [1], [1], True)])  # "b" is now the oldest
    ra = res.row["a"]
    res.plan([make_group(["c", "a"], [[3], [1]], [1, 3], [0, 2], [1, 1], True)])
    assert "b" not in res.row and res.row["a"] == ra and res.row["c"] != ra
    # "b" comes back: its row is re-uploaded from scratch
    plan = res.plan([make_group(["b"], [[2]], [1], [0], [1], True)])
    assert plan.n_new_ids == 1


# ------------------------------------------ speculative-step derivations


def _host_meta(ref: "M.Meta", headroom=None) -> DeviceAttnMeta:
    """A DeviceAttnMeta built from the oracle's lists on CPU tensors (the
    derivations are tensor arithmetic; the device case is tested on the GPU)."""
    q = [hi - lo for lo, hi in ref.token_slices]
    cu = [0]
    for x in q:
        cu.append(cu[-1] + x)
    i32 = lambda v: torch.tensor(v, dtype=torch.int32)  # noqa: E731
    return DeviceAttnMeta(ref.token_slices, torch.from_numpy(M.padded_tables(ref.block_tables)),
                          i32(ref.context_lens), i32(ref.start_positions), i32(cu), q,
                          max(ref.context_lens), max(q), ref.is_decode, headroom)


def _same(meta: DeviceAttnMeta, ref: "M.Meta"):
    assert meta.token_slices == ref.token_slices
    assert meta.context_lens.tolist() == ref.context_lens
    assert meta.start_positions.tolist() == ref.start_positions
    cu = meta.cu_query_lens.tolist()
    assert [(cu[b], cu[b + 1]) for b in range(len(cu) - 1)] == ref.token_slices
    assert meta.query_lens == [hi - lo for lo, hi in ref.token_slices]
    assert meta.max_context_len == max(ref.context_lens) and meta.max_query_len == max(meta.query_lens)
    assert meta.is_decode


def test_speculative_metadata_derivations_match_the_runner():
    items = [M.DecodeItem(0, 5, 16, [3, 4], 17), M.DecodeItem(1, 6, 40, [7, 8, 9, 10], 41),
             M.DecodeItem(2, 7, 0, [1], 1)]
    base = _host_meta(M.decode_meta(items), headroom=min(len(i.block_ids) * 16 - i.context_len for i in items))
    for j in range(4):
        _same(base.advanced(j), M.draft_meta(items, j))
    for n in (1, 2, 4):
        _same(base.verify(n), M.verify_meta(items, n))
    # hand-checked: verify(3) of the item at position 16 covers positions 16..18
    v = base.verify(3)
    assert v.token_slices[0] == (0, 3) and v.context_lens[0] == 19 and v.start_positions[0] == 16
    # the sequence at context 41 of 64 slots and the one at 1 of 16 leave 15 spare positions
    assert base.headroom == 15
    with pytest.raises(IndexError, match="holds only 15 positions"):
        base.advanced(16)
    with pytest.raises(IndexError):
        base.verify(17)
    with pytest.raises(ValueError):
        base.verify(2).verify(2)


def test_invalidate_forces_whole_tables_next_time():
    """A step whose upload failed leaves its rows unknown: the next plan
    re-sends those tables whole, and other rows keep their deltas."""
    res = TableResidency(4, 8, block_size=16, num_blocks=100)
    res.plan([make_group([1, 2], [[1, 2, 3], [4, 5]], [40, 20], [39, 19], [1, 1], True)])
    plan = res.plan([make_group([1], [[1, 2, 3, 6]], [49], [48], [1], True)])
    assert plan.n_new_ids == 1
    res.invalidate(plan)
    again = res.plan([make_group([1, 2], [[1, 2, 3, 6], [4, 5]], [49, 20], [48, 19], [1, 1], True)])
    assert again.n_new_ids == 4  # sequence 1 whole, sequence 2 unchanged
