"""Attention metadata that stays in HBM across scheduler steps.

helios' runner builds a ``BatchedAttnMeta`` of Python lists for every step
(reference exec/runner.py:188-225, 250-268; exec/model.py:254-277), and each
attention call of each layer converts those lists into device tensors again
(exec/triton_attn.py:156-165, paged_attn.py:106, 347-348), a synchronising
host-to-device copy per layer, plus the per-layer ``positions[0].item()``
of exec/model.py:205.

``DeviceBlockTables`` keeps one int32 row per resident sequence in device
memory.  Between steps a sequence's table changes only at its tail (a block
appended every ``block_size`` tokens, a copy-on-write replacement, a
re-admission after preemption), so ``prepare`` finds the first entry that
differs from what the device already holds and uploads only that suffix.
One pinned buffer carries every sequence's changed suffix, context length,
start position and query-length prefix sums in a single asynchronous copy,
and one ``hpa_step_tables`` launch writes the suffixes into the resident
rows and gathers the step's tables in batch order.  The returned
``DeviceAttnMeta`` holds only device tensors and host integers, so
``write_kv_batched`` and ``batched_attention`` launch for every layer with no
host work and no synchronisation.

A ``DeviceAttnMeta`` stays valid until the second ``prepare`` call after the
one that made it (its buffers alternate between two slots); kernels that
read it must be enqueued on the stream that was current at ``prepare``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Hashable, List, Optional, Sequence, Tuple

import numpy as np
import torch

from ._lib import check, lib, ptr, stream_ptr
from .paged_attn import PagedKVCache, paged_attention_decode_hip, paged_attention_varlen, write_kv

_ENTRY = 5  # (row, n_blocks, upd_first, upd_count, upd_offset), as hpa_step_tables reads it


@dataclass
class DeviceAttnMeta:
    """``BatchedAttnMeta`` (exec/model.py:254-277) with device tensors.

    block_tables     int32 [n, width], zero-padded past each table's end
    context_lens     int32 [n]
    start_positions  int32 [n]
    cu_query_lens    int32 [n + 1], prefix sums of query_lens
    """

    token_slices: List[Tuple[int, int]]
    block_tables: torch.Tensor
    context_lens: torch.Tensor
    start_positions: torch.Tensor
    cu_query_lens: torch.Tensor
    query_lens: List[int]
    max_context_len: int
    max_query_len: int
    is_decode: bool
    # positions every table can still hold past its context (None: unknown)
    headroom: Optional[int] = None

    @property
    def n_seqs(self) -> int:
        return len(self.query_lens)

    @property
    def n_tokens(self) -> int:
        return self.token_slices[-1][1] if self.token_slices else 0

    def _need(self, extra: int) -> None:
        if extra < 0:
            raise ValueError("a speculative step cannot go backwards")
        if self.headroom is not None and extra > self.headroom:
            raise IndexError(f"a block table holds only {self.headroom} positions past its context; "
                             f"{extra} needed")

    def advanced(self, j: int) -> "DeviceAttnMeta":
        """The same one-token decode batch j tokens later -- draft step j of
        speculative decoding (exec/runner.py:330-346, exec/qassd.py:291-305):
        every context length and position + j.  Device arithmetic only, no
        upload and no synchronisation."""
        if not self.is_decode or self.max_query_len != 1:
            raise ValueError("advanced() applies to a one-token decode batch")
        self._need(j)
        return DeviceAttnMeta(
            self.token_slices, self.block_tables, self.context_lens + j, self.start_positions + j,
            self.cu_query_lens, self.query_lens, self.max_context_len + j, 1, True,
            None if self.headroom is None else self.headroom - j)

    def verify(self, n: int) -> "DeviceAttnMeta":
        """n query tokens per sequence from each decode position: the verify
        pass over [last token] + drafted[:-1] at positions position ..
        position + n - 1, attending context_len + n - 1 keys
        (exec/runner.py:352-362, exec/qassd.py:309-314).  The same metadata
        serves the re-sync of the draft's KV shadow (runner.py:397-406)
        when it is run over all n positions: K/V written past a sequence's
        committed tokens lie beyond every later draft step's context until
        that step rewrites them.  Device arithmetic only."""
        if not self.is_decode or self.max_query_len != 1:
            raise ValueError("verify() applies to a one-token decode batch")
        if n < 1:
            raise ValueError("verify needs at least one token per sequence")
        self._need(n - 1)
        b = self.n_seqs
        cu = torch.arange(0, (b + 1) * n, n, dtype=torch.int32, device=self.context_lens.device)
        return DeviceAttnMeta(
            [(i * n, (i + 1) * n) for i in range(b)], self.block_tables, self.context_lens + (n - 1),
            self.start_positions, cu, [n] * b, self.max_context_len + n - 1, n, True,
            None if self.headroom is None else self.headroom - (n - 1))


@dataclass
class _Group:
    seq_ids: List[Hashable]
    tables: List[List[int]]
    context_lens: List[int]
    start_positions: List[int]
    query_lens: List[int]
    is_decode: bool


@dataclass
class StepPlan:
    """One step's upload, packed as hpa_step_tables and the metadata read it:
    [entries 5 N | per group: context_lens n, start_positions n,
    cu_query_lens n + 1 | new ids]."""

    packed: np.ndarray                  # int32
    n_entries: int
    new_ids_offset: int
    n_new_ids: int
    width: int                          # step table width (>= 1)
    groups: List[Tuple[int, int, int, _Group]]   # (first entry, n, packed offset, group)


class TableResidency:
    """Host half of ``DeviceBlockTables``: which row holds which sequence,
    what each row holds on the device, and the packed delta of a step.  No
    GPU is touched here."""

    def __init__(self, max_seqs: int, width: int, block_size: Optional[int] = None,
                 num_blocks: Optional[int] = None):
        if max_seqs <= 0 or width <= 0 or max_seqs > 65535:
            raise ValueError("max_seqs must be in [1, 65535] and max_blocks_per_seq positive")
        self.max_seqs, self.width = int(max_seqs), int(width)
        self.block_size, self.num_blocks = block_size, num_blocks
        self.row: Dict[Hashable, int] = {}
        self.seq_of_row: List[Optional[Hashable]] = [None] * self.max_seqs
        self.mirror: List[List[int]] = [[] for _ in range(self.max_seqs)]
        self.last_use = [0] * self.max_seqs
        self.free = list(range(self.max_seqs - 1, -1, -1))
        self.tick = 0

    def release(self, seq_id: Hashable) -> None:
        row = self.row.pop(seq_id, None)
        if row is not None:
            self.seq_of_row[row] = None
            self.mirror[row] = []
            self.free.append(row)

    def invalidate(self, plan: "StepPlan") -> None:
        """Forget what the rows of a planned step hold (their upload did not
        happen): their next plan uploads whole tables."""
        for _, _, _, g in plan.groups:
            for sid in g.seq_ids:
                row = self.row.get(sid)
                if row is not None:
                    self.mirror[row] = []

    def check(self, groups: List[_Group]) -> None:
        ids = [sid for g in groups for sid in g.seq_ids]
        if len(ids) > self.max_seqs:
            raise ValueError(f"{len(ids)} sequences in one step; the tables hold {self.max_seqs}")
        if len(set(ids)) != len(ids):
            dup = next(x for i, x in enumerate(ids) if x in ids[:i])
            raise ValueError(f"sequence {dup!r} appears twice in one step")
        for g in groups:
            n = len(g.seq_ids)
            if not (len(g.tables) == len(g.context_lens) == len(g.start_positions) == len(g.query_lens) == n):
                raise ValueError("seq_ids, block_tables, context_lens, start_positions and query_lens differ in length")
            if not n:
                continue
            if g.is_decode and len(set(g.query_lens)) != 1:
                raise ValueError("a decode batch needs the same number of query tokens for every sequence")
            if min(g.query_lens) < 0 or min(g.start_positions) < 0 or min(g.context_lens) < 0:
                raise ValueError("negative length or position")
            nbl = [len(t) for t in g.tables]
            if max(nbl) > self.width:
                b = max(range(n), key=nbl.__getitem__)
                raise ValueError(f"sequence {g.seq_ids[b]!r} has {nbl[b]} blocks; rows hold {self.width}")
            if self.block_size:
                bs = self.block_size
                for c, m in zip(g.context_lens, nbl):
                    if (c + bs - 1) // bs > m:
                        raise IndexError(f"context_len {c} needs {(c + bs - 1) // bs} blocks, have {m}")

    def first_change(self, sid: Hashable, table: List[int]) -> int:
        """First index where ``table`` differs from the device's copy."""
        row = self.row.get(sid)
        old = self.mirror[row] if row is not None else []
        lo = len(old)
        if len(table) >= lo and table[:lo] == old:
            return lo
        m = min(lo, len(table))
        i = 0
        while i < m and table[i] == old[i]:
            i += 1
        return i

    def _take_row(self, sid: Hashable, keep: set) -> int:
        row = self.row.get(sid)
        if row is not None:
            return row
        if self.free:
            row = self.free.pop()
        else:
            row = min((r for r in range(self.max_seqs) if self.seq_of_row[r] not in keep),
                      key=lambda r: self.last_use[r])
            del self.row[self.seq_of_row[row]]
        self.row[sid] = row
        self.seq_of_row[row] = sid
        self.mirror[row] = []
        return row

    def plan(self, groups: List[_Group]) -> StepPlan:
        """Validate, then commit residency and pack the step's delta.
        Nothing changes when validation raises."""
        self.check(groups)
        row_of, mirror, nbk = self.row, self.mirror, self.num_blocks
        firsts: List[List[int]] = []
        n_new = 0
        for g in groups:
            f = []
            for sid, t in zip(g.seq_ids, g.tables):
                r = row_of.get(sid)
                old = mirror[r] if r is not None else []
                lo = len(old)
                nt = len(t)
                if (t == old) if nt == lo else (nt > lo and t[:lo] == old):
                    i = lo
                else:
                    i = self.first_change(sid, t)
                f.append(i)
                if i < len(t):
                    n_new += len(t) - i
                    if nbk is not None:
                        for b in t[i:]:
                            if not 0 <= b < nbk:
                                raise IndexError(f"block id {b} is outside the pool of {nbk} blocks")
            firsts.append(f)
        n_all = sum(len(g.seq_ids) for g in groups)
        width = max([len(t) for g in groups for t in g.tables] + [1])

        self.tick += 1
        tick = self.tick
        keep = {sid for g in groups for sid in g.seq_ids}
        ent: List[Tuple[int, int, int, int, int]] = []
        new_ids: List[int] = []
        for g, f in zip(groups, firsts):
            for sid, t, i in zip(g.seq_ids, g.tables, f):
                row = row_of.get(sid)
                if row is None:
                    row = self._take_row(sid, keep)
                self.last_use[row] = tick
                nt = len(t)
                ent.append((row, nt, i, nt - i, len(new_ids)))
                if i < nt:
                    suffix = t[i:]
                    new_ids.extend(suffix)
                    m = mirror[row]
                    if i == len(m):
                        m.extend(suffix)
                    else:
                        mirror[row] = list(t)
                elif nt != len(mirror[row]):
                    mirror[row] = list(t)
        packed = np.empty(_ENTRY * n_all + sum(3 * len(g.seq_ids) + 1 for g in groups) + n_new, dtype=np.int32)
        if n_all:
            packed[: _ENTRY * n_all] = np.asarray(ent, dtype=np.int32).reshape(-1)
        off = _ENTRY * n_all
        layout = []
        e0 = 0
        for g in groups:
            n = len(g.seq_ids)
            packed[off: off + n] = g.context_lens
            packed[off + n: off + 2 * n] = g.start_positions
            packed[off + 2 * n] = 0
            packed[off + 2 * n + 1: off + 3 * n + 1] = np.cumsum(np.asarray(g.query_lens, dtype=np.int64))
            layout.append((e0, n, off, g))
            off += 3 * n + 1
            e0 += n
        packed[off:] = new_ids
        return StepPlan(packed, n_all, off, n_new, width, layout)


class DeviceBlockTables:
    """Resident block tables for up to ``max_seqs`` sequences of up to
    ``max_blocks_per_seq`` blocks each.

    With ``block_size`` / ``num_blocks`` given (``for_cache`` takes them from
    a cache), ``prepare`` raises helios' ``IndexError`` for a table too short
    for its context (paged_attn.py:100-104) and for block ids outside the
    pool, before anything is uploaded.  Sequences leave with ``release``;
    when every row is taken, the least recently used row of a sequence not in
    the current call is reused.
    """

    def __init__(self, max_seqs: int, max_blocks_per_seq: int, device=None,
                 block_size: Optional[int] = None, num_blocks: Optional[int] = None):
        self.host = TableResidency(max_seqs, max_blocks_per_seq, block_size, num_blocks)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if dev.type != "cuda":
            raise RuntimeError(f"DeviceBlockTables lives on the GPU, got {dev}")
        if dev.index is None:
            dev = torch.device("cuda", torch.cuda.current_device())
        self.device = dev
        self.max_seqs, self.width = self.host.max_seqs, self.host.width
        self.resident = torch.zeros(self.max_seqs, self.width, dtype=torch.int32, device=dev)
        self._step_tables = [torch.zeros(self.max_seqs * self.width, dtype=torch.int32, device=dev)
                             for _ in range(2)]
        self._pinned: List[Optional[torch.Tensor]] = [None, None]
        self._dev: List[Optional[torch.Tensor]] = [None, None]
        self._copied: List[Optional[torch.cuda.Event]] = [None, None]
        self._slot = 0

    @classmethod
    def for_cache(cls, kv_cache: PagedKVCache, max_seqs: int, max_blocks_per_seq: int) -> "DeviceBlockTables":
        return cls(max_seqs, max_blocks_per_seq, kv_cache.k_cache.device,
                   kv_cache.block_size, kv_cache.num_blocks)

    def release(self, seq_id: Hashable) -> None:
        """Forget a finished or preempted sequence; its row is reused."""
        self.host.release(seq_id)

    def __contains__(self, seq_id: Hashable) -> bool:
        return seq_id in self.host.row

    def __len__(self) -> int:
        return len(self.host.row)

    def prepare(self, seq_ids: Sequence[Hashable], block_tables: Sequence[Sequence[int]],
                context_lens: Sequence[int], start_positions: Sequence[int],
                query_lens: Sequence[int], is_decode: bool = False) -> DeviceAttnMeta:
        """Device metadata for one batch: sequence b owns tokens
        [sum(query_lens[:b]), +query_lens[b]) of the flattened batch, sits at
        start_positions[b] and attends context_lens[b] keys.  A decode batch
        (is_decode) has the same number of query tokens, q_per_seq, for every
        sequence (1 for decode, gamma + 1 for speculative verify)."""
        return self._prepare([make_group(seq_ids, block_tables, context_lens, start_positions,
                                         query_lens, is_decode)])[0]

    def prepare_step(self, step) -> Tuple[Optional[DeviceAttnMeta], Optional[DeviceAttnMeta]]:
        """(prefill meta, decode meta) of a scheduler ``ExecStep``
        (core/execstep.py:58-100), as the runner derives them
        (exec/runner.py:203-225 for prefill chunks, :261-268 for decodes),
        in one upload and one launch.  None for an empty phase."""
        groups, which = step_groups(step)
        out: List[Optional[DeviceAttnMeta]] = [None, None]
        if groups:
            for w, m in zip(which, self._prepare(groups)):
                out[w] = m
        return out[0], out[1]

    def _buffers(self, slot: int, n_ints: int) -> Tuple[torch.Tensor, torch.Tensor]:
        pinned, dev = self._pinned[slot], self._dev[slot]
        if pinned is None or pinned.numel() < n_ints:
            cap = max(n_ints, 8 * self.max_seqs + 4096)
            cap = 1 << (cap - 1).bit_length()
            pinned = torch.empty(cap, dtype=torch.int32, pin_memory=True)
            dev = torch.empty(cap, dtype=torch.int32, device=self.device)
            self._pinned[slot], self._dev[slot] = pinned, dev
        return pinned, dev

    def _prepare(self, groups: List[_Group]) -> List[DeviceAttnMeta]:
        plan = self.host.plan(groups)
        try:
            return self._upload(plan)
        except BaseException:
            self.host.invalidate(plan)
            raise

    def _upload(self, plan: StepPlan) -> List[DeviceAttnMeta]:
        slot = self._slot
        self._slot ^= 1
        if self._copied[slot] is not None:
            self._copied[slot].synchronize()  # the pinned buffer's previous copy has left
        n_ints = plan.packed.size
        pinned, dev = self._buffers(slot, n_ints)
        pinned.numpy()[:n_ints] = plan.packed
        stream = torch.cuda.current_stream(self.device)
        dev[:n_ints].copy_(pinned[:n_ints], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        self._copied[slot] = ev

        tables = self._step_tables[slot]
        width = plan.width
        base = ptr(dev)
        check(lib().hpa_step_tables(base, plan.n_entries, base + 4 * plan.new_ids_offset if plan.n_new_ids else None,
                                    plan.n_new_ids, ptr(self.resident), self.max_seqs, self.width, ptr(tables),
                                    width, stream_ptr(self.device)), "hpa_step_tables")
        metas = []
        for e0, n, o, g in plan.groups:
            cu = plan.packed[o + 2 * n: o + 3 * n + 1]
            metas.append(DeviceAttnMeta(
                token_slices=[(int(cu[b]), int(cu[b + 1])) for b in range(n)],
                block_tables=tables[e0 * width: (e0 + n) * width].view(n, width),
                context_lens=dev[o: o + n],
                start_positions=dev[o + n: o + 2 * n],
                cu_query_lens=dev[o + 2 * n: o + 3 * n + 1],
                query_lens=list(g.query_lens),
                max_context_len=max(g.context_lens, default=0),
                max_query_len=max(g.query_lens, default=0),
                is_decode=g.is_decode,
                headroom=(min((len(t) * self.host.block_size - c for t, c in zip(g.tables, g.context_lens)),
                              default=0) if self.host.block_size else None),
            ))
        return metas


def make_group(seq_ids, block_tables, context_lens, start_positions, query_lens, is_decode) -> _Group:
    """The tables are referenced, not copied: they are read during the
    ``plan`` call only, and what the device holds is copied from them."""
    return _Group(list(seq_ids), [t if isinstance(t, list) else list(t) for t in block_tables],
                  [int(c) for c in context_lens], [int(s) for s in start_positions],
                  [int(q) for q in query_lens], bool(is_decode))


def step_groups(step) -> Tuple[List[_Group], List[int]]:
    """The prefill and decode groups of an ExecStep, with their slot (0
    prefill, 1 decode): exec/runner.py:203-225 and :261-268."""
    groups, which = [], []
    pre, dec = list(getattr(step, "prefills", []) or []), list(getattr(step, "decodes", []) or [])
    if pre:
        groups.append(make_group([p.seq_id for p in pre], [p.block_ids for p in pre],
                                 [p.start_pos + p.num_tokens for p in pre], [p.start_pos for p in pre],
                                 [p.num_tokens for p in pre], False))
        which.append(0)
    if dec:
        groups.append(make_group([d.seq_id for d in dec], [d.block_ids for d in dec],
                                 [d.context_len for d in dec], [d.position for d in dec],
                                 [1] * len(dec), True))
        which.append(1)
    return groups, which


# ------------------------------------------------------------ consumers


def write_kv_batched(kv_cache: PagedKVCache, meta: DeviceAttnMeta, k: torch.Tensor, v: torch.Tensor,
                     rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> None:
    """Every sequence's K/V of the step into the cache, one launch, no host
    synchronisation (the per-sequence write loop of exec/model.py:244-247,
    optionally with apply_rope of K fused, :200-201)."""
    if k.shape[0] != meta.n_tokens:
        raise ValueError(f"k has {k.shape[0]} rows, the batch has {meta.n_tokens} tokens")
    if meta.n_seqs == 0:
        return
    write_kv(kv_cache, meta.block_tables, meta.start_positions, k, v,
             cu_query_lens=meta.cu_query_lens, max_query_len=meta.max_query_len, rope=rope)


def batched_attention(query: torch.Tensor, kv_cache: PagedKVCache, meta: DeviceAttnMeta,
                      scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                      workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``BatchedAttention.run`` (exec/model.py:287-318) on device metadata:
    a decode batch goes to the decode kernel (q_per_seq query tokens per
    sequence, the speculative verify form when above 1), anything else to the
    ragged causal prefill, each one launch.  ``out`` and a caller-owned
    decode ``workspace`` (``decode_workspace``) make the call allocate
    nothing, as code under HIP graph capture needs."""
    if query.shape[0] != meta.n_tokens:
        raise ValueError(f"query has {query.shape[0]} rows, the batch has {meta.n_tokens} tokens")
    if meta.is_decode:
        ks, vs = kv_cache._scales()
        return paged_attention_decode_hip(
            query, kv_cache.k_cache, kv_cache.v_cache, meta.block_tables, meta.context_lens, scale,
            ks, vs, q_per_seq=max(meta.max_query_len, 1), max_context_len=meta.max_context_len,
            out=out, workspace=workspace)
    return paged_attention_varlen(
        query, kv_cache, meta.block_tables, None, meta.start_positions, meta.context_lens, scale,
        max_query_len=meta.max_query_len, cu_query_lens=meta.cu_query_lens, out=out)
