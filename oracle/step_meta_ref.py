"""Restatement of helios' per-step attention metadata -- TEST INFRASTRUCTURE.

Only tests/ may import this module; the product never does.  It rebuilds, in
plain Python, what helios' model runner derives from a scheduler step before
the attention calls (reference = anish41338/helios, python/helios/):

  prefill_meta   exec/runner.py:188-225  (chunks concatenated: token slices,
                 tables, context = start + n, start positions)
  decode_meta    exec/runner.py:250-268  (one token per sequence: context_len
                 and position from the DecodeItem)
  padded_tables  exec/triton_attn.py:156-165 (int32 [n, max len], zero-padded)
  draft_meta     exec/runner.py:330-346 (draft step j: position and context + j)
  verify_meta    exec/runner.py:352-362 (n tokens from the decode position,
                 context_len + n - 1)

Pinned by tests/test_step_meta.py: hand-built steps whose expected metadata
is written out literally, and the invariants the runner relies on (slices
tile the token axis in order, context = start + chunk length).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Sequence, Tuple

import numpy as np


@dataclass
class PrefillItem:
    """The fields of core/execstep.py:24-39 the metadata reads."""

    seq_id: int
    token_ids: List[int]
    start_pos: int
    block_ids: List[int] = field(default_factory=list)

    @property
    def num_tokens(self) -> int:
        return len(self.token_ids)


@dataclass
class DecodeItem:
    """The fields of core/execstep.py:42-51 the metadata reads."""

    seq_id: int
    last_token_id: int
    position: int
    block_ids: List[int] = field(default_factory=list)
    context_len: int = 0


@dataclass
class Meta:
    """BatchedAttnMeta (exec/model.py:254-277)."""

    token_slices: List[Tuple[int, int]]
    block_tables: List[List[int]]
    context_lens: List[int]
    start_positions: List[int]
    is_decode: bool


def prefill_meta(items: Sequence[PrefillItem]) -> Meta:
    """exec/runner.py:203-225."""
    slices, tables, ctx, starts = [], [], [], []
    n = 0
    for it in items:
        lo = n
        n += it.num_tokens
        slices.append((lo, n))
        tables.append(list(it.block_ids))
        ctx.append(it.start_pos + it.num_tokens)
        starts.append(it.start_pos)
    return Meta(slices, tables, ctx, starts, False)


def decode_meta(items: Sequence[DecodeItem]) -> Meta:
    """exec/runner.py:261-268."""
    return Meta(
        [(i, i + 1) for i in range(len(items))],
        [list(it.block_ids) for it in items],
        [it.context_len for it in items],
        [it.position for it in items],
        True,
    )


def padded_tables(tables: Sequence[Sequence[int]]) -> np.ndarray:
    """exec/triton_attn.py:156-165: int32 [n, max(len)], zero-padded (width 1
    for an empty batch, 0 when every table of a batch is empty)."""
    width = max((len(t) for t in tables), default=1)
    out = np.zeros((len(tables), width), dtype=np.int32)
    for i, t in enumerate(tables):
        out[i, : len(t)] = t
    return out


def draft_meta(items: Sequence[DecodeItem], j: int) -> Meta:
    """exec/runner.py:330-346: the draft's j-th forward after the decode
    item, one token at position + j attending context_len + j keys."""
    return decode_meta([DecodeItem(it.seq_id, 0, it.position + j, it.block_ids, it.context_len + j)
                        for it in items])


def verify_meta(items: Sequence[DecodeItem], n: int) -> Meta:
    """exec/runner.py:352-362: verify tokens [last] + drafted[:-1] (n of
    them) at positions position .. position + n - 1, context_len + n - 1."""
    return Meta(
        [(i * n, (i + 1) * n) for i in range(len(items))],
        [list(it.block_ids) for it in items],
        [it.context_len + n - 1 for it in items],
        [it.position for it in items],
        True,
    )
