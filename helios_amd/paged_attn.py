"""helios' paged-attention API, executed by hand-written gfx950 kernels.

Drop-in for ``helios.exec.paged_attn`` (reference python/helios/exec/
paged_attn.py): same classes, same functions, same argument meaning and the
same IndexError messages, so helios' scheduler, copy-on-write allocator,
prefix cache and speculative verifier run unchanged on top of it.  Every
data-moving call goes through ``libheliosattn.so`` (include/helios_attn.h);
nothing falls back to PyTorch math, and a missing library or GPU raises
RuntimeError.

Beyond helios' surface this module adds the batched forms the engine's
callers need (one launch per step instead of one per sequence):
``paged_attention_varlen`` (chunked prefill of many sequences),
``paged_attention_verify_batched`` (speculative verify, gamma+1 tokens per
sequence), ``copy_blocks`` (every layer's CoW copies in one launch) and the
raw-tensor ``paged_attention_decode_hip`` (the form of helios'
``paged_attention_decode_triton``, triton_attn.py:133-140, plus INT8 scales).
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple, Union

import torch

from . import _lib
from ._lib import DTYPE_CODE, check, lib, ptr, stream_ptr

TableArg = Union[Sequence[Sequence[int]], torch.Tensor]
LensArg = Union[Sequence[int], torch.Tensor]


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"{what} is on {t.device}; helios_amd kernels run on the GPU only "
            "(there is no CPU path)"
        )


def _i32(values, device) -> torch.Tensor:
    return torch.tensor(values, dtype=torch.int32, device=device)


def _meta(t: torch.Tensor, name: str, device: torch.device, dim: int) -> torch.Tensor:
    """A metadata tensor handed to a kernel as-is: it must be an int32,
    contiguous, ``dim``-dimensional tensor on the kernels' device (an int64
    tensor would be read as pairs of int32 words)."""
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32, got {t.dtype}")
    if t.dim() != dim:
        raise ValueError(f"{name} must be {dim}-dimensional, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device != torch.device(device):
        raise ValueError(f"{name} is on {t.device}, the kernels run on {device}")
    return t


def _out_for(query: torch.Tensor, out: Optional[torch.Tensor]) -> torch.Tensor:
    """A row-major output of query's shape and dtype: the kernels write
    [tokens, heads, head_dim] densely, whatever strides query came with."""
    if out is None:
        return torch.empty(query.shape, dtype=query.dtype, device=query.device)
    if out.shape != query.shape or out.dtype != query.dtype or out.device != query.device:
        raise ValueError(f"out must be {query.dtype} {tuple(query.shape)} on {query.device}")
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")
    return out


def _check_context(block_ids: Sequence[int], context_len: int, block_size: int,
                   num_blocks: int) -> None:
    """helios' gather preconditions (paged_attn.py:100-104) plus pool bounds."""
    n_blocks = (context_len + block_size - 1) // block_size
    if n_blocks > len(block_ids):
        raise IndexError(
            f"context_len {context_len} needs {n_blocks} blocks, have {len(block_ids)}"
        )
    for b in block_ids[:n_blocks]:
        if not 0 <= int(b) < num_blocks:
            raise IndexError(f"block id {b} is outside the pool of {num_blocks} blocks")


def _padded_tables(tables: Sequence[Sequence[int]], device) -> torch.Tensor:
    """int32 [n, max_blocks] zero-padded table (triton_attn.py:156-165)."""
    width = max((len(t) for t in tables), default=1) or 1
    rows = [list(map(int, t)) + [0] * (width - len(t)) for t in tables]
    return torch.tensor(rows, dtype=torch.int32, device=device).reshape(len(tables), width)


class PagedKVCache:
    """Physical KV storage, [num_blocks, n_kv_heads, block_size, head_dim]
    (paged_attn.py:25-55).  One per layer; the allocator owns the mapping."""

    def __init__(
        self,
        num_blocks: int,
        block_size: int,
        n_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype = torch.float32,
        device: str = "cpu",
    ) -> None:
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device

        shape = (num_blocks, n_kv_heads, block_size, head_dim)
        self.k_cache = torch.zeros(shape, dtype=dtype, device=device)
        self.v_cache = torch.zeros(shape, dtype=dtype, device=device)

    # storage helpers shared with the quantized subclass
    @property
    def pool_dtype(self) -> torch.dtype:
        return self.k_cache.dtype

    def _scales(self) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        return None, None

    @property
    def nbytes(self) -> int:
        return self.k_cache.numel() * self.k_cache.element_size() * 2

    def write(self, block_ids: List[int], start_pos: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Scatter k/v [n_tokens, n_kv_heads, head_dim] to positions
        start_pos.. (paged_attn.py:57-85).  Like helios, positions before the
        first one without a block are written, then IndexError is raised."""
        n_tokens = k.shape[0]
        if n_tokens == 0:
            return
        bs = self.block_size
        n_ok = n_tokens
        for i in range(n_tokens):
            if (start_pos + i) // bs >= len(block_ids):
                n_ok = i
                break
        needed = (start_pos + n_ok - 1) // bs + 1 if n_ok else 0
        for b in block_ids[:needed]:
            if not 0 <= int(b) < self.num_blocks:
                raise IndexError(f"block id {b} is outside the pool of {self.num_blocks} blocks")
        if n_ok:
            _require_gpu(self.k_cache, "the KV cache")
            write_kv(self, [list(block_ids)], [start_pos], k[:n_ok], v[:n_ok])
        if n_ok < n_tokens:
            pos = start_pos + n_ok
            raise IndexError(
                f"position {pos} needs logical block {pos // bs} but the "
                f"sequence has only {len(block_ids)} blocks"
            )

    def gather(self, block_ids: List[int], context_len: int) -> tuple:
        """Contiguous [context_len, n_kv_heads, head_dim] K and V
        (paged_attn.py:87-110, dequantised for int8: :213-235)."""
        if context_len == 0:
            empty = torch.zeros(
                (0, self.n_kv_heads, self.head_dim), dtype=self.dtype, device=self.device
            )
            return empty, empty
        _check_context(block_ids, context_len, self.block_size, self.num_blocks)
        _require_gpu(self.k_cache, "the KV cache")
        dev = self.k_cache.device
        n_blocks = (context_len + self.block_size - 1) // self.block_size
        table = _i32(list(block_ids[:n_blocks]), dev)
        ko = torch.empty((context_len, self.n_kv_heads, self.head_dim), dtype=self.dtype, device=dev)
        vo = torch.empty_like(ko)
        ks, vs = self._scales()
        st = lib().hpa_kv_gather(
            ptr(self.k_cache), ptr(self.v_cache), DTYPE_CODE[self.pool_dtype], ptr(ks), ptr(vs),
            DTYPE_CODE[ks.dtype] if ks is not None else 0, ptr(table), context_len, ptr(ko),
            ptr(vo), DTYPE_CODE[self.dtype], self.n_kv_heads, self.head_dim, self.block_size,
            self.num_blocks, stream_ptr(dev),
        )
        check(st, "hpa_kv_gather")
        return ko, vo

    def copy_block(self, src: int, dst: int) -> None:
        """Physical block copy for copy-on-write and swap (paged_attn.py:112-115);
        the int8 cache copies its scales too (:237-245)."""
        copy_blocks([self], [(src, dst)])


class QuantizedPagedKVCache(PagedKVCache):
    """INT8 paged KV storage with per-(block, head, token) symmetric scales
    (paged_attn.py:118-245).  ``dtype`` is the compute dtype gather and
    attention return; storage is int8 plus ``scale_dtype`` scales (fp16, as
    helios stores them, by default; fp32 optionally)."""

    def __init__(
        self,
        num_blocks: int,
        block_size: int,
        n_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype = torch.float32,
        device: str = "cpu",
        scale_dtype: torch.dtype = torch.float16,
    ) -> None:
        # Like helios, the fp tensors of the base class are never allocated.
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        if scale_dtype not in (torch.float16, torch.float32):
            raise ValueError(f"scale_dtype must be float16 or float32, got {scale_dtype}")

        shape = (num_blocks, n_kv_heads, block_size, head_dim)
        self.k_cache = torch.zeros(shape, dtype=torch.int8, device=device)
        self.v_cache = torch.zeros(shape, dtype=torch.int8, device=device)
        sshape = (num_blocks, n_kv_heads, block_size)
        self.k_scale = torch.ones(sshape, dtype=scale_dtype, device=device)
        self.v_scale = torch.ones(sshape, dtype=scale_dtype, device=device)

    def _scales(self):
        return self.k_scale, self.v_scale

    @property
    def nbytes(self) -> int:
        return 2 * (
            self.k_cache.numel() * self.k_cache.element_size()
            + self.k_scale.numel() * self.k_scale.element_size()
        )


# ---------------------------------------------------------------- data movement


def write_kv(
    kv_cache: PagedKVCache,
    block_tables: TableArg,
    start_positions: LensArg,
    k: torch.Tensor,
    v: torch.Tensor,
    query_lens: Optional[LensArg] = None,
    cu_query_lens: Optional[torch.Tensor] = None,
    max_query_len: Optional[int] = None,
    rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
) -> None:
    """Scatter (fp) or quantize-and-scatter (int8) K/V of a ragged batch in
    one launch.  With rope=(cos, sin) -- fp32 [max_positions, head_dim / 2]
    device tables, as helios' build_rope_cache makes them (model.py:117-132)
    -- K is rotated rotate-half style by each token's position on the way in
    (apply_rope, model.py:135-153, fused into the write) and V is written as
    is; positions without a table row are skipped like positions without a
    block.  k, v: [sum(query_lens), n_kv_heads, head_dim]; sequence b's
    tokens go to positions start_positions[b].. through block_tables[b].
    With one sequence and no query_lens, every token belongs to it.  A caller
    that keeps int32 device metadata passes cu_query_lens ([n + 1] offsets)
    and max_query_len instead of query_lens, and the call does no host work
    beyond the launch.  Table entries are not bounds-checked here
    (PagedKVCache.write checks them)."""
    _require_gpu(k, "k")
    dev = kv_cache.k_cache.device
    if isinstance(block_tables, torch.Tensor):
        tables = _meta(block_tables, "block_tables", dev, 2)
        n_seqs = tables.shape[0]
    else:
        n_seqs = len(block_tables)
        tables = _padded_tables(block_tables, dev)
    if cu_query_lens is not None:
        if max_query_len is None:
            raise ValueError("max_query_len is required with cu_query_lens")
        _meta(cu_query_lens, "cu_query_lens", dev, 1)
        if cu_query_lens.numel() != n_seqs + 1:
            raise ValueError("cu_query_lens must be int32 [n_seqs + 1]")
        cu_t, max_q = cu_query_lens, int(max_query_len)
    else:
        if query_lens is None:
            if n_seqs != 1:
                raise ValueError("query_lens is required for more than one sequence")
            query_lens = [k.shape[0]]
        qlens = [int(x) for x in (query_lens.tolist() if isinstance(query_lens, torch.Tensor) else query_lens)]
        cu = [0]
        for x in qlens:
            cu.append(cu[-1] + x)
        cu_t, max_q = _i32(cu, dev), (max(qlens) if qlens else 0)
    starts = (_meta(start_positions, "start_positions", dev, 1) if isinstance(start_positions, torch.Tensor)
              else _i32(list(start_positions), dev))
    if starts.numel() != n_seqs:
        raise ValueError(f"start_positions has {starts.numel()} entries for {n_seqs} sequences")
    k = k.contiguous()
    v = v.contiguous()
    ks, vs = kv_cache._scales()
    args = (
        ptr(k), ptr(v), DTYPE_CODE[k.dtype], ptr(kv_cache.k_cache), ptr(kv_cache.v_cache),
        DTYPE_CODE[kv_cache.pool_dtype], ptr(ks), ptr(vs),
        DTYPE_CODE[ks.dtype] if ks is not None else 0, ptr(tables), tables.shape[1],
        ptr(cu_t), ptr(starts), n_seqs, max_q,
        kv_cache.n_kv_heads, kv_cache.head_dim, kv_cache.block_size, kv_cache.num_blocks,
    )
    if rope is None:
        check(lib().hpa_kv_write(*args, stream_ptr(dev)), "hpa_kv_write")
        return
    cos, sin = rope
    half = kv_cache.head_dim // 2
    for t, name in ((cos, "cos"), (sin, "sin")):
        _require_gpu(t, f"the rope {name} table")
        if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != half or not t.is_contiguous():
            raise ValueError(f"rope {name} must be a contiguous float32 [rows, {half}] tensor")
    if cos.shape != sin.shape:
        raise ValueError("rope cos and sin tables differ in shape")
    check(lib().hpa_kv_write_rope(*args, ptr(cos), ptr(sin), cos.shape[0], stream_ptr(dev)),
          "hpa_kv_write_rope")


def copy_blocks(caches: Sequence[PagedKVCache], pairs: Sequence[Tuple[int, int]]) -> None:
    """All copy-on-write / swap copies of a step, every layer, one launch
    (the runner's loop, reference exec/runner.py:155-165).  Pairs are applied
    as if in order; chains (a destination reused as a source) are split into
    successive launches so the result matches sequential copies."""
    if not pairs or not caches:
        return
    c0 = caches[0]
    for c in caches:
        _require_gpu(c.k_cache, "the KV cache")
        if (c.num_blocks, c.block_size, c.n_kv_heads, c.head_dim, c.pool_dtype) != (
            c0.num_blocks, c0.block_size, c0.n_kv_heads, c0.head_dim, c0.pool_dtype
        ):
            raise ValueError("copy_blocks needs caches of one shape and dtype")
    for s, d in pairs:
        for b in (s, d):
            if not 0 <= int(b) < c0.num_blocks:
                raise IndexError(f"block id {b} is outside the pool of {c0.num_blocks} blocks")
    # split into waves with no dst reused as src / dst within a wave
    waves: List[List[Tuple[int, int]]] = [[]]
    touched_dst: set = set()
    srcs: set = set()
    for s, d in pairs:
        s, d = int(s), int(d)
        if s == d:
            continue
        if d in touched_dst or d in srcs or s in touched_dst:
            waves.append([])
            touched_dst, srcs = set(), set()
        waves[-1].append((s, d))
        touched_dst.add(d)
        srcs.add(s)
    dev = c0.k_cache.device
    scaled = isinstance(c0, QuantizedPagedKVCache)
    kp = torch.tensor([c.k_cache.data_ptr() for c in caches], dtype=torch.int64, device=dev)
    vp = torch.tensor([c.v_cache.data_ptr() for c in caches], dtype=torch.int64, device=dev)
    ksp = vsp = None
    sbytes = 0
    if scaled:
        ksp = torch.tensor([c.k_scale.data_ptr() for c in caches], dtype=torch.int64, device=dev)
        vsp = torch.tensor([c.v_scale.data_ptr() for c in caches], dtype=torch.int64, device=dev)
        sbytes = c0.k_scale[0].numel() * c0.k_scale.element_size()
    bbytes = c0.k_cache[0].numel() * c0.k_cache.element_size()
    for wave in waves:
        if not wave:
            continue
        pr = _i32([x for p in wave for x in p], dev)
        st = lib().hpa_copy_blocks(
            ptr(kp), ptr(vp), ptr(ksp), ptr(vsp), len(caches), ptr(pr), len(wave),
            c0.num_blocks, bbytes, sbytes, stream_ptr(dev),
        )
        check(st, "hpa_copy_blocks")


# ------------------------------------------------------------------- attention


def _repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """GQA head expansion [n, n_kv, hd] -> [n, n_kv * n_rep, hd]
    (paged_attn.py:248-261).  A view helper kept for API parity; the kernels
    never materialise it (query heads are packed per KV head instead)."""
    if n_rep == 1:
        return x
    n_tokens, n_kv_heads, head_dim = x.shape
    return (
        x[:, :, None, :]
        .expand(n_tokens, n_kv_heads, n_rep, head_dim)
        .reshape(n_tokens, n_kv_heads * n_rep, head_dim)
    )


def _repeat_kv_batched(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """GQA head expansion for [n_seqs, ctx, n_kv, hd] (paged_attn.py:356-365)."""
    if n_rep == 1:
        return x
    n_seqs, ctx, n_kv_heads, head_dim = x.shape
    return (
        x[:, :, :, None, :]
        .expand(n_seqs, ctx, n_kv_heads, n_rep, head_dim)
        .reshape(n_seqs, ctx, n_kv_heads * n_rep, head_dim)
    )


def paged_attention_decode_hip(
    query: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: TableArg,
    context_lens: LensArg,
    scale: Optional[float] = None,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    q_per_seq: int = 1,
    max_context_len: Optional[int] = None,
    part_tokens: int = 0,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Fused paged decode / verify attention on raw tensors.

    The form of helios' ``paged_attention_decode_triton(query, k_cache,
    v_cache, block_tables, context_lens, scale)`` (triton_attn.py:133-140),
    extended with int8 pools (``k_scale``/``v_scale`` [num_blocks, n_kv_heads,
    block_size], fp16 or fp32) and with ``q_per_seq`` query tokens per
    sequence (query [n_seqs * q_per_seq, n_q_heads, head_dim], token t of a
    sequence with context c attending keys [0, c - q_per_seq + t]).
    ``block_tables`` / ``context_lens`` may be Python lists (converted like
    triton_attn.py:156-165) or int32 device tensors; with tensors pass
    ``max_context_len`` to avoid a device sync.  ``max_context_len`` only
    sizes the launch: every context is honoured as given, and with list
    contexts a bound below the largest one is rejected.  ``out`` (contiguous,
    query's shape and dtype) and ``workspace`` (uint8, at least
    ``decode_workspace_bytes(...)``, zero-filled before its first use) may be
    passed in to keep the call allocation-free.
    """
    _require_gpu(query, "query")
    n_tok, n_q_heads, head_dim = query.shape
    n_blocks_total, n_kv_heads, block_size, _ = k_cache.shape
    scale = scale or 1.0 / math.sqrt(head_dim)
    dev = query.device
    for t in (k_cache, v_cache, k_scale, v_scale):
        if t is not None and not t.is_contiguous():
            raise ValueError("KV pools and scales must be contiguous")
    if isinstance(block_tables, torch.Tensor):
        tables = _meta(block_tables, "block_tables", dev, 2)
    else:
        tables = _padded_tables(block_tables, dev)
    if isinstance(context_lens, torch.Tensor):
        lens = _meta(context_lens, "context_lens", dev, 1)
        if max_context_len is None:
            max_context_len = int(lens.max().item()) if lens.numel() else 0
    else:
        longest = max((int(c) for c in context_lens), default=0)
        if max_context_len is None:
            max_context_len = longest
        elif max_context_len < longest:
            raise ValueError(f"max_context_len {max_context_len} is below a context of {longest}")
        lens = _i32(list(context_lens), dev)
    n_seqs = lens.shape[0]
    if n_tok != n_seqs * q_per_seq:
        raise ValueError(f"query has {n_tok} rows, expected {n_seqs} x {q_per_seq}")
    if tables.shape[0] < n_seqs:
        raise ValueError(f"block_tables has {tables.shape[0]} rows for {n_seqs} sequences")
    query = query.contiguous()
    out = _out_for(query, out)
    if n_seqs == 0:
        return out
    L = lib()
    ws_bytes = L.hpa_decode_workspace_size(
        n_seqs, q_per_seq, n_q_heads, n_kv_heads, head_dim, max_context_len, part_tokens
    )
    if workspace is not None:
        if workspace.device != dev or not workspace.is_contiguous():
            raise ValueError(f"workspace must be a contiguous tensor on {dev}")
        if workspace.numel() * workspace.element_size() < ws_bytes:
            raise ValueError(f"workspace holds {workspace.nbytes} bytes, {ws_bytes} needed")
        ws = workspace
    else:
        ws = _cached_workspace(dev, ws_bytes)
    quant = k_cache.dtype == torch.int8
    st = L.hpa_paged_decode(
        ptr(query), ptr(out), DTYPE_CODE[query.dtype], ptr(k_cache), ptr(v_cache),
        DTYPE_CODE[k_cache.dtype], ptr(k_scale) if quant else None,
        ptr(v_scale) if quant else None,
        DTYPE_CODE[k_scale.dtype] if (quant and k_scale is not None) else 0,
        ptr(tables), tables.shape[1], ptr(lens), n_seqs, q_per_seq, n_q_heads, n_kv_heads,
        head_dim, block_size, n_blocks_total, max_context_len, float(scale), part_tokens,
        ptr(ws), ws_bytes, stream_ptr(dev),
    )
    check(st, "hpa_paged_decode")
    return out


_WORKSPACES: dict = {}


def _cached_workspace(device: torch.device, nbytes: int) -> Optional[torch.Tensor]:
    """The decode kernel's split-K workspace, one per (device, stream), grown
    on demand.  It starts zero-filled and every call leaves its arrival
    counters at zero, so calls ordered on one stream can share it; calls on
    different streams, which may overlap, get different workspaces."""
    if nbytes == 0:
        return None
    key = (device.type, device.index if device.index is not None else torch.cuda.current_device(),
           stream_ptr(device))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def decode_workspace_bytes(n_seqs: int, q_per_seq: int, n_q_heads: int, n_kv_heads: int,
                           head_dim: int, max_context_len: int, part_tokens: int = 0) -> int:
    """Split-K workspace hpa_paged_decode needs for these shapes."""
    return int(_lib.load_library().hpa_decode_workspace_size(
        n_seqs, q_per_seq, n_q_heads, n_kv_heads, head_dim, max_context_len, part_tokens))


def decode_workspace(n_seqs: int, q_per_seq: int, n_q_heads: int, n_kv_heads: int, head_dim: int,
                     max_context_len: int, device, part_tokens: int = 0) -> torch.Tensor:
    """A zero-filled, caller-owned decode workspace for these shapes (and
    any smaller ones).  Pass it as ``workspace=`` to keep calls free of
    allocation, e.g. under HIP graph capture.  Calls that may overlap need
    workspaces of their own.  If a call did not complete (a launch error),
    zero it again (``reset_decode_workspace``) before reusing it."""
    n = decode_workspace_bytes(n_seqs, q_per_seq, n_q_heads, n_kv_heads, head_dim, max_context_len,
                               part_tokens)
    return torch.zeros(max(n, 1), dtype=torch.uint8, device=device)


def reset_decode_workspace(workspace: torch.Tensor) -> None:
    """Return a workspace's split-K arrival counters to zero.  Every call
    that completes leaves them at zero; this is for a call that did not."""
    workspace.zero_()


def _cache_tensors(kv_cache: PagedKVCache):
    ks, vs = kv_cache._scales()
    return kv_cache.k_cache, kv_cache.v_cache, ks, vs


def _check_query_dtype(query: torch.Tensor, kv_cache: PagedKVCache) -> None:
    if query.dtype != kv_cache.dtype:
        raise RuntimeError(
            f"query dtype {query.dtype} does not match the cache's compute dtype {kv_cache.dtype}"
        )


def paged_attention_decode(
    query: torch.Tensor,
    kv_cache: PagedKVCache,
    block_ids: List[int],
    context_len: int,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Single-token attention for one sequence; query [n_q_heads, head_dim]
    -> [n_q_heads, head_dim] (paged_attn.py:264-295)."""
    n_q_heads, head_dim = query.shape
    scale = scale or 1.0 / math.sqrt(head_dim)
    _check_context(block_ids, context_len, kv_cache.block_size, kv_cache.num_blocks)
    _check_query_dtype(query, kv_cache)
    k, v, ks, vs = _cache_tensors(kv_cache)
    out = paged_attention_decode_hip(
        query.reshape(1, n_q_heads, head_dim), k, v, [list(block_ids)], [context_len], scale,
        ks, vs,
    )
    return out.reshape(n_q_heads, head_dim)


def paged_attention_decode_batched(
    query: torch.Tensor,
    kv_cache: PagedKVCache,
    block_tables: List[List[int]],
    context_lens: List[int],
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Decode for a batch, one query token per sequence; query [n_seqs,
    n_q_heads, head_dim] -> same shape (paged_attn.py:298-353).  An empty
    batch returns ``query`` itself, as helios does."""
    n_seqs, n_q_heads, head_dim = query.shape
    scale = scale or 1.0 / math.sqrt(head_dim)
    if n_seqs == 0:
        return query
    for blocks, ctx in zip(block_tables, context_lens):
        _check_context(blocks, ctx, kv_cache.block_size, kv_cache.num_blocks)
    _check_query_dtype(query, kv_cache)
    k, v, ks, vs = _cache_tensors(kv_cache)
    return paged_attention_decode_hip(query, k, v, block_tables, context_lens, scale, ks, vs)


def paged_attention_verify_batched(
    query: torch.Tensor,
    kv_cache: PagedKVCache,
    block_tables: List[List[int]],
    context_lens: List[int],
    q_per_seq: int,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Speculative verify for a batch: q_per_seq (= gamma + 1) tokens per
    sequence, query [n_seqs * q_per_seq, n_q_heads, head_dim], causal among
    the sequence's own tokens; the last token sits at context_len - 1.  Equals
    one paged_attention_prefill(q_b, cache, table_b, ctx_b - q_per_seq, ctx_b)
    per sequence (the verify call of reference exec/runner.py:354-362)."""
    n_tok, n_q_heads, head_dim = query.shape
    scale = scale or 1.0 / math.sqrt(head_dim)
    for blocks, ctx in zip(block_tables, context_lens):
        _check_context(blocks, ctx, kv_cache.block_size, kv_cache.num_blocks)
    _check_query_dtype(query, kv_cache)
    k, v, ks, vs = _cache_tensors(kv_cache)
    return paged_attention_decode_hip(
        query, k, v, block_tables, context_lens, scale, ks, vs, q_per_seq=q_per_seq
    )


def paged_attention_varlen(
    query: torch.Tensor,
    kv_cache: PagedKVCache,
    block_tables: TableArg,
    query_lens: LensArg,
    start_positions: LensArg,
    context_lens: LensArg,
    scale: Optional[float] = None,
    max_query_len: Optional[int] = None,
    cu_query_lens: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Causal attention for a ragged batch of prompt chunks in one launch.

    query [sum(query_lens), n_q_heads, head_dim]; sequence b's token i sits at
    start_positions[b] + i and attends keys [0, min(start + i + 1,
    context_lens[b])).  Row-for-row equal to calling paged_attention_prefill
    per sequence, which is what reference exec/model.py:303-317 does.
    ``cu_query_lens`` (int32 device tensor [n + 1], the prefix sums of
    ``query_lens``) and ``max_query_len`` may be passed to skip building them
    per call.  Device metadata is not read back: query tokens it places at or
    past ``query``'s last row are neither read nor written, and a sum of
    ``query_lens`` known on the host must equal the row count."""
    _require_gpu(query, "query")
    n_tok, n_q_heads, head_dim = query.shape
    scale = scale or 1.0 / math.sqrt(head_dim)
    _check_query_dtype(query, kv_cache)
    dev = query.device
    if isinstance(block_tables, torch.Tensor):
        tables = _meta(block_tables, "block_tables", dev, 2)
    else:
        for blocks, ctx in zip(block_tables, (context_lens.tolist() if isinstance(context_lens, torch.Tensor) else context_lens)):
            _check_context(blocks, int(ctx), kv_cache.block_size, kv_cache.num_blocks)
        tables = _padded_tables(block_tables, dev)
    if cu_query_lens is not None:
        cu = _meta(cu_query_lens, "cu_query_lens", dev, 1)
        n_seqs = cu.numel() - 1
        if max_query_len is None:
            max_query_len = int((cu[1:] - cu[:-1]).max().item()) if n_seqs > 0 else 0
    elif isinstance(query_lens, torch.Tensor):
        if query_lens.device.type == "cpu" and int(query_lens.sum()) != n_tok:
            raise ValueError(f"query has {n_tok} rows but query_lens sum to {int(query_lens.sum())}")
        qlens_t = query_lens.to(device=dev, dtype=torch.int32)
        cu = torch.zeros(qlens_t.numel() + 1, dtype=torch.int32, device=dev)
        cu[1:] = torch.cumsum(qlens_t, 0)
        if max_query_len is None:
            max_query_len = int(qlens_t.max().item()) if qlens_t.numel() else 0
        n_seqs = qlens_t.numel()
    else:
        ql = [int(x) for x in query_lens]
        acc = [0]
        for x in ql:
            acc.append(acc[-1] + x)
        if acc[-1] != n_tok:
            raise ValueError(f"query has {n_tok} rows but query_lens sum to {acc[-1]}")
        cu = _i32(acc, dev)
        if max_query_len is None:
            max_query_len = max(ql, default=0)
        n_seqs = len(ql)
    pos = (_meta(start_positions, "start_positions", dev, 1) if isinstance(start_positions, torch.Tensor)
           else _i32(list(start_positions), dev))
    lens = (_meta(context_lens, "context_lens", dev, 1) if isinstance(context_lens, torch.Tensor)
            else _i32(list(context_lens), dev))
    if pos.numel() != n_seqs or lens.numel() != n_seqs or tables.shape[0] < n_seqs:
        raise ValueError(f"start_positions, context_lens and block_tables must cover {n_seqs} sequences")
    query = query.contiguous()
    out = _out_for(query, out)
    if n_seqs == 0 or n_tok == 0:
        return out
    k, v, ks, vs = _cache_tensors(kv_cache)
    st = lib().hpa_paged_prefill(
        ptr(query), ptr(out), DTYPE_CODE[query.dtype], ptr(k), ptr(v), DTYPE_CODE[k.dtype],
        ptr(ks), ptr(vs), DTYPE_CODE[ks.dtype] if ks is not None else 0, ptr(tables),
        tables.shape[1], ptr(cu), ptr(pos), ptr(lens), n_seqs, max_query_len, n_tok, n_q_heads,
        kv_cache.n_kv_heads, head_dim, kv_cache.block_size, kv_cache.num_blocks, float(scale),
        stream_ptr(dev),
    )
    check(st, "hpa_paged_prefill")
    return out


def paged_attention_prefill(
    query: torch.Tensor,
    kv_cache: PagedKVCache,
    block_ids: List[int],
    start_pos: int,
    context_len: int,
    scale: Optional[float] = None,
) -> torch.Tensor:
    """Causal attention for one prompt chunk (also the speculative-verify
    pass); query [n_tokens, n_q_heads, head_dim] -> same shape
    (paged_attn.py:368-408)."""
    n_tokens, n_q_heads, head_dim = query.shape
    scale = scale or 1.0 / math.sqrt(head_dim)
    _check_context(block_ids, context_len, kv_cache.block_size, kv_cache.num_blocks)
    return paged_attention_varlen(
        query, kv_cache, [list(block_ids)], [n_tokens], [start_pos], [context_len], scale
    )


def hip_available() -> bool:
    """True when libheliosattn.so is built and a GPU is visible (the analogue
    of helios' triton_available, triton_attn.py:43-49)."""
    return _lib.hip_available()
