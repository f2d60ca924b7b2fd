"""NumPy restatement of helios' paged-attention path -- TEST INFRASTRUCTURE.

This module is the checker for libheliosattn.so and the CPU baseline of
bench.py.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import it; the product never does.

Every function follows the reference file:line it cites (reference =
anish41338/helios, python/helios/exec/paged_attn.py unless stated).  How
each one is pinned (tests/test_oracle.py):

  round_bf16               torch's own float32 -> bfloat16 conversion on
                           random values, ties and carries into the exponent
  quantize / store_scale   closed form + hand-built round-half-even ties,
                           clamp and zero-row cases, an independent float64
                           division, and the round-trip bound of the
                           reference's tests/quant/test_kv_quant.py:61-90
  apply_rope               position 0 is the identity, exact hand-computed
                           rotations, and bit-equality with torch's CPU
                           elementwise ops evaluating helios' expression
  PagedPool.write/gather   closed-form position -> (block, offset) mapping,
                           scattered-block round trips and the IndexError
                           texts of tests/parity/test_parity.py:134-148 and
                           tests/quant/test_kv_quant.py:134-152
  attention_*              brute-force softmax attention in pure Python
                           (math.exp) on tiny inputs, the dense reference of
                           tests/parity/test_parity.py:77-86, chunked ==
                           single-shot, GQA head mapping, order invariance
  paged_verify_batched     equals per-sequence prefill (runner.py:354-362)
  paged_varlen             per-token brute force on each sequence's dense
                           K/V across a ragged batch (row offsets, an empty
                           chunk, per-sequence starts, a context cutting a
                           chunk's causal reach), with planted offset /
                           start / table mistakes shown to fail

No function here is "parity unpinned".  The math runs in float64 unless a
function says otherwise; empty softmax rows give NaN exactly as helios'
torch code does (-inf everywhere), and callers compare against the GPU's
defined zeros where that case matters.
"""

from __future__ import annotations

import math
from typing import List, Optional, Sequence, Tuple

import numpy as np

F32 = np.float32


# ------------------------------------------------------------ int8 quantizer


def quantize(x: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """QuantizedPagedKVCache._quantize (paged_attn.py:177-183).

    x: [..., head_dim] -> (int8 payload, fp32 scale [...]).  absmax over the
    last axis in fp32, clamped to >= fp32(1e-8); s = absmax / 127 (IEEE fp32
    division); q = round-half-even(x / s) (fp32 division per element),
    clamped to [-127, 127].
    """
    x = np.asarray(x, dtype=F32)
    absmax = np.abs(x).max(axis=-1)
    absmax = np.maximum(absmax, F32(1e-8))
    scale = (absmax / F32(127.0)).astype(F32)
    q = np.rint(x / scale[..., None]).astype(F32)
    q = np.clip(q, -127, 127).astype(np.int8)
    return q, scale


def store_scale(scale: np.ndarray, scale_dtype=np.float16) -> np.ndarray:
    """Scale as stored: `ks[i].to(torch.float16)` (paged_attn.py:210-211),
    round to nearest even; or kept fp32 (the configs' fp32-scale mode)."""
    return np.asarray(scale, dtype=F32).astype(scale_dtype)


def dequantize(q: np.ndarray, s_stored: np.ndarray, out_dtype=np.float32) -> np.ndarray:
    """QuantizedPagedKVCache.gather's deq (paged_attn.py:228-233):
    (q.float() * s.float()).to(dtype).  out_dtype "bfloat16" rounds to
    bfloat16 (returned as the float32 values it represents)."""
    prod = q.astype(F32) * np.asarray(s_stored).astype(F32)[..., None]
    if isinstance(out_dtype, str) and out_dtype == "bfloat16":
        return round_bf16(prod)
    return prod.astype(out_dtype)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16, round to nearest even (torch's .to(torch.bfloat16)),
    as float32.  Finite inputs only."""
    u = np.asarray(x, dtype=F32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(F32)


# ------------------------------------------------------------------ KV pool


# ------------------------------------------------------------------ rotary


def build_rope_cache(max_pos: int, head_dim: int, theta: float = 10000.0) -> Tuple[np.ndarray, np.ndarray]:
    """exec/model.py:117-132: inv_freq = 1 / theta^(2i/d), cos and sin of
    pos x inv_freq, [max_pos, head_dim / 2] float32.  (Tests that need
    helios' exact tables build them with torch; callers pass tables in.)"""
    inv = (1.0 / (np.float32(theta) ** (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim))))
    freqs = np.outer(np.arange(max_pos, dtype=np.float32), inv.astype(np.float32)).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, positions: np.ndarray) -> np.ndarray:
    """exec/model.py:135-153, rotate-half: x [n, heads, d] (promoted to
    float32), c, s = cos/sin[positions]; (x1 c - x2 s, x2 c + x1 s).  Every
    product and sum is a separate float32 operation, rounded on its own, as
    torch's elementwise ops round them."""
    x = np.asarray(x, dtype=np.float32)
    c = np.asarray(cos, np.float32)[positions][:, None, :]
    s = np.asarray(sin, np.float32)[positions][:, None, :]
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate((x1 * c - x2 * s, x2 * c + x1 * s), axis=-1).astype(np.float32)


class PagedPool:
    """PagedKVCache / QuantizedPagedKVCache storage (paged_attn.py:25-245).

    k, v: [num_blocks, n_kv_heads, block_size, head_dim]; int8 pools carry
    k_scale / v_scale [num_blocks, n_kv_heads, block_size] of scale_dtype.
    `dtype` is the compute dtype gather returns.
    """

    def __init__(self, num_blocks, block_size, n_kv_heads, head_dim, dtype=np.float32,
                 quantized=False, scale_dtype=np.float16):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.quantized = quantized
        shape = (num_blocks, n_kv_heads, block_size, head_dim)
        if quantized:
            self.k = np.zeros(shape, np.int8)
            self.v = np.zeros(shape, np.int8)
            self.k_scale = np.ones(shape[:3], scale_dtype)
            self.v_scale = np.ones(shape[:3], scale_dtype)
        else:
            self.k = np.zeros(shape, dtype)
            self.v = np.zeros(shape, dtype)
            self.k_scale = self.v_scale = None

    def write(self, block_ids: Sequence[int], start_pos: int, k: np.ndarray, v: np.ndarray) -> None:
        """paged_attn.py:57-85 / :185-211: position p -> block
        block_ids[p // bs], offset p % bs; raises at the first position
        without a block, after writing the ones before it."""
        n = k.shape[0]
        if n == 0:
            return
        if self.quantized:
            kq, ks = quantize(np.asarray(k, F32))
            vq, vs = quantize(np.asarray(v, F32))
        for i in range(n):
            pos = start_pos + i
            lb, off = pos // self.block_size, pos % self.block_size
            if lb >= len(block_ids):
                raise IndexError(
                    f"position {pos} needs logical block {lb} but the "
                    f"sequence has only {len(block_ids)} blocks"
                )
            phys = block_ids[lb]
            if self.quantized:
                self.k[phys, :, off, :] = kq[i]
                self.v[phys, :, off, :] = vq[i]
                self.k_scale[phys, :, off] = store_scale(ks[i], self.k_scale.dtype)
                self.v_scale[phys, :, off] = store_scale(vs[i], self.v_scale.dtype)
            else:
                self.k[phys, :, off, :] = np.asarray(k[i]).astype(self.k.dtype)
                self.v[phys, :, off, :] = np.asarray(v[i]).astype(self.v.dtype)

    def gather(self, block_ids: Sequence[int], context_len: int) -> Tuple[np.ndarray, np.ndarray]:
        """paged_attn.py:87-110 / :213-235 -> [context_len, n_kv_heads, head_dim]."""
        if context_len == 0:
            e = np.zeros((0, self.n_kv_heads, self.head_dim), self.dtype)
            return e, e
        nb = (context_len + self.block_size - 1) // self.block_size
        if nb > len(block_ids):
            raise IndexError(f"context_len {context_len} needs {nb} blocks, have {len(block_ids)}")
        idx = np.asarray(block_ids[:nb], dtype=np.int64)

        def take(pool, scales):
            x = pool[idx].transpose(0, 2, 1, 3).reshape(-1, self.n_kv_heads, self.head_dim)
            x = x[:context_len]
            if scales is None:
                return x.astype(self.dtype)
            s = scales[idx].transpose(0, 2, 1).reshape(-1, self.n_kv_heads)[:context_len]
            return dequantize(x, s, self.dtype)

        return take(self.k, self.k_scale), take(self.v, self.v_scale)

    def copy_block(self, src: int, dst: int) -> None:
        """paged_attn.py:112-115 / :237-245 (scales included)."""
        self.k[dst] = self.k[src]
        self.v[dst] = self.v[src]
        if self.quantized:
            self.k_scale[dst] = self.k_scale[src]
            self.v_scale[dst] = self.v_scale[src]


# ---------------------------------------------------------------- attention


def _softmax_rows(scores: np.ndarray) -> np.ndarray:
    """torch.softmax over the last axis; an all -inf row gives NaN, as torch does."""
    m = np.max(scores, axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        e = np.exp(scores - m)
        return e / e.sum(axis=-1, keepdims=True)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, q_positions: np.ndarray,
              scale: float) -> np.ndarray:
    """Masked GQA attention in float64.

    q [T, Hq, D], k/v [ctx, Hkv, D]; query row i may attend keys
    0..q_positions[i] (paged_attn.py:401-404).  Query head h reads KV head
    h // (Hq / Hkv) (paged_attn.py:248-261, triton_attn.py:83).
    """
    T, Hq, D = q.shape
    ctx, Hkv, _ = k.shape
    rep = Hq // Hkv
    q64 = q.astype(np.float64)
    k64 = np.repeat(k.astype(np.float64), rep, axis=1)  # [ctx, Hq, D]
    v64 = np.repeat(v.astype(np.float64), rep, axis=1)
    scores = np.einsum("thd,khd->htk", q64, k64) * scale
    mask = np.arange(ctx)[None, :] > np.asarray(q_positions)[:, None]  # [T, ctx]
    scores = np.where(mask[None], -np.inf, scores)
    p = _softmax_rows(scores)
    return np.einsum("htk,khd->thd", p, v64)


def attention_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """paged_attention_decode's math (paged_attn.py:282-295): q [Hq, D]
    attends every key."""
    out = attention(q[None], k, v, np.array([k.shape[0] - 1]), scale)
    return out[0]


def default_scale(head_dim: int, scale: Optional[float]) -> float:
    """`scale or 1.0 / math.sqrt(head_dim)` (paged_attn.py:283, :322, :389)."""
    return scale or 1.0 / math.sqrt(head_dim)


def paged_decode(q, pool: PagedPool, block_ids, context_len, scale=None):
    """paged_attention_decode (paged_attn.py:264-295), q [Hq, D]."""
    scale = default_scale(q.shape[-1], scale)
    k, v = pool.gather(block_ids, context_len)
    return attention_decode(q, k, v, scale)


def paged_decode_batched(q, pool: PagedPool, block_tables, context_lens, scale=None):
    """paged_attention_decode_batched (paged_attn.py:298-353), q [B, Hq, D].
    Padding keys are masked, so this is the per-sequence decode."""
    scale = default_scale(q.shape[-1], scale)
    if q.shape[0] == 0:
        return q
    return np.stack([paged_decode(q[i], pool, t, c, scale)
                     for i, (t, c) in enumerate(zip(block_tables, context_lens))])


def paged_prefill(q, pool: PagedPool, block_ids, start_pos, context_len, scale=None):
    """paged_attention_prefill (paged_attn.py:368-408), q [T, Hq, D]."""
    scale = default_scale(q.shape[-1], scale)
    k, v = pool.gather(block_ids, context_len)
    pos = start_pos + np.arange(q.shape[0])
    return attention(q, k, v, pos, scale)


def paged_verify_batched(q, pool: PagedPool, block_tables, context_lens, q_per_seq, scale=None):
    """Speculative verify of every sequence: q [B * T, Hq, D]; the verify
    call of reference exec/runner.py:354-362 is paged_attention_prefill with
    start_pos = context_len - T."""
    scale = default_scale(q.shape[-1], scale)
    T = q_per_seq
    outs = [paged_prefill(q[i * T:(i + 1) * T], pool, t, c - T, c, scale)
            for i, (t, c) in enumerate(zip(block_tables, context_lens))]
    return np.concatenate(outs, axis=0) if outs else q


def paged_varlen(q, pool: PagedPool, block_tables, query_lens, start_positions, context_lens,
                 scale=None):
    """BatchedAttention.run's prefill branch (reference exec/model.py:303-317):
    one paged_attention_prefill per sequence over its token span."""
    scale = default_scale(q.shape[-1], scale)
    outs, lo = [], 0
    for t, n, s, c in zip(block_tables, query_lens, start_positions, context_lens):
        outs.append(paged_prefill(q[lo:lo + n], pool, t, s, c, scale))
        lo += n
    return np.concatenate(outs, axis=0) if outs else q


def dense_causal_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_rep: int) -> np.ndarray:
    """The reference's unpaged oracle (tests/parity/test_parity.py:77-86):
    q/k/v of one sequence, causal, scale 1/sqrt(D)."""
    T = q.shape[0]
    return attention(q, k, v, np.arange(T), 1.0 / math.sqrt(q.shape[-1]))


def brute_force_attention(q, k, v, q_positions, scale) -> List[List[List[float]]]:
    """Softmax attention with explicit Python loops and math.exp; tiny inputs
    only.  Independent of numpy's vector code: used to pin `attention`."""
    T, Hq, D = q.shape
    ctx, Hkv, _ = k.shape
    rep = Hq // Hkv
    out = []
    for t in range(T):
        rows = []
        for h in range(Hq):
            kh = h // rep
            keys = [j for j in range(ctx) if j <= q_positions[t]]
            s = [sum(float(q[t, h, d]) * float(k[j, kh, d]) for d in range(D)) * scale for j in keys]
            if not s:
                rows.append([float("nan")] * D)
                continue
            mx = max(s)
            e = [math.exp(x - mx) for x in s]
            z = sum(e)
            rows.append([sum(e[i] * float(v[j, kh, d]) for i, j in enumerate(keys)) / z
                         for d in range(D)])
        out.append(rows)
    return out


# ------------------------------------------------- helios' CPU route (baseline)


def helios_cpu_decode_batched_fp32(q, pool: PagedPool, block_tables, context_lens, scale=None):
    """The exact route of paged_attention_decode_batched on CPU, in fp32
    (helios' CPU dtype, reference engine.py:135-138): gather every sequence
    into a right-padded [B, max_ctx, Hkv, D] tensor (:328-337), expand GQA
    heads (:340-341), batched matmul, -inf pad mask (:346-349), fp32 softmax,
    matmul.  Timed as bench.py's CPU baseline, not used as the checker."""
    B, Hq, D = q.shape
    scale = default_scale(D, scale)
    max_ctx = max(context_lens)
    rep = Hq // pool.n_kv_heads
    kp = np.zeros((B, max_ctx, pool.n_kv_heads, D), F32)
    vp = np.zeros_like(kp)
    for i, (t, c) in enumerate(zip(block_tables, context_lens)):
        k, v = pool.gather(t, c)
        kp[i, :c] = k
        vp[i, :c] = v
    kr = np.repeat(kp, rep, axis=2).transpose(0, 2, 1, 3)  # [B, Hq, ctx, D]
    vr = np.repeat(vp, rep, axis=2).transpose(0, 2, 1, 3)
    scores = np.matmul(q.astype(F32)[:, :, None, :], kr.transpose(0, 1, 3, 2)) * F32(scale)
    idx = np.arange(max_ctx)[None, None, None, :]
    scores = np.where(idx >= np.asarray(context_lens)[:, None, None, None], -np.inf, scores)
    p = _softmax_rows(scores).astype(F32)
    return np.matmul(p, vr)[:, :, 0, :]


def helios_cpu_prefill_fp32(q, pool: PagedPool, block_ids, start_pos, context_len, scale=None):
    """paged_attention_prefill's CPU route in fp32 (paged_attn.py:388-408):
    gather, GQA expansion, [Hq, T, ctx] scores, causal mask, softmax, PV."""
    T, Hq, D = q.shape
    scale = default_scale(D, scale)
    k, v = pool.gather(block_ids, context_len)
    rep = Hq // pool.n_kv_heads
    kr = np.repeat(k.astype(F32), rep, axis=1).transpose(1, 2, 0)  # [Hq, D, ctx]
    vr = np.repeat(v.astype(F32), rep, axis=1).transpose(1, 0, 2)  # [Hq, ctx, D]
    scores = np.matmul(q.astype(F32).transpose(1, 0, 2), kr) * F32(scale)  # [Hq, T, ctx]
    mask = np.arange(context_len)[None, :] > (start_pos + np.arange(T))[:, None]
    scores = np.where(mask[None], -np.inf, scores)
    p = _softmax_rows(scores).astype(F32)
    return np.matmul(p, vr).transpose(1, 0, 2)
