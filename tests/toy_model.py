"""helios' toy Llama model, restated for the greedy-decode parity tests -- TEST
INFRASTRUCTURE.

The dense parts (embedding, RMSNorm, rotate-half RoPE, q/k/v/o projections,
SwiGLU MLP, final norm, LM head) follow reference python/helios/exec/model.py
and run in torch fp32; attention goes through a pluggable backend so the same
model drives the NumPy oracle on the CPU and libheliosattn.so on the GPU:

  RMSNorm                  model.py:95-114 (fp32, x * rsqrt(mean(x^2) + eps) * w)
  build_rope_cache         model.py:117-132 (inv_freq = theta^(-2i/d), cos/sin of pos x inv_freq)
  apply_rope               model.py:135-153 (rotate-half: (x1 c - x2 s, x2 c + x1 s))
  Attention.forward        model.py:183-217 (write K/V before attending; decode for a
                           single decode token, causal prefill otherwise)
  MLP                      model.py:321-338 (down(silu(gate x) * up x))
  DecoderLayer.forward     model.py:350-370 (pre-norm, two residuals)
  HeliosModel.forward      model.py:432-463 (logits of the last position only)

Weights: save_toy_model (exec/loader.py:179-210) seeds torch's generator,
constructs HeliosModel -- nn.Embedding's normal_ and nn.Linear's
kaiming_uniform_(a=sqrt(5)) consume the generator in construction order --
then redraws every parameter of rank >= 2 from N(0, 0.02) in registration
order.  toy_weights() replays exactly those draws; tests/golden/toy_greedy.json
holds helios' per-parameter checksums, which pin it.
"""

from __future__ import annotations

import math
from collections import OrderedDict
from typing import Dict, List

import torch
import torch.nn.functional as F

TOY = dict(vocab_size=259, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
           num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512,
           rms_norm_eps=1e-5, rope_theta=10000.0)


def _linear_shapes(cfg) -> List[tuple]:
    H, I = cfg["hidden_size"], cfg["intermediate_size"]
    hd = H // cfg["num_attention_heads"]
    nq, nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    return [("self_attn.q_proj", (nq * hd, H)), ("self_attn.k_proj", (nkv * hd, H)),
            ("self_attn.v_proj", (nkv * hd, H)), ("self_attn.o_proj", (H, nq * hd)),
            ("mlp.gate_proj", (I, H)), ("mlp.up_proj", (I, H)), ("mlp.down_proj", (H, I))]


def toy_weights(cfg=TOY, seed: int = 0) -> Dict[str, torch.Tensor]:
    """The toy checkpoint's parameters, by helios' module names, on the CPU."""
    V, H, L = cfg["vocab_size"], cfg["hidden_size"], cfg["num_hidden_layers"]
    gen_state = torch.random.get_rng_state()
    try:
        torch.manual_seed(seed)
        p: "OrderedDict[str, torch.Tensor]" = OrderedDict()
        # construction: the default initialisers, in module construction order
        p["embed_tokens.weight"] = torch.empty(V, H).normal_()
        for li in range(L):
            for name, shape in _linear_shapes(cfg):
                w = torch.empty(*shape)
                torch.nn.init.kaiming_uniform_(w, a=math.sqrt(5))
                p[f"layers.{li}.{name}.weight"] = w
            p[f"layers.{li}.input_layernorm.weight"] = torch.ones(H)
            p[f"layers.{li}.post_attention_layernorm.weight"] = torch.ones(H)
        p["norm.weight"] = torch.ones(H)
        lm = torch.empty(V, H)
        torch.nn.init.kaiming_uniform_(lm, a=math.sqrt(5))
        p["lm_head.weight"] = lm
        # save_toy_model's re-initialisation, in registration order
        for t in p.values():
            if t.dim() >= 2:
                torch.nn.init.normal_(t, mean=0.0, std=0.02)
        return dict(p)
    finally:
        torch.random.set_rng_state(gen_state)


class AttentionBackend:
    """What the model needs from a paged-attention implementation: one cache per
    layer, write-before-attend, and the two attention entry points."""

    def new_cache(self, layer: int):
        raise NotImplementedError

    def write(self, cache, block_ids, start_pos, k, v):
        raise NotImplementedError

    def decode(self, q, cache, block_ids, context_len, scale):   # q [Hq, D]
        raise NotImplementedError

    def prefill(self, q, cache, block_ids, start_pos, context_len, scale):  # q [T, Hq, D]
        raise NotImplementedError


class ToyModel:
    def __init__(self, weights: Dict[str, torch.Tensor], device: str, cfg=TOY):
        self.cfg = cfg
        self.device = device
        self.w = {k: v.to(device=device, dtype=torch.float32) for k, v in weights.items()}
        self.nq, self.nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
        self.hd = cfg["hidden_size"] // self.nq
        self.scale = 1.0 / math.sqrt(self.hd)
        inv_freq = 1.0 / (cfg["rope_theta"] ** (
            torch.arange(0, self.hd, 2, dtype=torch.float32, device=device) / self.hd))
        pos = torch.arange(cfg["max_position_embeddings"], dtype=torch.float32, device=device)
        freqs = torch.outer(pos, inv_freq)
        self.cos, self.sin = freqs.cos(), freqs.sin()

    def _norm(self, x, w):
        x = x.float()
        var = x.pow(2).mean(-1, keepdim=True)
        return x * torch.rsqrt(var + self.cfg["rms_norm_eps"]) * w

    def _rope(self, x, pos):
        c = self.cos[pos].unsqueeze(1)
        s = self.sin[pos].unsqueeze(1)
        x1, x2 = x.chunk(2, dim=-1)
        return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)

    def forward(self, tokens: List[int], positions: List[int], caches, block_ids: List[int],
                is_decode: bool, context_len: int, attn: AttentionBackend) -> torch.Tensor:
        """One chunk of one sequence; logits [vocab] of its last position."""
        W = self.w
        ids = torch.tensor(tokens, dtype=torch.long, device=self.device)
        pos = torch.tensor(positions, dtype=torch.long, device=self.device)
        n = len(tokens)
        h = W["embed_tokens.weight"][ids]
        for li, cache in enumerate(caches):
            pre = f"layers.{li}."
            x = self._norm(h, W[pre + "input_layernorm.weight"])
            q = (x @ W[pre + "self_attn.q_proj.weight"].T).view(n, self.nq, self.hd)
            k = (x @ W[pre + "self_attn.k_proj.weight"].T).view(n, self.nkv, self.hd)
            v = (x @ W[pre + "self_attn.v_proj.weight"].T).view(n, self.nkv, self.hd)
            q = self._rope(q, pos)
            # a backend that fuses the rotation into its K write gets K as
            # projected, plus the model's rotary tables
            if not getattr(attn, "fused_rope", False):
                k = self._rope(k, pos)
            start = positions[0]
            attn.write(cache, block_ids, start, k, v)
            if is_decode:
                o = attn.decode(q[0], cache, block_ids, context_len, self.scale).reshape(1, -1)
            else:
                o = attn.prefill(q, cache, block_ids, start, context_len, self.scale).reshape(n, -1)
            h = h + o @ W[pre + "self_attn.o_proj.weight"].T
            x = self._norm(h, W[pre + "post_attention_layernorm.weight"])
            m = F.silu(x @ W[pre + "mlp.gate_proj.weight"].T) * (x @ W[pre + "mlp.up_proj.weight"].T)
            h = h + m @ W[pre + "mlp.down_proj.weight"].T
        h = self._norm(h, W["norm.weight"])
        return (h[-1:] @ W["lm_head.weight"].T)[0]


    def forward_tokens(self, tokens: List[int], positions: List[int], caches, attend) -> torch.Tensor:
        """A flattened multi-sequence batch (Attention.forward_batched,
        model.py:219-247, and forward_all_logits): every layer calls
        ``attend(cache, q, k, v)`` with K already rotated, which writes K/V
        and returns the attention output [n, Hq, D]; logits [n, vocab] of
        every row."""
        W = self.w
        ids = torch.tensor(tokens, dtype=torch.long, device=self.device)
        pos = torch.tensor(positions, dtype=torch.long, device=self.device)
        n = len(tokens)
        h = W["embed_tokens.weight"][ids]
        for li, cache in enumerate(caches):
            pre = f"layers.{li}."
            x = self._norm(h, W[pre + "input_layernorm.weight"])
            q = (x @ W[pre + "self_attn.q_proj.weight"].T).view(n, self.nq, self.hd)
            k = (x @ W[pre + "self_attn.k_proj.weight"].T).view(n, self.nkv, self.hd)
            v = (x @ W[pre + "self_attn.v_proj.weight"].T).view(n, self.nkv, self.hd)
            q, k = self._rope(q, pos), self._rope(k, pos)
            o = attend(cache, q, k, v).reshape(n, -1)
            h = h + o @ W[pre + "self_attn.o_proj.weight"].T
            x = self._norm(h, W[pre + "post_attention_layernorm.weight"])
            m = F.silu(x @ W[pre + "mlp.gate_proj.weight"].T) * (x @ W[pre + "mlp.up_proj.weight"].T)
            h = h + m @ W[pre + "mlp.down_proj.weight"].T
        h = self._norm(h, W["norm.weight"])
        return h @ W["lm_head.weight"].T


def int4_draft_weights(weights: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """A stand-in for helios' int4 draft view (exec/qassd.py:153-181): every
    decoder-layer Linear weight rounded to 16 symmetric levels per output
    row, s = absmax / 7, w = clamp(round(w / s), -8, 7) * s.  helios'
    quantize_model is weight quantization, outside the attention path; the
    speculative tests only need a draft that disagrees with the target now
    and then, since the committed tokens must equal the target's greedy
    tokens whatever the draft proposes (tests/quant/test_qassd.py:147-193)."""
    out = {}
    for name, w in weights.items():
        if name.startswith("layers.") and w.dim() == 2:
            s = w.abs().amax(dim=1, keepdim=True).clamp_min(1e-8) / 7.0
            w = torch.clamp(torch.round(w / s), -8, 7) * s
        out[name] = w
    return out


def greedy(model: ToyModel, attn: AttentionBackend, prompt: List[int], n_new: int,
           block_table: List[int]) -> List[int]:
    """Engine-style greedy generation: one prefill of the prompt, then one
    decode step per new token, every step writing its K/V before attending
    (the engine path of tests/parity/test_parity.py:273-304)."""
    caches = [attn.new_cache(li) for li in range(model.cfg["num_hidden_layers"])]
    seq = list(prompt)
    logits = model.forward(seq, list(range(len(seq))), caches, block_table, False, len(seq), attn)
    out = []
    for step in range(n_new):
        nxt = int(torch.argmax(logits))
        out.append(nxt)
        if step + 1 == n_new:
            break
        p = len(seq)
        seq.append(nxt)
        logits = model.forward([nxt], [p], caches, block_table, True, p + 1, attn)
    return out


def checksums(weights: Dict[str, torch.Tensor]) -> Dict[str, tuple]:
    return {k: (float(v.double().sum()), float((v.double() ** 2).sum())) for k, v in weights.items()}


__all__ = ["TOY", "toy_weights", "ToyModel", "AttentionBackend", "greedy", "checksums",
           "int4_draft_weights"]
