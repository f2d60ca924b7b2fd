"""Writes tests/golden/toy_greedy.json: helios' own greedy token ids for its toy
model -- the one part of the attention path's parity bar that only running
helios can pin.

Run once, in a container that holds the reference checkout, from the repo
root:

    python tests/golden/make_toy_greedy.py /path/to/helios/python

It imports helios (reference python/helios), builds the toy model exactly as
the reference's parity tests do (TOY_CONFIG and seed 0,
tests/parity/test_parity.py:36-53; weights by save_toy_model,
exec/loader.py:179-231), and for each prompt records

  * the greedy tokens of the direct forward loop that re-runs the whole
    sequence each step (tests/parity/test_parity.py:273-304),
  * the same prompt through helios' engine (paged prefill + decode), which
    must agree,
  * the top-1 / top-2 logit margin of every step (how much numerical
    headroom a token has), and
  * per-parameter checksums of the toy weights, which pin the test-side
    restatement of the weight initialisation.

Nothing from helios is written out except these numbers.
"""

from __future__ import annotations

import json
import os
import shutil
import sys
import tempfile

import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "toy_greedy.json")

PROMPTS = [
    ([5, 9, 14, 22, 33], 8),                               # the reference test's case
    ([(7 * i + 3) % 256 + 3 for i in range(37)], 30),      # crosses four 16-token blocks
]


def main(helios_python: str) -> None:
    sys.path.insert(0, helios_python)
    from helios.core.types import SamplingParams
    from helios.engine import EngineConfig, LLMEngine
    from helios.exec.loader import load_model, save_toy_model
    from helios.exec.model import ModelConfig
    from helios.exec.paged_attn import PagedKVCache

    cfg = ModelConfig(vocab_size=259, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)
    tmp = tempfile.mkdtemp(prefix="toy_greedy_")
    try:
        save_toy_model(tmp, cfg, seed=0)
        model = load_model(tmp)
        weights = {}
        for name, p in model.named_parameters():
            t = p.detach().double()
            weights[name] = {"shape": list(p.shape), "sum": float(t.sum()), "sumsq": float((t * t).sum())}

        cases = []
        for prompt, n_new in PROMPTS:
            seq, toks, margins = list(prompt), [], []
            with torch.inference_mode():
                for _ in range(n_new):
                    caches = [PagedKVCache(64, 16, cfg.num_key_value_heads, cfg.head_dim)
                              for _ in range(cfg.num_hidden_layers)]
                    blocks = list(range(len(seq) // 16 + 1))
                    logits = model.forward(seq, list(range(len(seq))), caches, blocks, False, len(seq))[0]
                    top = torch.topk(logits.double(), 2)
                    nxt = int(top.indices[0])
                    margins.append(float(top.values[0] - top.values[1]))
                    toks.append(nxt)
                    seq.append(nxt)
            engine = LLMEngine(EngineConfig(model_dir=tmp, kv_cache_bytes=8 * 1024 * 1024, block_size=16,
                                            max_model_len=256))
            engine.add_request("g", list(prompt), SamplingParams(max_tokens=n_new, temperature=0.0))
            got = engine.run_until_complete()[0].token_ids
            assert list(got) == toks, (got, toks)
            cases.append({"prompt": list(prompt), "n_new": n_new, "tokens": toks, "margins": margins})
    finally:
        shutil.rmtree(tmp, ignore_errors=True)

    data = {
        "source": "helios toy model (TOY_CONFIG, seed 0); direct greedy loop == engine greedy",
        "config": {"vocab_size": 259, "hidden_size": 64, "intermediate_size": 128, "num_hidden_layers": 2,
                   "num_attention_heads": 4, "num_key_value_heads": 2, "max_position_embeddings": 512,
                   "rms_norm_eps": 1e-5, "rope_theta": 10000.0, "seed": 0},
        "torch": torch.__version__,
        "weights": weights,
        "cases": cases,
    }
    with open(OUT, "w") as f:
        json.dump(data, f, indent=1)
    print("wrote", OUT)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/python")
