"""Write tests/golden/hf_tiny.npz: HF transformers LlamaForCausalLM outputs for tiny seeded configs.

transformers is an independent third-party implementation of Llama (not the reference).  The weights
are oracle.model.random_weights(cfg, seed, std) (regenerated bit-identically by the tests from the
seed, so the fixture stores only inputs and outputs); they are written as an HF checkpoint and loaded
by LlamaForCausalLM.  Variants mirror the reference's test_matches_hf (tests/test_model.py:9-36):
default RoPE, tied embeddings, llama3 RoPE scaling (the prompt crosses its frequency bands).

    python tests/golden/make_hf_golden.py
"""

from __future__ import annotations

import json
import sys
import tempfile
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.model import OracleConfig, random_weights  # noqa: E402

LLAMA3_ROPE = {"rope_type": "llama3", "rope_theta": 500000.0, "factor": 8.0, "low_freq_factor": 1.0,
               "high_freq_factor": 4.0, "original_max_position_embeddings": 64}
VARIANTS = {
    "default": dict(tie=False, rope=None, theta=10000.0),
    "tied": dict(tie=True, rope=None, theta=10000.0),
    "llama3_rope": dict(tie=False, rope=LLAMA3_ROPE, theta=500000.0),
}
SEED, STD, N_IDS = 1, 0.1, 150


def oracle_cfg(v: dict) -> OracleConfig:
    sc = None
    if v["rope"] is not None:
        sc = dict(v["rope"])
    return OracleConfig(vocab_size=64, dim=64, n_layers=6, n_heads=4, n_kv_heads=2, head_dim=16,
                        intermediate_size=128, norm_eps=1e-5, rope_theta=v["theta"], max_position_embeddings=512,
                        tie_word_embeddings=v["tie"], rope_scaling=sc)


def hf_config(v: dict) -> dict:
    rope = v["rope"] or {"rope_type": "default", "rope_theta": v["theta"]}
    return {"architectures": ["LlamaForCausalLM"], "model_type": "llama", "vocab_size": 64, "hidden_size": 64,
            "intermediate_size": 128, "num_hidden_layers": 6, "num_attention_heads": 4, "num_key_value_heads": 2,
            "max_position_embeddings": 512, "rms_norm_eps": 1e-5, "tie_word_embeddings": v["tie"],
            "bos_token_id": 1, "eos_token_id": 2, "rope_parameters": rope, "torch_dtype": "float32",
            "hidden_act": "silu", "attention_bias": False, "mlp_bias": False}


def main() -> None:
    from safetensors.torch import save_file
    from transformers import LlamaForCausalLM

    out = {}
    ids = torch.randint(3, 64, (1, N_IDS), generator=torch.Generator().manual_seed(0))
    ids[0, 0] = 1
    out["ids"] = ids[0].numpy()
    for name, v in VARIANTS.items():
        cfg = oracle_cfg(v)
        w = random_weights(cfg, seed=SEED, std=STD)
        with tempfile.TemporaryDirectory() as d:
            (Path(d) / "config.json").write_text(json.dumps(hf_config(v)))
            save_file({k: t.contiguous() for k, t in w.items()}, str(Path(d) / "model.safetensors"))
            hf = LlamaForCausalLM.from_pretrained(d, dtype=torch.float32).eval()
            with torch.inference_mode():
                res = hf(ids, output_hidden_states=True)
                nxt = int(res.logits[0, -1].argmax())
                res2 = hf(torch.cat([ids, torch.tensor([[nxt]])], 1))
        out[f"{name}/logits_last"] = res.logits[0, -1].numpy()
        out[f"{name}/hidden_last"] = np.stack([h[0, -1].numpy() for h in res.hidden_states[1:]])
        out[f"{name}/next_token"] = np.array(nxt)
        out[f"{name}/decode_logits"] = res2.logits[0, -1].numpy()
    path = Path(__file__).with_name("hf_tiny.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
