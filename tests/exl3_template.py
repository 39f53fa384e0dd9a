"""A synthetic EXL3 model directory for the writer tests.

The layout matches what export_exl3.py splices into (export_exl3.py:86-148 of
the reference): model.safetensors.index.json with a weight_map over several
safetensors shards, per-module trellis/suh/svh tensors (plus the .mul1 codebook
scalar EXL3 stores per module), non-quantized tensors (norms, embeddings), an
lm_head outside the decoder layers, config/tokenizer files and an
ARTIFACTS.sha256.  Tensor contents are seeded random bytes.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import torch
from safetensors.torch import save_file


def make_template(root, modules, seed: int = 0, n_shards: int = 2) -> Path:
    """modules: [(layer, module, k_in, n_out, K)].  Returns the template dir."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    gen = torch.Generator().manual_seed(seed)
    tensors = {}
    for layer, module, k, n, K in modules:
        base = f"model.language_model.layers.{layer}.{module}"
        tensors[base + ".trellis"] = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K),
                                                   generator=gen, dtype=torch.int16)
        tensors[base + ".suh"] = torch.randn(k, generator=gen).half()
        tensors[base + ".svh"] = torch.randn(n, generator=gen).half()
        tensors[base + ".mul1"] = torch.tensor([0x83DCD12D], dtype=torch.int64)
        tensors[f"model.language_model.layers.{layer}.input_layernorm.weight"] = \
            torch.randn(k, generator=gen).to(torch.bfloat16)
    k0 = modules[0][2]
    tensors["model.language_model.embed_tokens.weight"] = torch.randn(64, k0, generator=gen).half()
    tensors["lm_head.trellis"] = torch.randint(-32768, 32768, (k0 // 16, 4, 64), generator=gen,
                                               dtype=torch.int16)
    tensors["lm_head.suh"] = torch.randn(k0, generator=gen).half()
    tensors["lm_head.svh"] = torch.randn(64, generator=gen).half()

    keys = sorted(tensors)
    weight_map = {}
    for i in range(n_shards):
        name = f"model-{i + 1:05d}-of-{n_shards:05d}.safetensors"
        part = {k: tensors[k].contiguous() for j, k in enumerate(keys) if j % n_shards == i}
        save_file(part, str(root / name), metadata={"format": "pt"})
        weight_map.update({k: name for k in part})
    (root / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {"total_size": 0}, "weight_map": weight_map}, indent=2))
    (root / "config.json").write_text(json.dumps({
        "model_type": "qwen3", "quantization_config": {"quant_method": "exl3", "bits": 5.0}}))
    (root / "quantization_config.json").write_text(json.dumps({"codebook": "mul1"}))
    (root / "tokenizer.json").write_text("{}")
    lines = []
    for item in sorted(root.iterdir()):
        if item.is_file():
            lines.append(f"{hashlib.sha256(item.read_bytes()).hexdigest()}  {item.name}")
    (root / "ARTIFACTS.sha256").write_text("stale\n" + "\n".join(lines) + "\n")
    return root
