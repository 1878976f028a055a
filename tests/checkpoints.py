"""Synthetic DeepSeek-OCR-style safetensors checkpoints for the weight-loading tests.

The tensor names follow the reference's loader (ds_ocr.c:653-686). MoE layer l's weights come from
the same seeds as oracle/bindings.py make_moe_layer(seed_of(l)), so the oracle's quantized blocks of
that layer are the expected device codes: gate_up = normal_bf16(2*I*H, base+10+2e) holds the gate rows
then the up rows (the reference's fused order), down = normal_bf16(H*I, base+11+2e).
"""
import os

import numpy as np

import bindings as B


def _bf16(arr_u16, shape):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr_u16).view(np.int16).reshape(shape)).view(torch.bfloat16)


def _f32(arr, shape):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float32).reshape(shape))


def layer_tensors(l, seed, hidden, inter, n_experts, n_shared, router_dtype="bf16", std=0.02):
    """The MoE layer l's tensors (name -> torch tensor) with make_moe_layer(seed)'s weights."""
    H, I, E, SI = hidden, inter, n_experts, n_shared * inter
    base = seed * 1000
    p = f"model.layers.{l}.mlp."
    t = {}
    rf = B.normal_f32(E * H, base + 1, std)
    if router_dtype == "bf16":
        t[p + "gate.weight"] = _bf16(B.f32_to_bf16_rne(rf), (E, H))
    else:
        t[p + "gate.weight"] = _f32(rf, (E, H))
    for e in range(E):
        gu = B.normal_bf16(2 * I * H, base + 10 + 2 * e, std).reshape(2 * I, H)
        dn = B.normal_bf16(H * I, base + 11 + 2 * e, std)
        t[p + f"experts.{e}.gate_proj.weight"] = _bf16(gu[:I], (I, H))
        t[p + f"experts.{e}.up_proj.weight"] = _bf16(gu[I:], (I, H))
        t[p + f"experts.{e}.down_proj.weight"] = _bf16(dn, (H, I))
    sgu = B.normal_bf16(2 * SI * H, base + 900, std).reshape(2 * SI, H)
    sdn = B.normal_bf16(H * SI, base + 901, std)
    t[p + "shared_experts.gate_proj.weight"] = _bf16(sgu[:SI], (SI, H))
    t[p + "shared_experts.up_proj.weight"] = _bf16(sgu[SI:], (SI, H))
    t[p + "shared_experts.down_proj.weight"] = _bf16(sdn, (H, SI))
    # tensors the MoE path does not read
    t[f"model.layers.{l}.self_attn.q_proj.weight"] = _bf16(B.normal_bf16(H * H, base + 7, std), (H, H))
    t[f"model.layers.{l}.input_layernorm.weight"] = _f32(np.ones(H, np.float32), (H,))
    return t


def write_checkpoint(dirpath, layers, hidden=256, inter=128, n_experts=16, n_shared=2, vocab=5000, lm_seed=77):
    """layers: [(l, seed, router_dtype)]. Writes one shard per MoE layer plus one with the LM head
    and the embedding; returns the shard paths."""
    from safetensors.torch import save_file
    files = []
    for i, (l, seed, rdt) in enumerate(layers):
        path = os.path.join(dirpath, f"model-{i + 1:05d}-of-{len(layers) + 1:05d}.safetensors")
        save_file(layer_tensors(l, seed, hidden, inter, n_experts, n_shared, rdt), path, metadata={"format": "pt"})
        files.append(path)
    path = os.path.join(dirpath, f"model-{len(layers) + 1:05d}-of-{len(layers) + 1:05d}.safetensors")
    save_file({"lm_head.weight": _bf16(lm_head(vocab, hidden, lm_seed), (vocab, hidden)),
               "model.norm.weight": _f32(np.ones(hidden, np.float32), (hidden,))}, path)
    files.append(path)
    return files


def lm_head(vocab, hidden, seed=77):
    return B.normal_bf16(vocab * hidden, seed, 0.02)
