"""A synthetic checkpoint directory in the R1 release layout (model.safetensors.index.json +
two shards; expert tensors model.layers.L.mlp.experts.E.{gate,up,down}_proj.{weight,
weight_scale_inv}), for the expert-store tests."""
import json
import os

import torch
from safetensors.torch import save_file

from amla import synth

PROJ = ("gate_proj", "up_proj", "down_proj")
SHARDS = ("model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors")


def expert(d, i, l, e, tag="store"):
    out = {}
    for p in PROJ:
        shape = (i, d) if p != "down_proj" else (d, i)
        out[p] = synth.quantize_fp8_blocks(synth.randn(shape, synth.seed_of(tag, l, e, p), 0.02))
    return out


def write_checkpoint(path, d, i, experts, layers, tag="store") -> dict:
    """Writes the checkpoint; returns {(layer, e): {proj: (fp8 weight, fp32 scales)}}.  Layer 0 sits
    in the first shard, the others in the second, except that the last expert of the last layer
    keeps its scales in the first shard (one expert over two files)."""
    ref = {(l, e): expert(d, i, l, e, tag) for l in range(layers) for e in range(experts)}
    shards = {s: {} for s in SHARDS}
    weight_map = {}
    for (l, e), ex in ref.items():
        for p in PROJ:
            for kind, t in (("weight", ex[p][0]), ("weight_scale_inv", ex[p][1])):
                split = l == layers - 1 and e == experts - 1 and kind != "weight"
                shard = SHARDS[0] if l == 0 or split else SHARDS[1]
                key = f"model.layers.{l}.mlp.experts.{e}.{p}.{kind}"
                shards[shard][key] = t.contiguous()
                weight_map[key] = shard
    shards[SHARDS[0]]["model.layers.0.self_attn.o_proj.weight"] = torch.zeros(4, 4)
    weight_map["model.layers.0.self_attn.o_proj.weight"] = SHARDS[0]
    for name, tensors in shards.items():
        save_file(tensors, os.path.join(path, name))
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    return ref
