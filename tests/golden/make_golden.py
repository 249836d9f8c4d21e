"""Write golden vectors from the reference's own functions (run in the build container only).

Imports inference/ops.py from /root/reference and records input/output vectors of
the functions that closed forms cannot pin bit for bit:
precompute_rope_freqs (torch.polar fp32 table), apply_rope and mla_attention
(the composite of its bf16 rounding points).  rms_norm, fp8_linear and
yarn_get_mscale are pinned by closed forms in tests/test_oracle.py instead.

Inputs come from amla.synth (seeded, sha256 recorded); outputs are stored as
safetensors with a JSON manifest.  Usage:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "deepseek-on-one-gpu_amd"))
sys.path.insert(0, "/root/reference")

from amla import synth  # noqa: E402
from amla.config import DeepSeekConfig  # noqa: E402
from inference import ops as ref  # noqa: E402  (the reference, read-only)

SMALL = dict(hidden_size=320, num_attention_heads=4, q_lora_rank=192, kv_lora_rank=160,
             qk_nope_head_dim=48, qk_rope_head_dim=16, v_head_dim=40, qk_head_dim=64)


def _bits(t: torch.Tensor) -> torch.Tensor:
    """Store bf16 / fp8 tensors by bit pattern so the fixture is exact."""
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16)
    if t.dtype == torch.float8_e4m3fn:
        return t.contiguous().view(torch.uint8)
    return t.contiguous()


def rope_fixtures(out, manifest):
    cfg = DeepSeekConfig()
    tab = ref.precompute_rope_freqs(cfg, 32768, torch.device("cpu"))
    rows = [0, 1, 2, 3, 63, 255, 256, 1000, 4095, 4096, 16383, 32767]
    out["rope.rows"] = torch.tensor(rows, dtype=torch.int64)
    out["rope.table_rows"] = torch.view_as_real(tab[rows]).contiguous()
    out["rope.table_0_64"] = torch.view_as_real(tab[:64]).contiguous()
    manifest["rope"] = {"seq_len": 32768, "rows": rows}

    x = synth.randn((2, 3, 5, 64), synth.seed_of("golden", "apply_rope", "x")).to(torch.bfloat16)
    out["apply_rope.x"] = _bits(x)
    for name, start in (("p0", 0), ("p300", 300), ("p32760", 32760)):
        f = tab[start:start + 5]
        out[f"apply_rope.{name}.y"] = _bits(ref.apply_rope(x, f))
        manifest[f"apply_rope.{name}"] = {"start": start}


def mla_case(out, manifest, key, cfg, tag, B, S, position, filled, max_seq):
    lay = synth.make_layer(cfg, tag)
    hidden = synth.make_hidden(cfg, B, S, tag)
    ckv, kpe = synth.make_kv_cache(cfg, B, max_seq, filled, tag)
    tab = ref.precompute_rope_freqs(cfg, max_seq, torch.device("cpu"))
    y = ref.mla_attention(hidden, lay.attn_weights, (ckv, kpe), position, tab, cfg)
    T = position + S
    out[f"{key}.out"] = _bits(y)
    out[f"{key}.ckv_new"] = _bits(ckv[:, position:T])
    out[f"{key}.kpe_new"] = _bits(kpe[:, position:T])
    sh = {k: synth.sha256_of(v[0]) for k, v in lay.attn_weights.items() if isinstance(v, tuple)}
    sh.update({k: synth.sha256_of(v) for k, v in lay.attn_weights.items() if not isinstance(v, tuple)})
    sh["hidden"] = synth.sha256_of(hidden)
    manifest[key] = {"tag": tag, "B": B, "S": S, "position": position, "filled": filled,
                     "max_seq": max_seq, "cfg": {k: getattr(cfg, k) for k in SMALL}, "sha256": sh}


def main():
    out, manifest = {}, {}
    torch.manual_seed(0)
    rope_fixtures(out, manifest)
    small = DeepSeekConfig(**SMALL)
    mla_case(out, manifest, "small_decode", small, "golden/small_decode", 2, 1, 3, 3, 8)
    mla_case(out, manifest, "small_prefill", small, "golden/small_prefill", 1, 5, 0, 0, 8)
    mla_case(out, manifest, "small_chunk", small, "golden/small_chunk", 2, 3, 4, 4, 12)
    r1 = DeepSeekConfig()
    mla_case(out, manifest, "r1_decode_t257", r1, "golden/r1_decode_t257", 1, 1, 256, 256, 264)
    mla_case(out, manifest, "r1_prefill_s8", r1, "golden/r1_prefill_s8", 1, 8, 0, 0, 8)
    save_file(out, os.path.join(HERE, "reference_vectors.safetensors"))
    with open(os.path.join(HERE, "reference_vectors.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("wrote", len(out), "tensors")


if __name__ == "__main__":
    main()
