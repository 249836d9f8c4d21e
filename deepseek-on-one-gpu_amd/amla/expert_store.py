"""Routed-expert weights from safetensors shards into a pinned host arena: the
counterpart of inference/weight_store.py:42-77 (ExpertCache) and :156-206
(`_load_expert_from_disk`, `get_expert`).

The reference reads each expert tensor with ``safe_open(...).get_tensor`` into an
ordinary CPU tensor, allocates a new pinned tensor per tensor (``pin_memory``) and
copies into it, and evicts whole entries from an LRU measured in bytes.  Here the
pinned memory is one arena allocated once, cut into expert-sized slots; a miss
reads the six tensors of the expert (three fp8 weights, three fp32 scale grids)
straight from the shard files into its slot with ``readinto`` at the offsets of
the shard header (no intermediate tensor, no per-miss pinned allocation).

A slot is refilled only after the device copies that read it have finished:
the streamer reports the event that follows its copies (``note_copy``) and the
store waits for it before overwriting the slot.
"""
from __future__ import annotations

import json
import math
import os
import re
import struct
from collections import OrderedDict

import torch

PROJ = ("gate_proj", "up_proj", "down_proj")
EXPERT_KEY = re.compile(
    r"model\.layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate_proj|up_proj|down_proj)\.(weight|weight_scale_inv)")

_DTYPES = {"F8_E4M3": torch.float8_e4m3fn, "F32": torch.float32, "BF16": torch.bfloat16, "F16": torch.float16}


def expert_tensor_keys(layer: int, expert: int) -> list[str]:
    """weight_store.py:28-35: the six safetensors keys of one expert."""
    prefix = f"model.layers.{layer}.mlp.experts.{expert}"
    return [f"{prefix}.{p}.{s}" for p in PROJ for s in ("weight", "weight_scale_inv")]


def read_header(path: str) -> tuple[dict, int]:
    """(tensor name -> {dtype, shape, data_offsets}, byte offset of the data section) of one shard."""
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
    header.pop("__metadata__", None)
    return header, 8 + n


class ExpertStore:
    """Expert weights of one checkpoint directory (``model.safetensors.index.json`` + shards)
    behind an LRU of pinned host slots.

    ``get_expert(layer, e)`` returns ``{proj: (weight, weight_scale_inv)}`` as pinned host
    tensors, the return shape of weight_store.py:183-206.  The views stay valid until the
    slot is evicted, which happens only after the device copies reported for it finished.
    """

    def __init__(self, model_path: str, config, capacity_bytes: int = 16 << 30, verbose: bool = False,
                 pinned: bool | None = None):
        self.path = str(model_path)
        self.config = config
        self.verbose = verbose
        with open(os.path.join(self.path, "model.safetensors.index.json")) as f:
            weight_map = json.load(f)["weight_map"]
        self.shard_of = {k: v for k, v in weight_map.items() if EXPERT_KEY.match(k)}
        self._headers: dict[str, tuple[dict, int]] = {}
        h, n = config.hidden_size, config.moe_intermediate_size
        w_shapes = {"gate_proj": (n, h), "up_proj": (n, h), "down_proj": (h, n)}
        # slot layout: the three fp8 weights, then the three fp32 scale grids (16-byte aligned)
        self.layout = {}
        off = 0
        for p in PROJ:
            r, c = w_shapes[p]
            self.layout[(p, "weight")] = (off, (r, c), torch.float8_e4m3fn)
            off += (r * c + 15) // 16 * 16
        for p in PROJ:
            r, c = w_shapes[p]
            sr, sc = math.ceil(r / 128), math.ceil(c / 128)
            self.layout[(p, "weight_scale_inv")] = (off, (sr, sc), torch.float32)
            off += (sr * sc * 4 + 15) // 16 * 16
        self.slot_bytes = off
        self.capacity = max(1, int(capacity_bytes) // self.slot_bytes)
        # pinned (page-locked) so that device copies out of it are asynchronous; plain host
        # memory where no GPU is present
        if pinned is None:
            pinned = torch.cuda.device_count() > 0
        self.arena = torch.empty(self.capacity * self.slot_bytes, dtype=torch.uint8, pin_memory=bool(pinned))
        self.lru: OrderedDict = OrderedDict()      # (layer, e) -> slot
        self.free = list(range(self.capacity - 1, -1, -1))
        self.pending: dict[int, object] = {}       # slot -> event after its last device copy
        self.hits = self.misses = 0

    # -------------------------------------------------------------- files

    def _header(self, shard: str) -> tuple[dict, int]:
        if shard not in self._headers:
            self._headers[shard] = read_header(os.path.join(self.path, shard))
        return self._headers[shard]

    def _read_into(self, slot: int, layer: int, e: int) -> None:
        base = slot * self.slot_bytes
        prefix = f"model.layers.{layer}.mlp.experts.{e}"
        by_shard: dict[str, list] = {}
        for p in PROJ:
            for kind in ("weight", "weight_scale_inv"):
                key = f"{prefix}.{p}.{kind}"
                if key not in self.shard_of:
                    raise KeyError(f"ExpertStore: {key} is not in the checkpoint index")
                by_shard.setdefault(self.shard_of[key], []).append((key, p, kind))
        buf = memoryview(self.arena.numpy())
        for shard, items in by_shard.items():
            header, data0 = self._header(shard)
            with open(os.path.join(self.path, shard), "rb", buffering=0) as f:
                for key, p, kind in items:
                    meta = header[key]
                    off, shape, dtype = self.layout[(p, kind)]
                    if _DTYPES.get(meta["dtype"]) != dtype or tuple(meta["shape"]) != shape:
                        raise ValueError(f"ExpertStore: {key} is {meta['dtype']} {meta['shape']}, "
                                         f"expected {dtype} {list(shape)}")
                    b0, b1 = meta["data_offsets"]
                    nbytes = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
                    if b1 - b0 != nbytes:
                        raise ValueError(f"ExpertStore: {key} spans {b1 - b0} bytes in {shard}, its shape "
                                         f"{list(shape)} needs {nbytes}")
                    f.seek(data0 + b0)
                    view = buf[base + off:base + off + nbytes]
                    done = 0
                    while done < nbytes:      # a raw read may return fewer bytes than asked
                        got = f.readinto(view[done:])
                        if not got:
                            raise IOError(f"ExpertStore: {shard} ends inside {key} ({done} of {nbytes} bytes)")
                        done += got

    # -------------------------------------------------------------- slots

    def _views(self, slot: int) -> dict:
        base = slot * self.slot_bytes
        out = {}
        for p in PROJ:
            t = []
            for kind in ("weight", "weight_scale_inv"):
                off, shape, dtype = self.layout[(p, kind)]
                nbytes = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
                t.append(self.arena[base + off:base + off + nbytes].view(dtype).view(shape))
            out[p] = (t[0], t[1])
        return out

    def _take_slot(self) -> int:
        if self.free:
            return self.free.pop()
        key, slot = self.lru.popitem(last=False)
        ev = self.pending.pop(slot, None)
        if ev is not None:
            ev.synchronize()       # the device copies that read this slot have finished
        return slot

    def get_expert(self, layer: int, expert: int) -> dict:
        """weight_store.py:183-206: {proj: (weight, weight_scale_inv)} in pinned host memory."""
        key = (int(layer), int(expert))
        if key in self.lru:
            self.lru.move_to_end(key)
            self.hits += 1
            if self.verbose:
                print(f"        [expert_cache] HIT   L{key[0]:02d}/E{key[1]:03d}")
            return self._views(self.lru[key])
        self.misses += 1
        if self.verbose:
            print(f"        [expert_cache] MISS  L{key[0]:02d}/E{key[1]:03d} "
                  f"({len(self.lru)}/{self.capacity} slots)")
        slot = self._take_slot()
        try:
            self._read_into(slot, *key)
        except Exception:
            self.free.append(slot)
            raise
        self.lru[key] = slot
        return self._views(slot)

    def note_copy(self, layer: int, expert: int, event) -> None:
        """An asynchronous device copy of this expert's slot completes at ``event``: the
        slot is not refilled before it."""
        slot = self.lru.get((int(layer), int(expert)))
        if slot is not None:
            self.pending[slot] = event
