"""Routed-expert streaming from pinned host memory: the counterpart of
inference/gpu_transfer.py:7-89 (GPUTransfer).

The reference copies the 8 experts of one token into 8 fixed device buffers on
a side stream, then waits for that stream on the host (``transfer_stream.
synchronize()``, gpu_transfer.py:79) before every token's expert compute.
Here the device side is a pool of expert slots kept as stacked tensors
``(slots, rows, cols)`` with an LRU map (layer, expert) -> slot, so experts
that stay hot are not copied again; copies run on a side stream and are ordered
with events only:

* the compute stream waits for a slot's copy (``wait_event``) before the work
  that reads it is enqueued, with no host synchronisation;
* a slot is reused only after an event recorded on the compute stream at
  eviction time, so compute already enqueued that reads the old expert finishes
  before the copy overwrites it.

``prefetch`` starts copies early (for example while the attention of the same
layer runs); ``transfer_experts`` keeps the reference's call and return shape;
``experts_for(layer)`` gives the mapping ``amla.ops.moe_block`` takes, and
``amla.ops.moe_block`` also takes the streamer itself (it then streams the
chosen experts in pool-sized waves, so any batch runs on any pool).

Lifetime of the returned views: the slots handed out by ``transfer_experts`` /
``experts_for`` are held (no ``prefetch`` may evict them) until ``release()`` or
the next ``transfer_experts`` / ``experts_for`` call, which records the
compute-stream event that later copies into those slots wait for.  Enqueue the
work that reads the views before that call.

The host side may be a callable ``(layer, e) -> weights`` (such as the reference's
``weight_store.get_expert``) or an object with ``get_expert`` and optionally
``note_copy(layer, e, event)`` (``amla.expert_store.ExpertStore``), which is told
when the copy out of its pinned slot completes.
"""
from __future__ import annotations

import math
from collections import OrderedDict
from typing import Iterable

import torch

PROJ = ("gate_proj", "up_proj", "down_proj")


class ExpertStreamer:
    """LRU pool of device expert slots filled from pinned host memory.

    host_experts(layer, e) -> {"gate_proj": (w, s), "up_proj": (w, s), "down_proj": (w, s)} with the
    fp8 weights and fp32 scales in host memory (pinned for asynchronous copies, as the reference's
    weight store keeps them, gpu_transfer.py:12).
    """

    def __init__(self, config, host_experts, device, slots: int | None = None, verbose: bool = False):
        self.config = config
        if hasattr(host_experts, "get_expert"):
            self.host_experts = host_experts.get_expert
            self._note_copy = getattr(host_experts, "note_copy", None)
        else:
            self.host_experts = host_experts
            owner = getattr(host_experts, "__self__", None)
            self._note_copy = getattr(owner, "note_copy", None)
        self.device = torch.device(device)
        self.verbose = verbose
        self.slots = int(slots or 4 * config.num_experts_per_tok)
        if self.slots < config.num_experts_per_tok:
            raise ValueError("ExpertStreamer: fewer slots than experts per token")
        h, f = config.hidden_size, config.moe_intermediate_size
        shapes = {"gate_proj": (f, h), "up_proj": (f, h), "down_proj": (h, f)}
        self.w = {p: torch.empty((self.slots, *s), dtype=torch.float8_e4m3fn, device=self.device)
                  for p, s in shapes.items()}
        self.s = {p: torch.empty((self.slots, math.ceil(s[0] / 128), math.ceil(s[1] / 128)), dtype=torch.float32,
                                 device=self.device) for p, s in shapes.items()}
        self.stream = torch.cuda.Stream(device=self.device)          # default priority
        self.lru: OrderedDict = OrderedDict()                           # (layer, e) -> slot
        self.ready: dict[int, torch.cuda.Event] = {}                    # slot -> copy done
        self.free = list(range(self.slots))
        self.held: set = set()                                          # slots handed out, not yet released
        self.copies = 0                                                 # experts copied so far

    # -------------------------------------------------------------- slots

    def _slot_for(self, layer: int, e: int, pinned: set) -> int:
        key = (layer, e)
        if key in self.lru:
            self.lru.move_to_end(key)
            return self.lru[key]
        if self.free:
            slot = self.free.pop()
        else:
            victim = next((k for k in self.lru if self.lru[k] not in pinned and self.lru[k] not in self.held), None)
            if victim is None:
                raise RuntimeError("ExpertStreamer: every slot is in use by this call or held; raise `slots` "
                                   "(amla.ops.moe_block streams larger sets in waves)")
            slot = self.lru.pop(victim)
            # compute already enqueued may still read the old expert
            done = torch.cuda.Event()
            done.record(torch.cuda.current_stream(self.device))
            self.stream.wait_event(done)
        host = self.host_experts(layer, e)
        with torch.cuda.stream(self.stream):
            for p in PROJ:
                hw, hs = host[p]
                self.w[p][slot].copy_(hw, non_blocking=True)
                self.s[p][slot].copy_(hs, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(self.stream)
        self.ready[slot] = ev
        if self._note_copy is not None:
            self._note_copy(layer, e, ev)
        self.lru[key] = slot
        self.copies += 1
        if self.verbose:
            print(f"      [expert_stream] L{layer:02d}: expert {e} -> slot {slot}")
        return slot

    def prefetch(self, layer: int, experts: Iterable[int]) -> list[int]:
        """Start the copies of these experts (no-op for resident ones); returns their slots."""
        ids = [int(e) for e in (experts.tolist() if isinstance(experts, torch.Tensor) else experts)]
        pinned: set = set()
        out = []
        for e in dict.fromkeys(ids):
            slot = self._slot_for(layer, e, pinned)
            pinned.add(slot)
            out.append(slot)
        return out

    def _views(self, slot: int) -> dict:
        return {p: (self.w[p][slot], self.s[p][slot]) for p in PROJ}

    # -------------------------------------------------------------- reference-shaped API

    def release(self) -> None:
        """Ends the hold on the slots handed out so far: work already enqueued on the current
        stream may read them; later copies into them wait for it."""
        if not self.held:
            return
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(self.device))
        self.stream.wait_event(done)
        self.held.clear()

    def transfer_experts(self, layer: int, expert_indices, verbose: bool = False) -> list[dict]:
        """gpu_transfer.py:50-89: the device weights of these experts, in the given order.

        The current stream waits for their copies on the device (no host synchronisation).
        The slots of the previous call are released first; these are held until the next
        call or ``release()``.
        """
        ids = [int(e) for e in (expert_indices.tolist() if isinstance(expert_indices, torch.Tensor)
                                else expert_indices)]
        self.release()
        slots = dict(zip(dict.fromkeys(ids), self.prefetch(layer, ids)))
        cur = torch.cuda.current_stream(self.device)
        for s in set(slots.values()):
            cur.wait_event(self.ready[s])
        self.held.update(slots.values())
        return [self._views(slots[e]) for e in ids]

    def experts_for(self, layer: int, expert_ids) -> dict:
        """{expert: weights} for ``amla.ops.moe_block``, the copies ordered before later work."""
        ids = sorted({int(e) for e in (expert_ids.reshape(-1).tolist() if isinstance(expert_ids, torch.Tensor)
                                       else expert_ids)})
        return dict(zip(ids, self.transfer_experts(layer, ids)))
