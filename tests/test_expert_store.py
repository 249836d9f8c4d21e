"""amla.expert_store.ExpertStore (inference/weight_store.py:42-77, :156-206) on a synthetic
checkpoint: the index and shard layout of the R1 release (expert tensors named
model.layers.L.mlp.experts.E.{gate,up,down}_proj.{weight,weight_scale_inv}), tensors
read straight into the pinned arena, LRU by slots, refills ordered after device copies."""
import os
from types import SimpleNamespace

import pytest
import torch
from _ckpt import write_checkpoint
from amla.expert_store import ExpertStore, expert_tensor_keys, read_header

D, I, E, LAYERS = 256, 384, 4, 2
CFG = SimpleNamespace(hidden_size=D, moe_intermediate_size=I)
PROJ = ("gate_proj", "up_proj", "down_proj")


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("ckpt")
    return str(d), write_checkpoint(str(d), D, I, E, LAYERS)


def _same(got, want):
    for p in PROJ:
        assert got[p][0].dtype == torch.float8_e4m3fn and got[p][1].dtype == torch.float32
        assert torch.equal(got[p][0].view(torch.uint8), want[p][0].view(torch.uint8))
        assert torch.equal(got[p][1], want[p][1])


def test_keys_and_header(ckpt):
    d, _ = ckpt
    assert expert_tensor_keys(1, 3)[0] == "model.layers.1.mlp.experts.3.gate_proj.weight"
    header, data0 = read_header(os.path.join(d, "model-00002-of-00002.safetensors"))
    meta = header["model.layers.1.mlp.experts.0.down_proj.weight"]
    assert meta["dtype"] == "F8_E4M3" and meta["shape"] == [D, I] and data0 > 8


def test_contents_bit_exact_and_lru(ckpt):
    d, ref = ckpt
    slot = ExpertStore(d, CFG, capacity_bytes=1).slot_bytes
    st = ExpertStore(d, CFG, capacity_bytes=3 * slot)
    assert st.capacity == 3
    _same(st.get_expert(1, 3), ref[(1, 3)])               # one expert over two shard files
    _same(st.get_expert(0, 0), ref[(0, 0)])
    _same(st.get_expert(0, 1), ref[(0, 1)])
    assert (st.hits, st.misses) == (0, 3)
    _same(st.get_expert(1, 3), ref[(1, 3)])               # hit, now most recent
    assert (st.hits, st.misses) == (1, 3)
    _same(st.get_expert(1, 2), ref[(1, 2)])               # evicts (0, 0), the least recent
    assert (0, 0) not in st.lru and (1, 3) in st.lru
    _same(st.get_expert(0, 0), ref[(0, 0)])               # read again
    assert st.misses == 5


class _Event:
    def __init__(self):
        self.waited = 0

    def synchronize(self):
        self.waited += 1


def test_refill_waits_for_the_copy_of_the_slot(ckpt):
    d, ref = ckpt
    slot = ExpertStore(d, CFG, capacity_bytes=1).slot_bytes
    st = ExpertStore(d, CFG, capacity_bytes=2 * slot)
    st.get_expert(0, 0)
    ev = _Event()
    st.note_copy(0, 0, ev)
    st.get_expert(0, 1)
    assert ev.waited == 0
    st.get_expert(0, 2)                                    # reuses the slot of (0, 0)
    assert ev.waited == 1
    _same(st.get_expert(0, 2), ref[(0, 2)])


def test_errors(ckpt, tmp_path):
    d, _ = ckpt
    st = ExpertStore(d, CFG, capacity_bytes=1 << 20)
    with pytest.raises(KeyError):
        st.get_expert(5, 0)
    wrong = SimpleNamespace(hidden_size=D, moe_intermediate_size=2 * I)
    with pytest.raises(ValueError):
        ExpertStore(d, wrong, capacity_bytes=1 << 24).get_expert(0, 0)


class _ShortReads:
    """A raw file whose reads return at most 1000 bytes (as signals, FUSE or network filesystems may)."""

    def __init__(self, path, mode="r", buffering=-1):
        self.f = open(path, mode, buffering=buffering)
        self.short = buffering == 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.f.close()

    def seek(self, off):
        return self.f.seek(off)

    def read(self, *a):
        return self.f.read(*a)

    def readinto(self, view):
        return self.f.readinto(view[:1000] if self.short else view)


def test_short_raw_reads_are_completed(ckpt, monkeypatch):
    import amla.expert_store as es
    d, ref = ckpt
    monkeypatch.setattr(es, "open", _ShortReads, raising=False)
    st = ExpertStore(d, CFG, capacity_bytes=1 << 24)
    for key in ((0, 1), (1, E - 1)):
        _same(st.get_expert(*key), ref[key])


def test_header_span_must_match_shape(ckpt, tmp_path):
    """A shard header whose byte offsets disagree with the tensor's shape is refused before any
    byte lands in the arena (it would spill into the next tensor's slot)."""
    import json
    import shutil
    import struct
    d, _ = ckpt
    for name in os.listdir(d):
        shutil.copy(os.path.join(d, name), tmp_path / name)
    shard = tmp_path / "model-00001-of-00002.safetensors"
    raw = shard.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    key = "model.layers.0.mlp.experts.0.gate_proj.weight"
    b0, b1 = header[key]["data_offsets"]
    header[key]["data_offsets"] = [b0, b1 - 16]
    text = json.dumps(header, separators=(",", ":")).encode()
    text += b" " * (n - len(text))
    assert len(text) == n
    shard.write_bytes(raw[:8] + text + raw[8 + n:])
    st = ExpertStore(str(tmp_path), CFG, capacity_bytes=1 << 24)
    with pytest.raises(ValueError, match="spans"):
        st.get_expert(0, 0)
    assert st.get_expert(1, 0) is not None        # the failed slot went back to the free list
