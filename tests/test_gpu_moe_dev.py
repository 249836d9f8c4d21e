"""amla_moe_experts_dev (the routed experts of moe_block grouped on the device) against the
oracle's expert_ffn of every (token, k) slot, and moe_block captured in a HIP graph.

The reference brings the chosen indices to the host before its expert loop
(gpu_transfer.py:60, forward.py:139-151); the device schedule replaces that step, so the
results are checked against the same oracle as amla_moe_experts: per slot,
expert_ffn(hidden[token], experts[index]) (oracle/ref_ffn.py), to the bf16 bar of _tol."""
import pytest
import torch

from oracle import ref_ffn as F
from amla import ops, synth
from _tol import assert_parity
from test_gpu_ffn import _cfg, _dev, _mlp, _x

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SENTINEL = 0x7E11   # bf16 bit pattern of rows the call must not write


def _stacked(table, E):
    return {k: (torch.stack([table[e][k][0] for e in range(E)]).to(DEV),
                torch.stack([table[e][k][1] for e in range(E)]).to(DEV)) for k in ("gate_proj", "up_proj", "down_proj")}


def _run_dev(h, idx, stacked, E, n_inter, null_experts=()):
    """amla_moe_experts_dev through the C-ABI; returns (expert_out, header ints)."""
    m, K = idx.shape
    d = h.shape[1]
    table, _ = ops._stacked_device_table(stacked, E, d, torch.device(DEV))
    if null_experts:
        table = table.clone().view(6, E)
        for e in null_experts:
            table[:, e] = 0
        table = table.view(-1)
    hd = h.to(DEV)
    eout = torch.full((m, K, d), SENTINEL, dtype=torch.int16, device=DEV).view(torch.bfloat16)
    need = ops.lib().amla_moe_experts_dev_workspace_bytes(m, d, K, n_inter, E)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    idx_d = idx.to(torch.int64).contiguous().to(DEV)
    ops.check(ops.lib().amla_moe_experts_dev(hd.data_ptr(), m, d, K, idx_d.data_ptr(), n_inter, E, table.data_ptr(),
                                             eout.data_ptr(), ws.data_ptr(), need, ops._stream_ptr(hd)),
              "moe_experts_dev")
    torch.cuda.synchronize()
    return eout.cpu(), ws[:16].view(torch.int32).cpu().tolist()


def _want(h, idx, table, skip=lambda e: False):
    m, K = idx.shape
    want = torch.empty(m, K, h.shape[1], dtype=torch.bfloat16)
    for e in sorted(set(idx.flatten().tolist())):
        if e < 0 or e not in table or skip(e):
            continue
        sel = (idx == e).nonzero()
        want[sel[:, 0], sel[:, 1]] = F.expert_ffn(h[sel[:, 0]], table[e])
    return want


@pytest.mark.parametrize("E,K,m,dup", [(256, 8, 8, False), (6, 3, 150, False), (16, 8, 200, False),
                                       (2, 1, 300, False), (8, 4, 5, True), (1, 4, 1, True),
                                       (4, 2, 40, False), (12, 3, 60, False)])
def test_moe_experts_dev_vs_expert_ffn(E, K, m, dup):
    """Skinny groups (at most min(m, 64) slots: up to 16 rows in one launch, 17 and more in
    another), GEMM tiles (larger groups) and groups made larger than m by repeated indices."""
    print(f"[case] moe_experts_dev E={E} K={K} m={m} dup={dup}", flush=True)
    d, i = 256, 256
    h = _x((m, d), f"mdev{E}{K}{m}")
    g = torch.Generator().manual_seed(E * 7919 + K * 31 + m)
    if dup:
        idx = torch.randint(0, E, (m, K), generator=g)
    else:
        idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(m)])
    table = {e: _mlp(d, i, f"mdev-expert{e}") for e in range(E)}
    got, hdr = _run_dev(h, idx, _stacked(table, E), E, i)
    assert hdr[0] == m * K and hdr[3] == 0
    counts = torch.bincount(idx.flatten(), minlength=E)
    sb = min(m, 64)
    assert hdr[1] == int(((counts >= 1) & (counts <= sb)).sum())
    assert hdr[2] == int(((counts + 255) // 256 * (counts > sb)).sum())
    assert_parity(got, _want(h, idx, table), f"moe_experts_dev E={E} K={K} m={m}")


def test_moe_experts_dev_skips_and_counts():
    """Negative indices are left out silently; indices >= E and experts with a NULL table entry
    are left out and counted; their rows keep what they held."""
    print("[case] moe_experts_dev skipped slots", flush=True)
    E, K, m, d, i = 12, 4, 40, 256, 256
    h = _x((m, d), "mdev-skip")
    g = torch.Generator().manual_seed(4242)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(m)])
    idx[::7, 0] = -1
    idx[3::11, 1] = E + 2
    null = (5,)
    table = {e: _mlp(d, i, f"mdev-skip{e}") for e in range(E)}
    got, hdr = _run_dev(h, idx, _stacked(table, E), E, i, null_experts=null)
    skipped = (idx >= E) | (idx == 5)
    left = idx < 0
    assert hdr[3] == int(skipped.sum())
    assert hdr[0] == m * K - int(skipped.sum()) - int(left.sum())
    untouched = got.view(torch.int16)[skipped | left]
    assert (untouched == SENTINEL).all()
    keep = ~(skipped | left)
    want = _want(h, idx, table, skip=lambda e: e in null)
    assert_parity(got[keep], want[keep], "moe_experts_dev with skipped slots")


@pytest.mark.parametrize("m", [8, 40])
def test_moe_experts_dev_r1_expert_shape(m):
    """Decode-sized batches at the R1 expert shape (hidden 7168, intermediate 2048): the K-part
    sums of the skinny path at full size, for groups of at most 16 rows (m = 8) and of 17-64
    rows (m = 40: each of the 4 experts gets about 20 rows), the class whose K parts and finish
    are sized from the 64-row bound."""
    print(f"[case] moe_experts_dev R1 shape m={m} K=2 E=4", flush=True)
    E, K, d, i = 4, 2, 7168, 2048
    h = _x((m, d), f"mdev-r1-{m}")
    g = torch.Generator().manual_seed(77 + m)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(m)])
    counts = torch.bincount(idx.flatten(), minlength=E)
    if m > 16:
        assert int(counts.min()) > 16, "every group should take the 17-64 row class"
    table = {e: _mlp(d, i, f"mdev-r1-{e}") for e in range(E)}
    got, hdr = _run_dev(h, idx, _stacked(table, E), E, i)
    assert hdr[0] == m * K and hdr[3] == 0
    assert_parity(got, _want(h, idx, table), f"moe_experts_dev R1 shape m={m}")


def test_moe_block_batch64_r1_shape_device_and_host_grouping_agree():
    """moe_block at batch 64 with R1-shaped experts (16 stacked experts, 8 per token): device
    grouping (groups of 17-64 rows) against host grouping, and the device path's expert
    outputs against the oracle's expert_ffn per slot."""
    print("[case] moe_block batch 64 R1 expert shape, device vs host grouping", flush=True)
    E, K, m, d, i = 16, 8, 64, 7168, 2048
    cfg = _cfg(E, 4, 2, K)
    h = _x((m, 1, d), "mdev-b64")
    gw = synth.randn((E, d), synth.seed_of("mdev-b64-router", E), 0.02).to(torch.bfloat16)
    shared = _mlp(d, i, "mdev-b64-shared")
    table = {e: _mlp(d, i, f"mdev-b64-{e}") for e in range(E)}
    stacked = _stacked(table, E)
    hd, gwd, shd = h.to(DEV), gw.to(DEV), _dev(shared)
    dev_got = ops.moe_block(hd, gwd, shd, stacked, cfg)
    host_got = ops.moe_block(hd, gwd, shd, stacked, cfg, device_grouping=False)
    idx, _ = ops.route(hd, gwd, cfg)
    torch.cuda.synchronize()
    idx = idx.reshape(m, K).cpu()
    counts = torch.bincount(idx.flatten(), minlength=E)
    assert int(counts.max()) > 16, "some group should take the 17-64 row class"
    assert_parity(dev_got, host_got, "moe_block batch 64: device vs host grouping")
    got, hdr = _run_dev(h.reshape(m, d), idx, stacked, E, i)
    assert hdr[0] == m * K and hdr[3] == 0
    assert_parity(got, _want(h.reshape(m, d), idx, table), "moe_experts_dev batch 64 R1 shape")


def test_device_table_not_reused_for_new_tensors_at_the_same_addresses():
    """Two stacked expert sets in a row with the same E but a different intermediate size; the
    first is freed before the second is made, so the allocator may hand out the same base
    addresses: the second call must get its own pointer table (right per-expert steps)."""
    print("[case] stacked device table keyed by shapes", flush=True)
    E, K, m, d = 4, 2, 6, 256
    h = _x((m, d), "mdev-key")
    g = torch.Generator().manual_seed(5)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(m)])
    for i in (256, 512):
        table = {e: _mlp(d, i, f"mdev-key-{i}-{e}") for e in range(E)}
        stacked = _stacked(table, E)
        got, hdr = _run_dev(h, idx, stacked, E, i)
        assert hdr[0] == m * K and hdr[3] == 0
        assert_parity(got, _want(h, idx, table), f"moe_experts_dev n_inter={i}")
        dtab, n_inter = ops._stacked_device_table(stacked, E, d, torch.device(DEV))
        step = stacked["gate_proj"][0][0].numel()
        assert n_inter == i
        assert int(dtab[1]) - int(dtab[0]) == step
        del stacked, table, dtab
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def test_moe_block_device_and_host_grouping_agree_with_the_oracle():
    print("[case] moe_block device vs host grouping", flush=True)
    E, d, i = 64, 256, 256
    cfg = _cfg(E, 8, 4, 6)
    h = _x((4, 3, d), "mdev-block")
    gw = synth.randn((E, d), synth.seed_of("mdev-router", E), 0.1).to(torch.bfloat16)
    shared = _mlp(d, i, "mdev-shared")
    table = {e: _mlp(d, i, f"mdev-b{e}") for e in range(E)}
    stacked = _stacked(table, E)
    dev_got = ops.moe_block(h.to(DEV), gw.to(DEV), _dev(shared), stacked, cfg)
    host_got = ops.moe_block(h.to(DEV), gw.to(DEV), _dev(shared), stacked, cfg, device_grouping=False)
    torch.cuda.synchronize()
    want = F.moe_block(h, gw, shared, lambda e: table[e], cfg)
    assert_parity(dev_got, want, "moe_block device grouping")
    assert_parity(host_got, want, "moe_block host grouping")


def test_moe_block_in_a_hip_graph():
    """route + shared expert + device-grouped experts + combine captured once, replayed on
    new inputs (so the routing changes), with eager work between replays: each replay equals
    the eager call on the same input, and the first also the oracle."""
    print("[case] moe_block graph capture E=32 K=4 B=6", flush=True)
    E, d, i = 32, 256, 256
    cfg = _cfg(E, 4, 2, 4)
    gw = synth.randn((E, d), synth.seed_of("mdev-graph-router", E), 0.1).to(torch.bfloat16)
    shared = _mlp(d, i, "mdev-graph-shared")
    table = {e: _mlp(d, i, f"mdev-g{e}") for e in range(E)}
    stacked = _stacked(table, E)
    gwd, shd = gw.to(DEV), _dev(shared)
    inputs = [_x((6, 1, d), f"mdev-graph-{r}") for r in range(4)]
    static_h = inputs[0].to(DEV)
    ops.moe_block(static_h, gwd, shd, stacked, cfg)            # warm-up: tables, workspaces
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = ops.moe_block(static_h, gwd, shd, stacked, cfg)
    routes = set()
    for r, x in enumerate(inputs):
        static_h.copy_(x.to(DEV))
        eager = ops.moe_block(x.to(DEV), gwd, shd, stacked, cfg)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"replay {r}"
        idx, _ = ops.route(x.to(DEV), gwd, cfg)
        routes.add(tuple(idx.flatten().tolist()))
        if r == 0:
            assert_parity(static_out, F.moe_block(x, gw, shared, lambda e: table[e], cfg), "graph replay vs oracle")
    assert len(routes) > 1, "the inputs should route differently"
