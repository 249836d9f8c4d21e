"""The C ABI (include/amla.h) without a GPU: exports, struct layout, host-side argument checks."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from amla import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "amla.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(amla_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    L = _lib.lib()
    names = _declared()
    assert len(names) >= 11
    for n in names:
        assert hasattr(L, n), n
    assert {s[0] for s in _lib.SIGNATURES} == set(names)
    assert L.amla_abi_version() == 104


def test_args_struct_layout_matches_c(tmp_path):
    fields = [f for f, _ in _lib.MlaArgs._fields_]
    src = tmp_path / "layout.c"
    body = "\n".join(f'  printf("{f} %zu\\n", offsetof(amla_mla_args, {f}));' for f in fields)
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "amla.h"\nint main(void){\n'
                   f'  printf("sizeof %zu\\n", sizeof(amla_mla_args));\n{body}\n  return 0;\n}}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines())
    assert int(out["sizeof"]) == ctypes.sizeof(_lib.MlaArgs)
    for f in fields:
        assert int(out[f]) == getattr(_lib.MlaArgs, f).offset, f


def test_null_and_bad_arguments_fail_before_launch():
    L = _lib.lib()
    assert L.amla_fp8_linear(None, 1, 128, 128, None, None, 16, None, 16, None, 0, None) == -1
    assert b"null" in L.amla_last_error()
    assert L.amla_fp8_block_dequant(None, None, 4, 4, None, None) == -1
    assert L.amla_rms_norm(None, 1, 8, 8, None, 1e-6, None, 8, None) == -1
    assert L.amla_apply_rope(None, 1, 1, 64, None, None, None) == -1
    assert L.amla_mla_decode(None, None) == -1
    assert L.amla_mla_prefill(None, None) == -1
    a = _lib.MlaArgs()
    a.batch, a.seq_len, a.hidden, a.heads, a.q_lora = 1, 1, 7168, 64, 1536
    a.kv_lora, a.qk_nope, a.qk_rope, a.v_dim, a.max_seq, a.rope_rows = 512, 128, 64, 128, 16, 16
    assert L.amla_mla_decode(ctypes.byref(a), None) == -3      # unsupported head count
    assert b"heads=128" in L.amla_last_error()
    a.heads = 128
    assert L.amla_mla_decode(ctypes.byref(a), None) == -1      # null pointers
    # a fake non-null workspace that is too small: rejected on the host
    buf = ctypes.create_string_buffer(64)
    p = ctypes.cast(buf, ctypes.c_void_p).value
    for f in ("positions", "hidden_states", "out", "w_q_a", "s_q_a", "w_q_b", "s_q_b", "w_kv_a", "s_kv_a",
              "w_kv_b", "s_kv_b", "w_o", "s_o", "gamma_q", "gamma_kv", "ckv_cache", "kpe_cache", "rope_table",
              "workspace"):
        setattr(a, f, p + 16 - p % 16 if p % 16 else p)
    a.workspace_bytes = 16
    assert L.amla_mla_decode(ctypes.byref(a), None) == -2
    assert b"workspace" in L.amla_last_error()
    # the profiling hook checks its eight events before anything else
    assert L.amla_mla_decode_profiled(ctypes.byref(a), None, None) == -1
    evs = (ctypes.c_void_p * 8)(*([p] * 8))
    evs[3] = None
    assert L.amla_mla_decode_profiled(ctypes.byref(a), None, evs) == -1
    assert b"null event 3" in L.amla_last_error()
    evs[3] = p
    assert L.amla_mla_decode_profiled_repeat(ctypes.byref(a), None, evs, 0) == -1
    assert b"repeat" in L.amla_last_error()
    a.seq_len = 2
    assert L.amla_mla_decode(ctypes.byref(a), None) == -1      # decode needs S == 1
    # fp8_linear shape constraints
    assert L.amla_fp8_linear(p, 1, 100, 100, p, p, 16, p, 16, None, 0, None) == -3
    assert L.amla_fp8_linear(p, 1, 128, 64, p, p, 16, p, 16, None, 0, None) == -1
    # a K that needs partial sums, without workspace: rejected before launch
    assert L.amla_fp8_linear(p, 16, 16384, 16384, p, p, 7168, p, 7168, None, 0, None) == -2
    assert b"workspace" in L.amla_last_error()
    # one row of x takes the streaming GEMV over the whole K, 2-8 rows at the projection shapes
    # the GEMV with x in LDS: no workspace; 9-64 rows the skinny GEMM's K parts
    assert L.amla_fp8_linear_workspace_bytes(1, 7168, 16384) == 0
    assert L.amla_fp8_linear_workspace_bytes(8, 7168, 16384) == 0
    assert L.amla_fp8_linear_workspace_bytes(8, 2112, 7168) == 0
    assert L.amla_fp8_linear_workspace_bytes(16, 7168, 16384) > 0


def test_workspace_queries():
    L = _lib.lib()
    # wo at M=16: K = 16384 is split into parts whose fp32 sums need workspace
    n = L.amla_fp8_linear_workspace_bytes(16, 7168, 16384)
    assert n > 0 and n % (16 * 7168 * 4) == 0
    assert L.amla_fp8_linear_workspace_bytes(8, 24576, 1536) == 0     # one K part
    assert L.amla_fp8_linear_workspace_bytes(4096, 24576, 1536) == 0   # the large-M GEMM needs none
    a = _lib.MlaArgs()
    a.batch, a.seq_len, a.hidden, a.heads, a.q_lora = 8, 1, 7168, 128, 1536
    a.kv_lora, a.qk_nope, a.qk_rope, a.v_dim = 512, 128, 64, 128
    a.max_seq = a.rope_rows = a.max_context = 32768
    n = L.amla_mla_decode_workspace_bytes(ctypes.byref(a))
    assert 32 * 8 * 128 * 512 * 2 <= n < 200 << 20   # bf16 split partials dominate


def test_python_api_rejects_cpu_tensors():
    from amla import ops
    x = torch.zeros(2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.rms_norm(x, torch.ones(128, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        ops.fp8_linear(x, torch.zeros(16, 128).to(torch.float8_e4m3fn), torch.ones(1, 1))


def test_ffn_moe_arguments_fail_before_launch():
    L = _lib.lib()
    buf = ctypes.create_string_buffer(256)
    p0 = ctypes.cast(buf, ctypes.c_void_p).value
    p = p0 + 16 - p0 % 16 if p0 % 16 else p0          # 16-byte aligned host address, never dereferenced
    # swiglu
    assert L.amla_swiglu(None, 1, 256, p, p, p, p, 256, p, p, p, p, 64, None) == -1
    assert L.amla_swiglu(p, 1, 200, p, p, p, p, 256, p, p, p, p, 64, None) == -3     # k % 128
    assert L.amla_swiglu(p, 1, 256, p, p, p, p, 256, p, p, p, p, 16, None) == -2     # workspace too small
    assert b"workspace" in L.amla_last_error()
    assert L.amla_swiglu_workspace_bytes(8, 7168, 2048) >= 8 * 3 * 2048 * 2
    assert L.amla_silu_mul(None, p, 8, p, None) == -1
    assert L.amla_silu_mul(p, p, -1, p, None) == -1
    # route: config constraints
    idx = ctypes.create_string_buffer(8 * 64)
    w = ctypes.create_string_buffer(4 * 64)
    ip, wp = ctypes.addressof(idx), ctypes.addressof(w)
    assert L.amla_moe_route(None, 1, 256, p, 16, 4, 2, 4, 1, ip, wp, p, 1 << 20, None) == -1
    assert L.amla_moe_route(p, 1, 256, p, 18, 4, 2, 4, 1, ip, wp, p, 1 << 20, None) == -1   # 18 % 4 != 0
    assert L.amla_moe_route(p, 1, 256, p, 16, 4, 5, 4, 1, ip, wp, p, 1 << 20, None) == -1   # topk_group > n_group
    assert L.amla_moe_route(p, 1, 256, p, 16, 4, 1, 5, 1, ip, wp, p, 1 << 20, None) == -1   # top_k > 1 group of 4
    assert L.amla_moe_route(p, 1, 100, p, 16, 4, 2, 4, 1, ip, wp, p, 1 << 20, None) == -3   # d % 32
    assert L.amla_moe_route(p, 1, 256, p, 16, 4, 2, 4, 1, ip, wp, p, 8, None) == -2          # workspace
    assert L.amla_moe_route_workspace_bytes(8, 256) >= 8 * 256 * 4
    # combine
    assert L.amla_moe_combine(None, p, p, 1, 8, 256, 2.5, p, None) == -1
    assert L.amla_moe_combine(p, p, p, 1, 0, 256, 2.5, p, None) == -1


def test_moe_experts_checks_indices_and_tables_on_the_host():
    L = _lib.lib()
    buf = ctypes.create_string_buffer(256)
    p0 = ctypes.cast(buf, ctypes.c_void_p).value
    p = p0 + 16 - p0 % 16 if p0 % 16 else p0
    E, m, top_k, d, n = 4, 2, 2, 256, 256
    tables = [(ctypes.c_void_p * E)(*([p] * E)) for _ in range(6)]
    args = lambda idx, ws=1 << 30: (p, m, d, top_k, ctypes.addressof(idx), n, E,
                                    *[ctypes.cast(t, ctypes.c_void_p) for t in tables], p, p, ws, None)
    bad = (ctypes.c_int64 * (m * top_k))(0, 1, 2, 4)          # expert 4 of 4
    assert L.amla_moe_experts(*args(bad)) == -1
    assert b"out of range" in L.amla_last_error()
    ok = (ctypes.c_int64 * (m * top_k))(0, 1, 2, 3)
    tables[4][2] = None                                         # expert 2 has no down weight
    assert L.amla_moe_experts(*args(ok)) == -1
    assert b"expert 2" in L.amla_last_error()
    tables[4][2] = p
    assert L.amla_moe_experts(*args(ok, ws=64)) == -2           # workspace too small
    assert L.amla_moe_experts(p, m, 200, top_k, ctypes.addressof(ok), n, E,
                              *[ctypes.cast(t, ctypes.c_void_p) for t in tables], p, p, 1 << 30, None) == -3
    need = L.amla_moe_experts_workspace_bytes(m, d, top_k, n)
    assert need >= 2 * m * top_k * d * 2


def test_moe_experts_dev_checks_sizes_on_the_host():
    """The device-grouped entry point rejects what its schedule cannot hold before any launch
    (it reads neither the indices nor the weight table on the host)."""
    L = _lib.lib()
    buf = ctypes.create_string_buffer(256)
    p0 = ctypes.cast(buf, ctypes.c_void_p).value
    p = p0 + 16 - p0 % 16 if p0 % 16 else p0
    m, d, top_k, n, E = 8, 256, 8, 256, 256
    need = L.amla_moe_experts_dev_workspace_bytes(m, d, top_k, n, E)
    assert need >= 2 * m * top_k * d * 2 + 3 * m * top_k * n * 2
    assert L.amla_moe_experts_dev_workspace_bytes(m, d, top_k, n, 513) == 0      # more than 512 experts
    assert L.amla_moe_experts_dev_workspace_bytes(8193, d, 8, n, E) == 0          # 65544 slots
    assert L.amla_moe_experts_dev(None, m, d, top_k, p, n, E, p, p, p, need, None) == -1
    assert L.amla_moe_experts_dev(p, m, d, top_k, p, n, 513, p, p, p, need, None) == -3
    assert L.amla_moe_experts_dev(p, 8193, d, 8, p, n, E, p, p, p, need, None) == -3
    assert L.amla_moe_experts_dev(p, m, 200, top_k, p, n, E, p, p, p, need, None) == -3
    assert L.amla_moe_experts_dev(p, m, d, top_k, p, n, E, p, p, p, 64, None) == -2
    assert b"workspace" in L.amla_last_error()
    assert L.amla_moe_experts_dev(p, 0, d, top_k, p, n, E, p, p, p, 0, None) == 0  # nothing to do


def test_sample_checks_sizes_on_the_host():
    """amla_sample: the workspace it asks for (three level histograms per row, chunk maxima and
    kept masses), and the arguments it rejects before any launch."""
    L = _lib.lib()
    # 8 rows of the R1 vocabulary: 64 chunks of 2048 per row (512 workgroups)
    need = L.amla_sample_workspace_bytes(8, 129280)
    assert need == 8 * 64 * 8 + 8 * 3 * 2048 * 8 + 8 * 3 * 32 + 8 * 64 * 16
    assert L.amla_sample_workspace_bytes(1, 129280) >= 3 * 2048 * 8 + 127 * 16     # 127 chunks of 1024
    assert L.amla_sample_workspace_bytes(0, 100) == 0
    assert L.amla_sample_workspace_bytes(4, 0) == 0
    buf = ctypes.create_string_buffer(1024)
    p0 = ctypes.cast(buf, ctypes.c_void_p).value
    p = p0 + 256 - p0 % 256 if p0 % 256 else p0       # 256-byte aligned host address, never dereferenced
    assert L.amla_sample(None, 8, 129280, 129280, 1.0, 0.9, 1, p, p, need, None) == -1
    assert L.amla_sample(p, 8, 129280, 100, 1.0, 0.9, 1, p, p, need, None) == -1          # ld < n
    assert L.amla_sample(p, 8, 129280, 129280, -1.0, 0.9, 1, p, p, need, None) == -1      # temperature < 0
    assert L.amla_sample(p, 8, 129280, 129280, 1.0, float("nan"), 1, p, p, need, None) == -1
    assert L.amla_sample(p, 8, 129280, 129280, 1.0, 0.9, 1, p, p, need - 1, None) == -2
    assert b"workspace" in L.amla_last_error()
    assert L.amla_sample(p, 8, 129280, 129280, 0.0, 0.9, 1, p, None, 0, None) == -2
    assert L.amla_sample(p, 8, 129280, 129280, 1.0, 0.9, 1, p, p + 16, need, None) == -1  # alignment
    assert b"aligned" in L.amla_last_error()
    assert L.amla_sample(p, 0, 129280, 129280, 1.0, 0.9, 1, p, None, 0, None) == 0        # nothing to do
