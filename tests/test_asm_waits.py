"""Every kernel of libamla, compiled for gfx950, uses a loaded register only after the
load has retired (tests/_asm_waits.py models the lgkm / vm counters).

Regression: the decode attention kernel's next-tile preparation once summed the squares
of rows it had read from LDS before the hand-counted wait for those reads (the compiler
had hoisted the plain VALU work above the wait asm), which made a cache row's r_t
depend on LDS timing: about one workgroup in 80 000 produced different partials.
"""
import os
from concurrent.futures import ThreadPoolExecutor

import pytest

from _asm_waits import device_asm, inflight_uses, kernels

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "deepseek-on-one-gpu_amd", "csrc")
INCLUDE = os.path.join(ROOT, "include")
SOURCES = ["mla_decode.hip", "mla_prefill.hip", "fp8_linear.hip", "ffn_moe.hip", "lm_head.hip"]
HIPCC = "/opt/rocm/bin/hipcc"


def test_checker_flags_a_use_before_its_wait():
    ok = ["ds_read_b128 v[10:13], v1 offset:0", "ds_read_b128 v[14:17], v1 offset:16",
          "s_waitcnt lgkmcnt(1)", "v_add_f32_e32 v20, v10, v11", "s_waitcnt lgkmcnt(0)",
          "v_add_f32_e32 v21, v14, v20"]
    assert inflight_uses(ok) == []
    hoisted = ["ds_read_b128 v[10:13], v1 offset:0", "ds_read_b128 v[14:17], v1 offset:16",
               "v_dot2c_f32_bf16_e32 v29, v10, v10", "s_waitcnt lgkmcnt(1)"]
    assert len(inflight_uses(hoisted)) == 1
    # lgkmcnt(1) retires all but the newest LDS operation
    older = ["ds_read_b128 v[10:13], v1", "ds_write_b32 v2, v3", "s_waitcnt lgkmcnt(1)", "v_mov_b32_e32 v5, v12"]
    assert inflight_uses(older) == []
    newest = ["ds_write_b32 v2, v3", "ds_read_b128 v[10:13], v1", "s_waitcnt lgkmcnt(1)", "v_mov_b32_e32 v5, v12"]
    assert len(inflight_uses(newest)) == 1
    # a copy into LDS holds no register
    assert inflight_uses(["global_load_lds_dwordx4 v4, s[2:3]", "v_mov_b32_e32 v4, 0"]) == []
    overwrite = ["global_load_dwordx4 v[40:43], v[2:3], off", "v_mov_b32_e32 v41, 0", "s_waitcnt vmcnt(0)"]
    assert len(inflight_uses(overwrite)) == 1


@pytest.mark.skipif(not os.path.exists(HIPCC),
                    reason="hipcc not available")
def test_no_kernel_uses_a_register_before_its_load_retired():
    with ThreadPoolExecutor(len(SOURCES)) as pool:
        asms = list(pool.map(lambda s: device_asm(os.path.join(CSRC, s), [CSRC, INCLUDE], HIPCC), SOURCES))
    problems, seen = [], 0
    for src, asm in zip(SOURCES, asms):
        for name, instrs in kernels(asm).items():
            seen += 1
            problems += [f"{src} {name[:60]}: {p}" for p in inflight_uses(instrs)[:3]]
    assert seen >= 10, "expected the library's kernels in the assembly"
    assert not problems, "\n".join(problems)
