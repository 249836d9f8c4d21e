"""amla: MI355X-native absorbed-MLA + block-FP8 linear path for DeepSeek-R1.

Drop-in for the MLA half of the reference's inference/ops.py (same function
names and signatures); every compute call runs hand-written gfx950 HIP kernels
in libamla.so through a C ABI (include/amla.h).
"""
from .config import DeepSeekConfig  # noqa: F401
from . import torch_ops  # noqa: F401  (registers the torch.ops.amla operators)
from .ops import (  # noqa: F401
    apply_rope,
    fp8_block_dequant,
    fp8_linear,
    mla_attention,
    mla_layer,
    precompute_rope_freqs,
    rms_norm,
    softmax_scale,
    yarn_get_mscale,
)
