# SPDX-License-Identifier: Apache-2.0
"""MI355X-native EXL3 (ExLlamaV3 trellis) quantized-linear hot path.

Mirrors the reference package omlx.exl3 (daig/omlx-exl3, src/omlx/exl3): kernels (decode_wt, rot,
norm_rot, swiglu_rot, TrellisGemvPlan), layers (EXL3Linear, EXL3SiblingGroup) and the checkpoint-tensor
loader, on PyTorch-ROCm with hand-written gfx950 HIP kernels behind the C ABI in include/exl3_mi355x.h.
The directory is imported under the module name `omlx_exl3_amd`.
"""
from . import kernels  # noqa: F401
from ._capi import LIB_PATH, Exl3Error  # noqa: F401
from .fusion import fuse_decode  # noqa: F401
from .linear import EXL3Linear, EXL3SiblingGroup, RowExactLinear, unpack_signs  # noqa: F401
from .loader import group_siblings, inventory, is_exl3_config, load_exl3  # noqa: F401

__version__ = "0.1.0"
