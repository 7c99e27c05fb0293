"""mini_mega_amd: MI355X-native fused FP8xFP8 MoE layer (single GPU).

The compute path is hand-written HIP for gfx950 in csrc/, built into
libmegakernel.so and reached through the C ABI of include/megakernel.h.
"""
from ._lib import LIB_PATH, MegaError, MegaLaunchArgs, MegaLayout, lib, layout  # noqa: F401
from .mega import (  # noqa: F401
    SymmBuffer,
    bf16_fp8_mega_moe,
    bf16_mega_moe,
    fp8_fp4_mega_moe,
    fp8_mega_moe,
    fp8_mega_moe_compute,
    fp8_mega_moe_reduce,
    fold_checkpoint_block_scales,
    get_symm_buffer_for_mega_moe,
    get_symm_buffer_size_for_mega_moe,
    get_token_alignment_for_mega_moe,
    pack_weights,
    pack_weights_from_reference,
    pairing_block,
    transform_weights_for_mega_moe,
    transform_weights_from_reference,
)
