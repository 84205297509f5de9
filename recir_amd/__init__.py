"""MI355X-native HSTU jagged attention (forward and backward) behind RecIR's operator surface.

The compute lives in ``librecir_hstu.so`` (hand-written HIP for gfx950, C ABI in
``include/recir_hstu.h``); this package is the thin host side: a ctypes binding, the
``torch.library`` operator with the argument list of ``hammer::triton_ragged_attention_fwd``,
and a keyword front end with the defaults of the packed accelerator kernel it replaces.
"""
from .ops import (  # noqa: F401
    hstu_jagged_attention_fwd,
    hstu_jagged_attention_bwd,
    triton_ragged_attention_fwd,
    jagged_hstu_attention,
    jagged_hstu_attention_backward,
    jagged_hstu_attention_fp8,
    quantize_e4m3_per_head,
    register_swaps,
    plan_cache_scope,
    set_plan_cache,
    set_generic_kernel_policy,
    hstu_attention_matcher,
    attention_via_fp8,
    attention_via_fp8_reference_rule,
    fp8_attention_region,
    KERNEL_AUTO,
    KERNEL_GENERIC,
    KERNEL_MFMA_GENERAL,
    KERNEL_TILED_DIRECT,
)

from .jagged import (  # noqa: F401,E402
    add_ts_pos_emb_fwd,
    concat_2D_jagged_fwd,
    concat_2d_jagged,
    dense_to_jagged,
    jagged_to_padded_dense,
    register_jagged_swaps,
    split_2D_jagged_fwd,
    split_2d_jagged,
)

__all__ = [
    "hstu_jagged_attention_fwd",
    "hstu_jagged_attention_bwd",
    "triton_ragged_attention_fwd",
    "jagged_hstu_attention",
    "jagged_hstu_attention_backward",
    "jagged_hstu_attention_fp8",
    "quantize_e4m3_per_head",
    "register_swaps",
    "plan_cache_scope",
    "set_plan_cache",
    "set_generic_kernel_policy",
    "hstu_attention_matcher",
    "attention_via_fp8",
    "attention_via_fp8_reference_rule",
    "fp8_attention_region",
]
