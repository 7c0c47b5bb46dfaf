"""MI355X-native FlexAttention with the public API of ``pallas_flexattn``
(``src/pallas_flexattn/__init__.py:3-46`` of the reference), plus the
FlexAttention front door (``flex_attention``, score mods, document masks)."""

from pallas_flexattn.flash_attn import (
    flash_attention,
    flash_attention_fwd,
    flash_attention_bwd,
    mha_reference,
    flex_attention,
    flex_decode,
    flex_attention_varlen,
    varlen_mask,
    flash_attention_bwd_preprocess,
    flash_attention_bwd_dkv,
    flash_attention_bwd_dq,
)
from pallas_flexattn.mask_mod import (
    MaskMod,
    MaskSpec,
    causal_mask,
    bidirectional_mask,
    sliding_window_mask,
    document_mask,
    document_ids_mask,
    and_masks,
)
from pallas_flexattn.score_mod import (
    ScoreSpec,
    alibi_slopes,
    alibi_score_mod,
    softcap_score_mod,
    compose_score_mods,
)
from pallas_flexattn.block_mask import (
    BlockMask,
    create_block_mask,
    create_causal_block_mask,
    create_sliding_window_block_mask,
)
from pallas_flexattn.fp8 import Fp8Tensor, dequantize_fp8, flex_attention_fp8, quantize_fp8
from pallas_flexattn.kernel_tuner import (
    get_optimal_params,
    get_kernel_config,
    print_kernel_config,
    tune,
)

__all__ = [
    "flash_attention",
    "flash_attention_fwd",
    "flash_attention_bwd",
    "mha_reference",
    "MaskMod",
    "causal_mask",
    "bidirectional_mask",
    "sliding_window_mask",
    "BlockMask",
    "create_block_mask",
    "create_causal_block_mask",
    "create_sliding_window_block_mask",
    "get_optimal_params",
    "get_kernel_config",
    "print_kernel_config",
    # MI355X FlexAttention surface
    "flex_attention",
    "flex_decode",
    "flex_attention_varlen",
    "varlen_mask",
    "flex_attention_fp8",
    "quantize_fp8",
    "dequantize_fp8",
    "Fp8Tensor",
    "flash_attention_bwd_preprocess",
    "flash_attention_bwd_dkv",
    "flash_attention_bwd_dq",
    "MaskSpec",
    "document_mask",
    "document_ids_mask",
    "and_masks",
    "ScoreSpec",
    "alibi_slopes",
    "alibi_score_mod",
    "softcap_score_mod",
    "compose_score_mods",
    "tune",
]
