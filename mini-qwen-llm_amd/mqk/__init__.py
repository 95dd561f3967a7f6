"""mqk -- MI355X-native fused QKV projection + QK-Norm + RoPE for mini-qwen-llm.

Drop-in for ``mini_qwen.kernels.fused_qkv_rope.fused_qkv_rope`` (same signature,
same output layout) and for the W4A16 attention front, backed by hand-written
gfx950 HIP kernels in ``libmqk.so`` (C ABI: include/mqk.h).
"""
from ._native import (MqkNativeError, decode_recomputes, get_option, library, release_workspaces, set_option,
                      tile_variants, version, workspace_bytes)
from .fused_qkv_rope import (fused_qkv_rope, fused_qkv_rope_ex, fused_qkv_rope_paged, fused_qkv_rope_varlen,
                             qk_norm_rope)
from .quantization import (dequantize, from_autoawq, gptq_zero_fix, pack_int4, per_group_minmax_quantize,
                           unpack_int4)
from .rope import RotaryEmbedding, apply_rotary_emb, rope_tables, rotate_half
from .w4a16 import (LinearW4A16, fused_qkv_rope_w4a16, fused_qkv_rope_w4a16_ex, fused_qkv_rope_w4a16_paged,
                    w4a16_gemm)

__all__ = [
    "MqkNativeError", "library", "set_option", "get_option", "tile_variants", "version", "decode_recomputes",
    "workspace_bytes", "release_workspaces",
    "fused_qkv_rope", "fused_qkv_rope_paged", "fused_qkv_rope_ex", "fused_qkv_rope_varlen", "qk_norm_rope",
    "pack_int4", "unpack_int4", "per_group_minmax_quantize", "dequantize", "gptq_zero_fix", "from_autoawq",
    "RotaryEmbedding", "rope_tables", "rotate_half", "apply_rotary_emb",
    "LinearW4A16", "w4a16_gemm", "fused_qkv_rope_w4a16", "fused_qkv_rope_w4a16_paged", "fused_qkv_rope_w4a16_ex",
]
