"""MI355X-native packed varlen causal GQA attention (gfx950 HIP kernels behind a C ABI).

`apply()` installs the attention patch, as the reference's solution.apply() does for
Qwen2Attention (solution/__init__.py:23-33, patch_qwen2_attention at line 25). The other patches
of the reference (MLP, loss, norms, NF4, trainer) are outside this package's scope.
"""

from .attention import (PackedAttention, PackRows, QKVRotate, VarlenAttention, pack_rows,
                        packed_attention, qkv_rotate, varlen_attention)
from .patches import patch_qwen2_attention

__all__ = ["apply", "patch_qwen2_attention", "packed_attention", "varlen_attention",
           "qkv_rotate", "pack_rows", "PackedAttention", "VarlenAttention", "QKVRotate",
           "PackRows"]


def apply():
    patch_qwen2_attention()
