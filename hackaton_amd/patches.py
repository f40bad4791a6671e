"""The Qwen2 attention patch: transformers' Qwen2Attention.forward with the rotation and the
attention of the packed rows done by the gfx950 kernels (solution/patches.py:81-113).

Calls that carry `packed=(b_idx, t_idx, batch, seq, lengths)` (a padding-free training step, as
built by solution/packed.py:153-176) take the packed path: the q/k/v projections, then
`packed_attention` when the rows are right padded (`lengths` is a list), otherwise the padded
layout with the caller's mask through `qkv_rotate(padded=True)`, SDPA and `pack_rows`. Every
other call runs the original forward unchanged.
"""

import torch

from .attention import pack_rows, packed_attention, qkv_rotate

_ORIGINAL = {}


def patch_qwen2_attention():
    from transformers.models.qwen2 import modeling_qwen2

    cls = modeling_qwen2.Qwen2Attention
    if "forward" not in _ORIGINAL:
        _ORIGINAL["forward"] = cls.forward
    original = _ORIGINAL["forward"]

    def forward(self, hidden_states, position_embeddings, attention_mask, past_key_values=None,
                **kwargs):
        packed = kwargs.pop("packed", None)
        if packed is None:  # an ordinary call (generation, eval, padded batches): unchanged
            return original(self, hidden_states, position_embeddings, attention_mask,
                            past_key_values, **kwargs)
        b_idx, t_idx, batch, seq, lengths = packed
        cos, sin = position_embeddings
        config = self.config
        q, k, v = (self.q_proj(hidden_states), self.k_proj(hidden_states),
                   self.v_proj(hidden_states))
        if lengths is not None:  # documents are contiguous row blocks: attend on the rows
            attn = packed_attention(q, k, v, cos, sin, b_idx, t_idx, seq,
                                    config.num_attention_heads, config.num_key_value_heads,
                                    lengths, self.scaling)
            return self.o_proj(attn), None
        # lengths unknown (e.g. left padding): rebuild the padded batch, use the caller's mask
        query, key, value = qkv_rotate(q, k, v, cos, sin, b_idx, t_idx, batch, seq,
                                       config.num_attention_heads, config.num_key_value_heads,
                                       True)
        attn = torch.nn.functional.scaled_dot_product_attention(
            query, key, value, attn_mask=attention_mask, dropout_p=0.0, scale=self.scaling)
        return self.o_proj(pack_rows(attn, b_idx, t_idx)), None

    cls.forward = forward


def unpatch_qwen2_attention():
    """Restore transformers' forward (tests)."""
    from transformers.models.qwen2 import modeling_qwen2

    if "forward" in _ORIGINAL:
        modeling_qwen2.Qwen2Attention.forward = _ORIGINAL["forward"]
