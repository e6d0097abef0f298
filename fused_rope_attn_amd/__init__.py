"""MI355X-native fused 2D-RoPE + varlen attention (drop-in for
sdan/fused-rope-attn's ``fused_attn`` and ``utils`` modules).

The device work runs in ``libfra.so``: hand-written gfx950 HIP kernels
behind the C ABI declared in ``include/fra.h``.
"""
from .fused_attn import (backward_plan, compute_rope_2d, fused_rope_attention, fused_rope_attention_bwd,
                         fused_rope_attention_fwd, fused_rope_attention_pos, next_pow2, plan, plan_pos,
                         rope_positions_2d)
from .utils import get_window_index, window_row_index, window_shuffle, window_unshuffle

__all__ = ["fused_rope_attention", "fused_rope_attention_fwd", "fused_rope_attention_bwd",
           "compute_rope_2d", "next_pow2", "plan", "backward_plan",
           "rope_positions_2d", "fused_rope_attention_pos", "plan_pos",
           "get_window_index", "window_shuffle", "window_unshuffle", "window_row_index"]
__version__ = "0.1.0"
