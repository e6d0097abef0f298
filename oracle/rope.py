"""2D vision RoPE tables, restated in numpy.

Test infrastructure only (see ``oracle/__init__.py``).

Restates ``compute_rope_2d`` of the reference (``fused_attn.py:33-136``):

* ``rotary_dim = head_dim // 2`` and
  ``inv_freq[j] = 1 / theta ** (2j / rotary_dim)`` for ``j < rotary_dim/2``
  (``fused_attn.py:59,78``);
* per image ``(t, h, w)`` the (h, w) patch coordinates are listed in
  spatial-merge block order -- ``reshape(h/m, m, w/m, m)`` then
  ``permute(0, 2, 1, 3)`` (``fused_attn.py:86-94``) -- and repeated ``t``
  times (``:97-99``);
* ``emb = [h * inv_freq || w * inv_freq]`` (``:109-113``), shape
  ``[N, rotary_dim]``; ``cos = cos(emb)``, ``sin = sin(emb)`` (``:115-116``);
* optional window reorder over merge units (``:124-134``).
"""
import numpy as np

from .numerics import round_to


def inv_freq(head_dim: int, theta: float = 10000.0) -> np.ndarray:
    """``1/theta**(arange(0, D/2, 2)/(D/2))`` in fp32 (fused_attn.py:78)."""
    rd = head_dim // 2
    expo = np.arange(0, rd, 2, dtype=np.float32) / np.float32(rd)
    return (np.float32(1.0) / np.power(np.float32(theta), expo, dtype=np.float32)).astype(np.float32)


def merge_order_positions(t: int, h: int, w: int, merge: int):
    """(h_pos, w_pos) int arrays of one image in merge-block token order.

    Token order is: merge block row ``bh``, merge block column ``bw``, then
    the ``merge x merge`` patches inside the block row-major, repeated ``t``
    times (fused_attn.py:86-99).
    """
    if h % merge or w % merge:
        raise ValueError(f"h={h} and w={w} must be divisible by spatial_merge_size={merge}")
    bh = np.arange(h // merge)[:, None, None, None]
    bw = np.arange(w // merge)[None, :, None, None]
    ih = np.arange(merge)[None, None, :, None]
    iw = np.arange(merge)[None, None, None, :]
    shape = (h // merge, w // merge, merge, merge)
    hp = np.broadcast_to(bh * merge + ih, shape).reshape(-1)
    wp = np.broadcast_to(bw * merge + iw, shape).reshape(-1)
    return np.tile(hp, t), np.tile(wp, t)


def positions(grid_thw, merge: int):
    """Concatenated (h_pos, w_pos) for a list of (t, h, w) grids."""
    hs, ws = [], []
    for t, h, w in grid_thw:
        hp, wp = merge_order_positions(int(t), int(h), int(w), merge)
        hs.append(hp)
        ws.append(wp)
    return np.concatenate(hs), np.concatenate(ws)


def rope_2d(grid_thw, head_dim: int, merge: int, theta: float = 10000.0,
            window_idx=None, dtype: str = "f32"):
    """cos, sin of shape ``[N, head_dim//2]`` as fp32 arrays.

    ``dtype`` rounds the tables the way ``.to(dtype)`` does in the
    reference (fused_attn.py:115-116); values are returned as fp32.
    """
    if head_dim <= 0 or head_dim % 4:
        raise ValueError(f"head_dim must be divisible by 4, got {head_dim}")
    rd = head_dim // 2
    f = inv_freq(head_dim, theta)
    hp, wp = positions(grid_thw, merge)
    fh = hp.astype(np.float32)[:, None] * f[None, :]
    fw = wp.astype(np.float32)[:, None] * f[None, :]
    emb = np.concatenate([fh, fw], axis=-1).astype(np.float32)
    cos = round_to(np.cos(emb).astype(np.float32), dtype)
    sin = round_to(np.sin(emb).astype(np.float32), dtype)
    if window_idx is not None:
        mu = merge * merge
        n = cos.shape[0] // mu
        widx = np.asarray(window_idx, dtype=np.int64)
        cos = cos.reshape(n, mu, rd)[widx].reshape(-1, rd)
        sin = sin.reshape(n, mu, rd)[widx].reshape(-1, rd)
    return np.ascontiguousarray(cos), np.ascontiguousarray(sin)


def full_width(table: np.ndarray) -> np.ndarray:
    """HF layout ``cat(t, t)``: ``[N, D/2] -> [N, D]``.

    HF's vision encoder duplicates the rotary embedding before taking
    cos/sin (transformers ``modeling_qwen2_5_vl.py:445-446``).
    """
    return np.ascontiguousarray(np.concatenate([table, table], axis=-1))
