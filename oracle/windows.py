"""Qwen2.5-VL window permutation and window cu_seqlens, restated in numpy.

Test infrastructure only (see ``oracle/__init__.py``).

Restates ``get_window_index`` (reference ``utils.py:12-102``):

* ``vit_window = window_size // spatial_merge_size // patch_size``
  (``utils.py:46``), counted in merge units;
* each image's ``(t, h/m, w/m)`` merge grid is padded to a multiple of
  ``vit_window`` with -100 (``:75-80``), cut into windows in row-major
  window order per frame (``:81-84``), and the padding is dropped
  (``:86-88``);
* the window index is offset by the running merge-unit count across images
  (``:90,95``);
* ``cu_seqlens`` is the cumulative window size times ``merge**2``
  (``:92-93``) with repeated entries removed (``:100-102``).

The window (un)shuffle of ``utils.py:105-153`` is a plain gather; the
product's copy (``fused_rope_attn_amd/utils.py``) is checked directly against
the Hugging Face encoder's reorder of its rotary tables
(``tests/test_golden.py``), so the oracle carries none.
"""
import numpy as np


def window_index(grid_thw, window_size: int = 112, spatial_merge_size: int = 2,
                 patch_size: int = 14):
    """Return ``(window_index int64 [N/m^2], cu_seqlens int32)``."""
    m = spatial_merge_size
    vw = window_size // m // patch_size
    if vw <= 0:
        raise ValueError("vit_window must be >= 1")
    mu = m * m
    idx_all, cu = [], [0]
    base = 0
    for t, h, w in grid_thw:
        t, h, w = int(t), int(h), int(w)
        if h % m or w % m:
            raise ValueError(f"h and w must be divisible by spatial_merge_size={m}, got h={h} w={w}")
        gh, gw = h // m, w // m
        nh, nw = -(-gh // vw), -(-gw // vw)
        for f in range(t):
            for wy in range(nh):
                for wx in range(nw):
                    ys = np.arange(wy * vw, min((wy + 1) * vw, gh))
                    xs = np.arange(wx * vw, min((wx + 1) * vw, gw))
                    ids = (f * gh * gw + ys[:, None] * gw + xs[None, :]).reshape(-1)
                    idx_all.append(ids + base)
                    cu.append(cu[-1] + ids.size * mu)
        base += t * gh * gw
    widx = np.concatenate(idx_all).astype(np.int64) if idx_all else np.zeros(0, np.int64)
    cu = np.asarray(cu, dtype=np.int64)
    keep = np.concatenate([[True], cu[1:] != cu[:-1]])
    return widx, cu[keep].astype(np.int32)


def full_cu_seqlens(grid_thw, per_frame: bool = True):
    """cu_seqlens of full-attention layers: one segment per frame (t) of
    each image, as the HF encoder builds them, or one per image."""
    cu = [0]
    for t, h, w in grid_thw:
        t, h, w = int(t), int(h), int(w)
        if per_frame:
            for _ in range(t):
                cu.append(cu[-1] + h * w)
        else:
            cu.append(cu[-1] + t * h * w)
    return np.asarray(cu, dtype=np.int32)

