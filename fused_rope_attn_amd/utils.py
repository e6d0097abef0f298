"""Window index and window (un)shuffle for Qwen2.5-VL-style window attention.

Drop-in for the reference module ``utils.py``:

* ``get_window_index`` -- reference ``utils.py:12-102``: the permutation of
  merge units into window order and the token-space ``cu_seqlens`` of the
  windows, which ``fused_rope_attention`` consumes.
* ``window_shuffle`` / ``window_unshuffle`` -- reference ``utils.py:105-153``.

The reference's ``flash_window_attention`` (``utils.py:156-195``) wraps the
CUDA-only flash-attn package and has no counterpart here; the fused op covers
its use (call it with cos=1, sin=0 tables for attention without rotation).
"""
import torch

__all__ = ["get_window_index", "window_shuffle", "window_unshuffle"]


def get_window_index(grid_thw, *, window_size: int = 112, spatial_merge_size: int = 2,
                     patch_size: int = 14, device=None):
    """Window permutation and window ``cu_seqlens``.

    Each image's ``(t, h/m, w/m)`` grid of merge units is tiled by windows of
    ``vw = window_size // spatial_merge_size // patch_size`` merge units per
    side (partial at the right and bottom edges).  Windows are numbered
    frame by frame, row-major; merge units inside a window row-major.

    Returns ``(window_index, cu_seqlens)``: ``window_index`` (int64, one entry
    per merge unit, offset by the merge units of earlier images) lists merge
    units in window order; ``cu_seqlens`` (int32) holds the cumulative window
    sizes in tokens (merge units times ``spatial_merge_size**2``), starting at
    0, without repeated entries.  Validation and messages follow reference
    utils.py:26-66.
    """
    if isinstance(grid_thw, torch.Tensor):
        if grid_thw.ndim != 2 or grid_thw.shape[-1] != 3:
            raise ValueError(f"grid_thw must be [N,3], got {tuple(grid_thw.shape)}")
        thw = [tuple(int(x) for x in row) for row in grid_thw.tolist()]
        if device is None:
            device = grid_thw.device
    else:
        thw = [(int(t), int(h), int(w)) for (t, h, w) in grid_thw]
        if device is None:
            device = torch.device("cpu")
    if not thw:
        raise ValueError("grid_thw must be non-empty")
    if window_size <= 0:
        raise ValueError(f"window_size must be > 0, got {window_size}")
    if spatial_merge_size <= 0:
        raise ValueError(f"spatial_merge_size must be > 0, got {spatial_merge_size}")
    if patch_size <= 0:
        raise ValueError(f"patch_size must be > 0, got {patch_size}")
    m = spatial_merge_size
    vw = window_size // m // patch_size
    if vw <= 0:
        raise ValueError(
            "vit_window computed as window_size//spatial_merge_size//patch_size must be >= 1, "
            f"got {vw} (window_size={window_size} spatial_merge_size={m} patch_size={patch_size})")

    orders, sizes = [], []
    base = 0
    for t, h, w in thw:
        if t <= 0:
            raise ValueError(f"grid_thw temporal size must be > 0, got t={t}")
        if h <= 0 or w <= 0:
            raise ValueError(f"grid_thw h/w must be > 0, got h={h} w={w}")
        if h % m != 0 or w % m != 0:
            raise ValueError(f"h and w must be divisible by spatial_merge_size={m}, got h={h} w={w}")
        gh, gw = h // m, w // m
        nwh, nww = -(-gh // vw), -(-gw // vw)
        f = torch.arange(t, dtype=torch.int64).view(t, 1, 1)
        y = torch.arange(gh, dtype=torch.int64).view(1, gh, 1)
        x = torch.arange(gw, dtype=torch.int64).view(1, 1, gw)
        win = (f * nwh + y // vw) * nww + x // vw                  # window of each merge unit
        key = win * (vw * vw) + (y % vw) * vw + x % vw              # window order, then row-major inside
        orders.append(torch.argsort(key.reshape(-1)) + base)
        sizes.append(torch.bincount(win.reshape(-1), minlength=t * nwh * nww))
        base += t * gh * gw

    window_index = torch.cat(orders).to(device=device, dtype=torch.long).contiguous()
    lens = torch.cat(sizes) * (m * m)
    lens = lens[lens > 0]
    cu = torch.zeros(lens.numel() + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(lens, 0)
    return window_index, cu.to(device=device, dtype=torch.int32).contiguous()


def _check_merge(x: torch.Tensor, window_index: torch.Tensor, spatial_merge_size: int) -> tuple:
    if x.ndim < 1:
        raise ValueError(f"x must have at least 1 dim, got {tuple(x.shape)}")
    mu = int(spatial_merge_size) ** 2
    if mu <= 0:
        raise ValueError(f"spatial_merge_size must be > 0, got {spatial_merge_size}")
    n = int(x.shape[0])
    if n % mu != 0:
        raise ValueError(f"seq_len must be divisible by merge_unit={mu}, got {n}")
    if window_index.numel() != n // mu:
        raise ValueError(f"window_index length must be {n // mu}, got {window_index.numel()}")
    return n, mu


def window_shuffle(x: torch.Tensor, window_index: torch.Tensor, *, spatial_merge_size: int = 2) -> torch.Tensor:
    """Gather tokens into window order, whole merge units at a time
    (reference utils.py:105-126)."""
    n, mu = _check_merge(x, window_index, spatial_merge_size)
    idx = window_index.to(device=x.device, dtype=torch.long)
    return x.reshape(n // mu, mu, *x.shape[1:]).index_select(0, idx).reshape(x.shape)


def window_unshuffle(x: torch.Tensor, window_index: torch.Tensor, *, spatial_merge_size: int = 2) -> torch.Tensor:
    """Inverse of ``window_shuffle`` (reference utils.py:129-153)."""
    n, mu = _check_merge(x, window_index, spatial_merge_size)
    idx = window_index.to(device=x.device, dtype=torch.long)
    inv = torch.empty_like(idx)
    inv[idx] = torch.arange(idx.numel(), device=idx.device, dtype=idx.dtype)
    return x.reshape(n // mu, mu, *x.shape[1:]).index_select(0, inv).reshape(x.shape)


def window_row_index(window_index: torch.Tensor, *, spatial_merge_size: int = 2) -> torch.Tensor:
    """The token-level gather of ``window_shuffle`` as an int32 index:
    ``window_shuffle(x)[i] == x[row[i]]`` with ``row[i] =
    window_index[i // m^2] * m^2 + i % m^2`` (reference utils.py:105-126).
    Passed as ``row_index`` to ``fused_rope_attention``, it lets a window
    layer run on tensors kept in image order (no shuffle before the encoder
    blocks, no unshuffle after)."""
    mu = int(spatial_merge_size) ** 2
    if mu <= 0:
        raise ValueError(f"spatial_merge_size must be > 0, got {spatial_merge_size}")
    idx = window_index.to(dtype=torch.int64)
    rows = idx[:, None] * mu + torch.arange(mu, device=idx.device, dtype=torch.int64)[None, :]
    return rows.reshape(-1).to(torch.int32)
