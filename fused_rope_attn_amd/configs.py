"""The workloads the benchmark and the parity tests run, and their
algorithmic cost.

Each workload is a list of image grids plus the encoder settings that turn
them into ``cu_seqlens`` and cos/sin tables with this package's own
``get_window_index`` and ``compute_rope_2d``:

* ``cfg0``  448^2 image, grid 32x32, window layer (16 x 64 tokens), H=16, D=80
* ``cfg1``  896^2 image, grid 64x64, window layer (64 x 64), H=16, D=80
* ``cfg2w`` 1344^2 image, grid 96x96, window layer (144 x 64), H=16, D=80
* ``cfg2f`` the same image, full-attention layer (1 x 9216)
* ``cfg3``  six images with grids 34x46, 22x66, 50x50, 16x80, 72x38 (merge 2)
  and 31x31 (merge 1: an odd grid cannot be merged 2x2), window layer with
  partial edge windows, H=16, D=80
* ``cfg3f`` the same six images as full-attention segments (one per image:
  1564, 1452, 2500, 1280, 2736 and 961 tokens), H=16, D=80
* ``cfg4v`` Qwen3-VL-style video, 8 temporal groups of a 48x48 grid, one
  segment per group (8 x 2304), H=16, D=72
* ``cfg4s`` the same tokens as a single 18432-token segment

Tables are built for the layer kind: window layers use cos/sin reordered by
the window permutation; full layers use the merge-block order.
"""
from dataclasses import dataclass, field

import torch

from .fused_attn import compute_rope_2d
from .utils import get_window_index

__all__ = ["Workload", "WORKLOADS", "make_inputs", "algorithmic_bytes", "algorithmic_flops",
           "algorithmic_bytes_bwd", "algorithmic_flops_bwd", "positions", "image_order"]


@dataclass(frozen=True)
class Workload:
    name: str
    groups: tuple            # ((grid_thw list, spatial_merge_size), ...)
    kind: str                # "window" | "full" | "full_single"
    heads: int = 16
    head_dim: int = 80
    window_size: int = 112
    patch_size: int = 14
    theta: float = 10000.0
    note: str = field(default="", compare=False)


WORKLOADS = {
    "cfg0": Workload("cfg0", ((((1, 32, 32),), 2),), "window", note="448^2 window layer"),
    "cfg1": Workload("cfg1", ((((1, 64, 64),), 2),), "window", note="896^2 window layer"),
    "cfg2w": Workload("cfg2w", ((((1, 96, 96),), 2),), "window", note="1344^2 window layer"),
    "cfg2f": Workload("cfg2f", ((((1, 96, 96),), 2),), "full", note="1344^2 full-attention layer"),
    "cfg3": Workload("cfg3", ((((1, 34, 46), (1, 22, 66), (1, 50, 50), (1, 16, 80), (1, 72, 38)), 2),
                              (((1, 31, 31),), 1)), "window", note="ragged 6-image window layer"),
    "cfg3f": Workload("cfg3f", ((((1, 34, 46), (1, 22, 66), (1, 50, 50), (1, 16, 80), (1, 72, 38)), 2),
                                (((1, 31, 31),), 1)), "full",
                      note="ragged 6-image full-attention layer"),
    "cfg4v": Workload("cfg4v", ((((8, 48, 48),), 2),), "full", head_dim=72, patch_size=16,
                      note="video, 8 x 2304-token segments"),
    "cfg4s": Workload("cfg4s", ((((8, 48, 48),), 2),), "full_single", head_dim=72, patch_size=16,
                      note="video, one 18432-token segment"),
}


def layout(w: Workload, device="cpu", rope_dtype=torch.float32):
    """``(cu_seqlens int32, cos, sin)`` of a workload on ``device``."""
    cus, coss, sins = [], [], []
    offset = 0
    for grids, merge in w.groups:
        grids = [tuple(g) for g in grids]
        if w.kind == "window":
            widx, cu = get_window_index(grids, window_size=w.window_size, spatial_merge_size=merge,
                                        patch_size=w.patch_size, device="cpu")
            cos, sin = compute_rope_2d(grids, w.head_dim, merge, w.theta, "cpu", rope_dtype, window_idx=widx)
        else:
            cos, sin = compute_rope_2d(grids, w.head_dim, merge, w.theta, "cpu", rope_dtype)
            lens = []
            for t, h, ww in grids:
                lens += [h * ww] * t if w.kind == "full" else [t * h * ww]
            cu = torch.zeros(len(lens) + 1, dtype=torch.int64)
            cu[1:] = torch.cumsum(torch.tensor(lens), 0)
        cus.append(cu.to(torch.int64)[(1 if cus else 0):] + offset)
        offset += int(cu[-1])
        coss.append(cos)
        sins.append(sin)
    cu = torch.cat(cus).to(torch.int32)
    return cu.to(device), torch.cat(coss).to(device), torch.cat(sins).to(device)


def positions(w: Workload, device="cpu"):
    """``(pos int32 [N, 2], inv_freq fp32 [head_dim // 4])`` of a workload
    for ``fused_rope_attention_pos``: the (h, w) position of every row of
    ``layout``'s tables, in the same order."""
    from .fused_attn import rope_positions_2d
    poss, inv = [], None
    for grids, merge in w.groups:
        grids = [tuple(g) for g in grids]
        widx = None
        if w.kind == "window":
            widx, _ = get_window_index(grids, window_size=w.window_size, spatial_merge_size=merge,
                                       patch_size=w.patch_size, device="cpu")
        pos, inv = rope_positions_2d(grids, w.head_dim, merge, w.theta, "cpu", window_idx=widx)
        poss.append(pos)
    return torch.cat(poss).to(device), inv.to(device)


def image_order(w: Workload, device="cpu", rope_dtype=torch.float32):
    """``(row_index int32 [N], cos, sin)`` of a window workload kept in image
    order: ``layout``'s tables without the window reorder, and the row of
    every window-order slot (``utils.window_row_index``, offset per image
    group), so that ``x_window = x_image[row_index]`` for every tensor."""
    from .utils import window_row_index
    assert w.kind == "window", w.kind
    rows, coss, sins = [], [], []
    offset = 0
    for grids, merge in w.groups:
        grids = [tuple(g) for g in grids]
        widx, cu = get_window_index(grids, window_size=w.window_size, spatial_merge_size=merge,
                                    patch_size=w.patch_size, device="cpu")
        cos, sin = compute_rope_2d(grids, w.head_dim, merge, w.theta, "cpu", rope_dtype)
        rows.append(window_row_index(widx, spatial_merge_size=merge) + offset)
        offset += int(cu[-1])
        coss.append(cos)
        sins.append(sin)
    return torch.cat(rows).to(device), torch.cat(coss).to(device), torch.cat(sins).to(device)


def make_inputs(w: Workload, seed: int = 0, device="cpu", dtype=torch.bfloat16, rope_dtype=torch.float32,
                heads: "int | None" = None):
    """Seeded synthetic inputs: q, k, v ~ N(0, 1) drawn in fp32 on the CPU
    and cast to ``dtype``; tables and cu_seqlens from ``layout``."""
    cu, cos, sin = layout(w, "cpu", rope_dtype)
    n = int(cu[-1])
    h = w.heads if heads is None else heads
    gen = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(n, h, w.head_dim, generator=gen, dtype=torch.float32) for _ in range(3))
    return {
        "q": q.to(dtype).to(device), "k": k.to(dtype).to(device), "v": v.to(dtype).to(device),
        "cos": cos.to(device), "sin": sin.to(device), "cu_seqlens": cu.to(device),
        "max_seqlen": int((cu[1:] - cu[:-1]).max()),
    }


def algorithmic_bytes(n: int, heads: int, head_dim: int, elem_bytes: int, rope_width: int,
                      rope_bytes: int, nseg: int) -> int:
    """HBM bytes one call must move at least: read Q, K, V and write O once,
    read cos and sin once, read cu_seqlens."""
    return 4 * n * heads * head_dim * elem_bytes + 2 * n * rope_width * rope_bytes + 4 * (nseg + 1)


def algorithmic_flops(heads: int, head_dim: int, seg_lens) -> int:
    """QK^T plus PV flops at the real head_dim, non-causal: 4*D*H*sum(L^2)."""
    return int(4 * head_dim * heads * sum(int(x) * int(x) for x in seg_lens))


def algorithmic_bytes_bwd(n: int, heads: int, head_dim: int, elem_bytes: int, rope_width: int,
                          rope_bytes: int, nseg: int) -> int:
    """HBM bytes one backward call must move at least: read Q, K, V, O and
    dO and write dQ, dK, dV once each, read cos and sin, the forward's
    log-sum-exp ([H, N] fp32) and cu_seqlens."""
    return (8 * n * heads * head_dim * elem_bytes + 2 * n * rope_width * rope_bytes + 4 * n * heads
            + 4 * (nseg + 1))


def algorithmic_flops_bwd(heads: int, head_dim: int, seg_lens) -> int:
    """The backward's five products per (segment, head) at the real head_dim
    -- S = QK^T (recomputed), dP = dO V^T, dV = P^T dO, dQ = dS K,
    dK = dS^T Q -- 2*L*L*D flops each: 10*D*H*sum(L^2)."""
    return int(10 * head_dim * heads * sum(int(x) * int(x) for x in seg_lens))
