#!/usr/bin/env python3
"""Writes the golden fixtures of this directory.

Run in a container that has ``transformers`` (any 5.x; 5.15.0 wrote the
committed files): ``python tests/golden/make_golden.py``.

The reference ships no tests or vectors, so the fixtures come from two
sources independent of this build's code:

* ``rope_window_golden.npz`` -- the Hugging Face Qwen2.5-VL vision helpers
  that the reference's ``compute_rope_2d`` (fused_attn.py:33-136) and
  ``get_window_index`` (utils.py:12-102) restate:
  ``transformers.vision_utils.get_vision_position_ids``,
  ``Qwen2_5_VisionRotaryEmbedding`` and
  ``transformers.vision_utils.get_vision_window_index``, combined the way
  ``Qwen2_5_VisionTransformerPretrainedModel.forward`` combines them (window
  reorder of the merge units, then ``cat(emb, emb)``).  Per grid set it holds
  the window index, the window cu_seqlens and the cos/sin tables (every
  ``ROW_STEP``-th row, to keep the file small).
* ``attention_kat.npz`` -- known-answer vectors of the fused op on tiny
  ragged inputs, computed here in float64 with explicit loops from the
  definition (rotate each pair, dot products, softmax, weighted sum of V).
  Inputs are bf16-representable so the GPU test feeds them unchanged.
"""
import math
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROW_STEP = 7

# (name, grid list, head_dim, spatial_merge_size, window_size, patch_size)
GRID_SETS = [
    ("cfg0", [(1, 32, 32)], 80, 2, 112, 14),
    ("ragged", [(1, 34, 46), (1, 22, 66), (1, 16, 80)], 80, 2, 112, 14),
    ("video_t2", [(2, 12, 20)], 80, 2, 112, 14),
    ("odd_edges", [(1, 10, 6), (1, 2, 2), (3, 6, 14)], 72, 2, 112, 14),
    ("patch16_d72", [(1, 48, 48)], 72, 2, 128, 16),
]


def hf_tables(grids, head_dim, merge, window_size, patch_size):
    from transformers.vision_utils import get_vision_position_ids, get_vision_window_index
    from transformers.models.qwen2_5_vl.modeling_qwen2_5_vl import Qwen2_5_VisionRotaryEmbedding

    thw = torch.tensor(grids, dtype=torch.int64)
    widx, cu = get_vision_window_index(thw, merge, window_size, patch_size)
    pos = get_vision_position_ids(thw, merge)
    rot = Qwen2_5_VisionRotaryEmbedding(head_dim // 2)
    emb = rot(pos)                                   # [N, head_dim/2]
    n = emb.shape[0]
    mu = merge * merge
    emb = emb.reshape(n // mu, mu, -1)[widx].reshape(n, -1)
    full = torch.cat((emb, emb), dim=-1)             # HF's [N, head_dim] layout
    return widx.numpy().astype(np.int64), cu.numpy().astype(np.int32), full.cos().numpy(), full.sin().numpy()


def bf16_round(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def kat_case(rng, cu, heads, d, width_full, scale):
    n = int(cu[-1])
    q = bf16_round(rng.standard_normal((n, heads, d)))
    k = bf16_round(rng.standard_normal((n, heads, d)))
    v = bf16_round(rng.standard_normal((n, heads, d)))
    w = d if width_full else d // 2
    ang = rng.uniform(-math.pi, math.pi, size=(n, w))
    cos = np.cos(ang).astype(np.float32)
    sin = np.sin(ang).astype(np.float32)
    half = d // 2
    out = np.full((n, heads, d), np.nan)
    for a, b in zip(cu[:-1], cu[1:]):
        for h in range(heads):
            rq = np.zeros((b - a, d))
            rk = np.zeros((b - a, d))
            for t in range(a, b):
                for i in range(half):
                    c0, s0 = float(cos[t, i]), float(sin[t, i])
                    c1, s1 = (float(cos[t, half + i]), float(sin[t, half + i])) if width_full else (c0, s0)
                    for src, dst in ((q, rq), (k, rk)):
                        x0, x1 = float(src[t, h, i]), float(src[t, h, half + i])
                        dst[t - a, i] = x0 * c0 - x1 * s0
                        dst[t - a, half + i] = x0 * s1 + x1 * c1
            for t in range(b - a):
                logits = [scale * sum(rq[t, j] * rk[u, j] for j in range(d)) for u in range(b - a)]
                m = max(logits)
                e = [math.exp(x - m) for x in logits]
                z = sum(e)
                for j in range(d):
                    out[a + t, h, j] = sum(e[u] * float(v[a + u, h, j]) for u in range(b - a)) / z
    return q, k, v, cos, sin, out


def main():
    tables = {}
    for name, grids, d, m, ws, ps in GRID_SETS:
        widx, cu, cos, sin = hf_tables(grids, d, m, ws, ps)
        rows = np.arange(0, cos.shape[0], ROW_STEP)
        tables[f"{name}/grids"] = np.asarray(grids, dtype=np.int64)
        tables[f"{name}/params"] = np.asarray([d, m, ws, ps], dtype=np.int64)
        tables[f"{name}/window_index"] = widx
        tables[f"{name}/cu_seqlens"] = cu
        tables[f"{name}/rows"] = rows.astype(np.int64)
        tables[f"{name}/cos"] = cos[rows].astype(np.float32)
        tables[f"{name}/sin"] = sin[rows].astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "rope_window_golden.npz"), **tables)

    rng = np.random.default_rng(20261201)
    kat = {}
    cases = [  # (name, cu_seqlens, heads, head_dim, full-width tables, scale)
        ("ragged_d64_half", [0, 5, 5, 13, 14, 30], 2, 64, False, 64 ** -0.5),
        ("ragged_d80_full", [0, 9, 20], 3, 80, True, 80 ** -0.5),
        ("window_d72_scale", [0, 3, 11, 64], 1, 72, False, 0.2),
        ("long_d80", [0, 70, 71], 1, 80, False, 80 ** -0.5),
    ]
    for name, cu, heads, d, full, scale in cases:
        q, k, v, cos, sin, out = kat_case(rng, cu, heads, d, full, scale)
        for key, val in (("q", q), ("k", k), ("v", v), ("cos", cos), ("sin", sin), ("out", out)):
            kat[f"{name}/{key}"] = val.astype(np.float64 if key == "out" else np.float32)
        kat[f"{name}/cu_seqlens"] = np.asarray(cu, dtype=np.int32)
        kat[f"{name}/scale"] = np.asarray([scale], dtype=np.float64)
    np.savez_compressed(os.path.join(HERE, "attention_kat.npz"), **kat)
    print("wrote", sorted({k.split("/")[0] for k in tables}), sorted({k.split("/")[0] for k in kat}))


if __name__ == "__main__":
    main()
