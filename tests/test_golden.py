"""Golden fixtures and third-party cross-checks (CPU).

* ``tests/golden/rope_window_golden.npz`` -- written by
  ``tests/golden/make_golden.py`` from the Hugging Face Qwen2.5-VL vision
  helpers (window index, window cu_seqlens, 2D RoPE tables after the window
  reorder).  The oracle and the product's host helpers
  (``compute_rope_2d``, reference fused_attn.py:33-136; ``get_window_index``,
  reference utils.py:12-102) must reproduce them.
* ``tests/golden/attention_kat.npz`` -- float64 known answers of the fused op
  on tiny ragged inputs, computed from the definition with explicit loops.
* When ``transformers`` is importable the same comparisons also run live on
  the full BASELINE grids (cfg0-cfg4).
"""
import os

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import rope as orope
from oracle import windows as owin
from fused_rope_attn_amd import compute_rope_2d
from fused_rope_attn_amd.utils import get_window_index

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ROPE = np.load(os.path.join(HERE, "rope_window_golden.npz"))
KAT = np.load(os.path.join(HERE, "attention_kat.npz"))
ROPE_SETS = sorted({k.split("/")[0] for k in ROPE.files})
KAT_CASES = sorted({k.split("/")[0] for k in KAT.files})

# fp32 cos/sin of the same fp32 angle from numpy, torch and the HF module can
# differ in the last bit; angles reach ~50 rad, so allow a few ulps of 1.
TABLE_ATOL = 2e-6


def _set(name):
    grids = [tuple(int(x) for x in g) for g in ROPE[f"{name}/grids"]]
    d, m, ws, ps = (int(x) for x in ROPE[f"{name}/params"])
    return grids, d, m, ws, ps


@pytest.mark.parametrize("name", ROPE_SETS)
def test_window_index_matches_hf_golden(name):
    grids, d, m, ws, ps = _set(name)
    want_idx, want_cu = ROPE[f"{name}/window_index"], ROPE[f"{name}/cu_seqlens"]
    idx, cu = owin.window_index(grids, window_size=ws, spatial_merge_size=m, patch_size=ps)
    np.testing.assert_array_equal(idx, want_idx)
    np.testing.assert_array_equal(cu, want_cu)
    pidx, pcu = get_window_index(torch.tensor(grids), window_size=ws, spatial_merge_size=m, patch_size=ps)
    assert pidx.dtype == torch.int64 and pcu.dtype == torch.int32
    np.testing.assert_array_equal(pidx.numpy(), want_idx)
    np.testing.assert_array_equal(pcu.numpy(), want_cu)


@pytest.mark.parametrize("name", ROPE_SETS)
def test_rope_tables_match_hf_golden(name):
    grids, d, m, ws, ps = _set(name)
    widx = ROPE[f"{name}/window_index"]
    rows = ROPE[f"{name}/rows"]
    want_cos, want_sin = ROPE[f"{name}/cos"], ROPE[f"{name}/sin"]
    cos, sin = orope.rope_2d(grids, d, m, window_idx=widx)
    np.testing.assert_allclose(orope.full_width(cos)[rows], want_cos, rtol=0, atol=TABLE_ATOL)
    np.testing.assert_allclose(orope.full_width(sin)[rows], want_sin, rtol=0, atol=TABLE_ATOL)
    pc, ps_ = compute_rope_2d(grids, d, m, 10000.0, "cpu", torch.float32, window_idx=torch.from_numpy(widx))
    assert pc.shape == (cos.shape[0], d // 2)
    np.testing.assert_allclose(torch.cat([pc, pc], 1).numpy()[rows], want_cos, rtol=0, atol=TABLE_ATOL)
    np.testing.assert_allclose(torch.cat([ps_, ps_], 1).numpy()[rows], want_sin, rtol=0, atol=TABLE_ATOL)


@pytest.mark.parametrize("name", KAT_CASES)
def test_oracle_matches_attention_kat(name):
    q, k, v, cos, sin = (KAT[f"{name}/{x}"] for x in ("q", "k", "v", "cos", "sin"))
    cu, scale, want = KAT[f"{name}/cu_seqlens"], float(KAT[f"{name}/scale"][0]), KAT[f"{name}/out"]
    got = oatt.fused_rope_attention(q, k, v, cos, sin, cu, softmax_scale=scale, mode="fp32")
    assert not np.isnan(want).any()
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)


def test_kat_detects_a_planted_sign_error():
    """A rotation with the sign of sin flipped (x0*c + x1*s) is a plausible
    slip; the known answers must reject it."""
    name = "ragged_d80_full"
    q, k, v, cos, sin = (KAT[f"{name}/{x}"] for x in ("q", "k", "v", "cos", "sin"))
    cu, scale, want = KAT[f"{name}/cu_seqlens"], float(KAT[f"{name}/scale"][0]), KAT[f"{name}/out"]
    got = oatt.fused_rope_attention(q, k, v, cos, -sin, cu, softmax_scale=scale, mode="fp32")
    assert np.abs(got - want).max() > 1e-2


# ---- live cross-checks against transformers ------------------------------------

hf = pytest.importorskip("transformers.vision_utils", reason="transformers not installed")


def _hf_window(grids, m, ws, ps):
    idx, cu = hf.get_vision_window_index(torch.tensor(grids), m, ws, ps)
    return idx.numpy(), cu.numpy()


def _hf_tables(grids, d, m, widx):
    from transformers.models.qwen2_5_vl.modeling_qwen2_5_vl import Qwen2_5_VisionRotaryEmbedding
    emb = Qwen2_5_VisionRotaryEmbedding(d // 2)(hf.get_vision_position_ids(torch.tensor(grids), m))
    if widx is not None:
        n = emb.shape[0]
        emb = emb.reshape(n // (m * m), m * m, -1)[torch.from_numpy(widx)].reshape(n, -1)
    return emb.cos().numpy(), emb.sin().numpy()


@pytest.mark.parametrize("wl", ["cfg0", "cfg1", "cfg2w", "cfg3", "cfg3f", "cfg4v"])
def test_workload_layouts_match_transformers(wl):
    from fused_rope_attn_amd.configs import WORKLOADS, layout
    w = WORKLOADS[wl]
    cu_all, cos_all, sin_all = layout(w)
    cus, coss, sins, off = [], [], [], 0
    for grids, m in w.groups:
        grids = [tuple(g) for g in grids]
        if w.kind == "window":
            widx, cu = _hf_window(grids, m, w.window_size, w.patch_size)
            owidx, ocu = owin.window_index(grids, w.window_size, m, w.patch_size)
            np.testing.assert_array_equal(owidx, widx)
            np.testing.assert_array_equal(ocu, cu)
        else:
            widx = None
            cu = owin.full_cu_seqlens(grids, per_frame=True)
        c, s = _hf_tables(grids, w.head_dim, m, widx)
        cus.append(cu[(1 if cus else 0):].astype(np.int64) + off)
        off += int(cu[-1])
        coss.append(c)
        sins.append(s)
    np.testing.assert_array_equal(cu_all.numpy(), np.concatenate(cus))
    np.testing.assert_allclose(cos_all.numpy(), np.concatenate(coss), rtol=0, atol=TABLE_ATOL)
    np.testing.assert_allclose(sin_all.numpy(), np.concatenate(sins), rtol=0, atol=TABLE_ATOL)
