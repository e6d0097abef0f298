"""Window (un)shuffle and window-index helpers of the product (CPU).

``fused_rope_attn_amd.utils.window_shuffle`` / ``window_unshuffle`` restate
reference ``utils.py:105-153``; ``get_window_index`` restates
``utils.py:12-102``.  What pins them:

* the Hugging Face Qwen2.5-VL encoder reorders its rotary table by window
  (``emb.reshape(n / mu, mu, -1)[window_index]``); the committed fixture
  ``tests/golden/rope_window_golden.npz`` holds HF's tables after that
  reorder, so shuffling this build's un-reordered tables with HF's window
  index must reproduce them;
* HF undoes the reorder with ``argsort(window_index)``
  (``modeling_qwen2_5_vl.py``, the encoder's ``reverse_indices``), a
  different construction of the inverse than the scatter the reference
  uses, so ``window_unshuffle`` must equal a gather by the argsort;
* round trips in both directions are the identity, for extra trailing dims
  and for every golden window index;
* the reference's ``ValueError`` conditions and messages
  (``utils.py:26-66, 112-123, 138-147``).
"""
import os

import numpy as np
import pytest
import torch

from fused_rope_attn_amd import compute_rope_2d
from fused_rope_attn_amd.utils import get_window_index, window_shuffle, window_unshuffle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ROPE = np.load(os.path.join(HERE, "rope_window_golden.npz"))
ROPE_SETS = sorted({k.split("/")[0] for k in ROPE.files})
TABLE_ATOL = 2e-6


def _set(name):
    grids = [tuple(int(x) for x in g) for g in ROPE[f"{name}/grids"]]
    d, m, ws, ps = (int(x) for x in ROPE[f"{name}/params"])
    return grids, d, m, ws, ps


@pytest.mark.parametrize("name", ROPE_SETS)
def test_shuffle_reorders_tables_like_hf(name):
    grids, d, m, _, _ = _set(name)
    widx = torch.from_numpy(ROPE[f"{name}/window_index"])
    rows = ROPE[f"{name}/rows"]
    cos, sin = compute_rope_2d(grids, d, m, 10000.0, "cpu", torch.float32)  # merge-block order, no reorder
    for tab, want in ((cos, ROPE[f"{name}/cos"]), (sin, ROPE[f"{name}/sin"])):
        got = window_shuffle(torch.cat([tab, tab], 1), widx, spatial_merge_size=m)
        np.testing.assert_allclose(got.numpy()[rows], want, rtol=0, atol=TABLE_ATOL)
        # ... and the unshuffle of HF's reordered rows gives back merge-block order
        back = window_unshuffle(got, widx, spatial_merge_size=m)
        assert torch.equal(back, torch.cat([tab, tab], 1))


def test_shuffle_is_not_the_identity_on_a_real_grid():
    # the golden comparison above would pass trivially for an identity index
    widx = torch.from_numpy(ROPE["cfg0/window_index"])
    assert not torch.equal(widx, torch.arange(widx.numel()))


@pytest.mark.parametrize("name", ROPE_SETS)
def test_unshuffle_is_the_hf_argsort_gather(name):
    _, _, m, _, _ = _set(name)
    widx = torch.from_numpy(ROPE[f"{name}/window_index"])
    mu = m * m
    g = torch.Generator().manual_seed(3)
    x = torch.randn(widx.numel() * mu, 3, 5, generator=g)
    rev = torch.argsort(widx)
    want = x.reshape(widx.numel(), mu, 3, 5)[rev].reshape(x.shape)
    assert torch.equal(window_unshuffle(x, widx, spatial_merge_size=m), want)


@pytest.mark.parametrize("name", ROPE_SETS)
@pytest.mark.parametrize("trailing", [(), (4,), (2, 6)])
def test_round_trips(name, trailing):
    _, _, m, _, _ = _set(name)
    widx = torch.from_numpy(ROPE[f"{name}/window_index"])
    n = widx.numel() * m * m
    x = torch.arange(n * int(np.prod(trailing, dtype=np.int64)), dtype=torch.float64).reshape(n, *trailing)
    s = window_shuffle(x, widx, spatial_merge_size=m)
    assert s.shape == x.shape and s.dtype == x.dtype
    assert torch.equal(window_unshuffle(s, widx, spatial_merge_size=m), x)
    assert torch.equal(window_shuffle(window_unshuffle(x, widx, spatial_merge_size=m), widx,
                                      spatial_merge_size=m), x)
    # whole merge units move together: row i*mu + j comes from unit widx[i]
    mu = m * m
    assert torch.equal(s.reshape(widx.numel(), mu, -1)[:, :, :1].reshape(-1, mu)[:, 0],
                       x.reshape(widx.numel(), mu, -1)[widx][:, 0, 0])


def test_shuffle_identity_index_and_merge_one():
    x = torch.randn(12, 2)
    idx = torch.arange(12)
    assert torch.equal(window_shuffle(x, idx, spatial_merge_size=1), x)
    perm = torch.tensor([2, 0, 1])
    got = window_shuffle(x, perm, spatial_merge_size=2)
    assert torch.equal(got, torch.cat([x[8:12], x[0:4], x[4:8]]))


@pytest.mark.parametrize("fn", [window_shuffle, window_unshuffle])
def test_shuffle_value_errors(fn):
    idx = torch.arange(3)
    with pytest.raises(ValueError, match=r"^x must have at least 1 dim, got \(\)$"):
        fn(torch.tensor(1.0), idx)
    with pytest.raises(ValueError, match=r"^spatial_merge_size must be > 0, got 0$"):
        fn(torch.zeros(12), idx, spatial_merge_size=0)
    with pytest.raises(ValueError, match=r"^seq_len must be divisible by merge_unit=4, got 10$"):
        fn(torch.zeros(10), idx)
    with pytest.raises(ValueError, match=r"^window_index length must be 3, got 4$"):
        fn(torch.zeros(12), torch.arange(4))


def test_get_window_index_value_errors():
    with pytest.raises(ValueError, match=r"^grid_thw must be \[N,3\], got \(3,\)$"):
        get_window_index(torch.tensor([1, 4, 4]))
    with pytest.raises(ValueError, match=r"^grid_thw must be non-empty$"):
        get_window_index([])
    with pytest.raises(ValueError, match=r"^window_size must be > 0, got 0$"):
        get_window_index([(1, 4, 4)], window_size=0)
    with pytest.raises(ValueError, match=r"^spatial_merge_size must be > 0, got -1$"):
        get_window_index([(1, 4, 4)], spatial_merge_size=-1)
    with pytest.raises(ValueError, match=r"^patch_size must be > 0, got 0$"):
        get_window_index([(1, 4, 4)], patch_size=0)
    with pytest.raises(ValueError, match=r"^vit_window computed as window_size//spatial_merge_size//patch_size "
                                         r"must be >= 1, got 0 \(window_size=20 spatial_merge_size=2 "
                                         r"patch_size=14\)$"):
        get_window_index([(1, 4, 4)], window_size=20)
    with pytest.raises(ValueError, match=r"^grid_thw temporal size must be > 0, got t=0$"):
        get_window_index([(0, 4, 4)])
    with pytest.raises(ValueError, match=r"^grid_thw h/w must be > 0, got h=0 w=4$"):
        get_window_index([(1, 0, 4)])
    with pytest.raises(ValueError, match=r"^h and w must be divisible by spatial_merge_size=2, got h=3 w=4$"):
        get_window_index([(1, 3, 4)])


def test_full_cu_seqlens_matches_hf_form():
    """The oracle's per-frame cu_seqlens of full-attention layers equals HF's
    ``repeat_interleave(h * w, t).cumsum()`` padded with a leading 0
    (the encoder's ``cu_seqlens`` construction in ``modeling_qwen2_5_vl.py``)."""
    from oracle import windows as owin
    grids = [(1, 34, 46), (3, 6, 14), (2, 12, 20), (1, 2, 2)]
    thw = torch.tensor(grids)
    want = torch.nn.functional.pad(torch.repeat_interleave(thw[:, 1] * thw[:, 2], thw[:, 0]).cumsum(0), (1, 0))
    np.testing.assert_array_equal(owin.full_cu_seqlens(grids, per_frame=True), want.numpy())
    assert owin.full_cu_seqlens(grids, per_frame=False)[-1] == int((thw[:, 0] * thw[:, 1] * thw[:, 2]).sum())


# ---- window_row_index: window_shuffle's gather as a row index --------------------------

@pytest.mark.parametrize("name", ROPE_SETS)
def test_window_row_index_is_the_shuffle_gather(name):
    from fused_rope_attn_amd.utils import window_row_index
    grids = [tuple(int(x) for x in g) for g in ROPE[f"{name}/grids"]]
    _, m, _, _ = (int(x) for x in ROPE[f"{name}/params"])
    widx = torch.from_numpy(ROPE[f"{name}/window_index"])
    rows = window_row_index(widx, spatial_merge_size=m)
    n = int(widx.numel()) * m * m
    assert rows.dtype == torch.int32 and rows.shape == (n,)
    assert torch.equal(torch.sort(rows.long()).values, torch.arange(n))  # a permutation
    x = torch.randn(n, 3)
    assert torch.equal(x[rows.long()], window_shuffle(x, widx, spatial_merge_size=m))
    assert torch.equal(window_unshuffle(x[rows.long()], widx, spatial_merge_size=m), x)


def test_window_row_index_value_error():
    from fused_rope_attn_amd.utils import window_row_index
    with pytest.raises(ValueError, match=r"^spatial_merge_size must be > 0, got 0$"):
        window_row_index(torch.arange(4), spatial_merge_size=0)
