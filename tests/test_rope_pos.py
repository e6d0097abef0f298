"""The position variant's host side and C ABI without a GPU.

``rope_positions_2d`` must give, for every row, the (h, w) position whose
angles ``[h * inv_freq || w * inv_freq]`` are the row of
``compute_rope_2d``'s table (reference fused_attn.py:78-116), so that the
kernels' in-register cos/sin evaluate exactly the reference's table.  Pinned
against the Hugging Face golden tables (``tests/golden/rope_window_golden.npz``)
and, bit for bit on the CPU, against ``compute_rope_2d``.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from fused_rope_attn_amd import _lib, compute_rope_2d, rope_positions_2d
from fused_rope_attn_amd.utils import get_window_index

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ROPE = np.load(os.path.join(HERE, "rope_window_golden.npz"))
ROPE_SETS = sorted({k.split("/")[0] for k in ROPE.files})
TABLE_ATOL = 2e-6  # fp32 cos/sin of one fp32 angle from two libraries (as test_golden)


def _angles(pos, inv):
    return torch.cat([pos[:, 0:1].float() * inv, pos[:, 1:2].float() * inv], dim=1)


@pytest.mark.parametrize("name", ROPE_SETS)
def test_positions_reproduce_hf_golden_tables(name):
    grids = [tuple(int(x) for x in g) for g in ROPE[f"{name}/grids"]]
    d, m, _, _ = (int(x) for x in ROPE[f"{name}/params"])
    widx = torch.from_numpy(ROPE[f"{name}/window_index"])
    rows = ROPE[f"{name}/rows"]
    pos, inv = rope_positions_2d(grids, d, m, 10000.0, "cpu", window_idx=widx)
    assert pos.dtype == torch.int32 and pos.shape == (int(widx.numel()) * m * m, 2)
    assert inv.dtype == torch.float32 and inv.shape == (d // 4,)
    ang = _angles(pos, inv)
    np.testing.assert_allclose(torch.cat([ang.cos()] * 2, 1).numpy()[rows], ROPE[f"{name}/cos"], rtol=0,
                               atol=TABLE_ATOL)
    np.testing.assert_allclose(torch.cat([ang.sin()] * 2, 1).numpy()[rows], ROPE[f"{name}/sin"], rtol=0,
                               atol=TABLE_ATOL)


@pytest.mark.parametrize("d", [64, 72, 80, 128])
@pytest.mark.parametrize("windowed", [False, True])
def test_positions_equal_compute_rope_2d_bitwise(d, windowed):
    grids = [(1, 34, 46), (2, 8, 12), (1, 16, 80)]
    widx = get_window_index(torch.tensor(grids))[0] if windowed else None
    pos, inv = rope_positions_2d(grids, d, 2, 10000.0, "cpu", window_idx=widx)
    cos, sin = compute_rope_2d(grids, d, 2, 10000.0, "cpu", torch.float32, window_idx=widx)
    ang = _angles(pos, inv)
    assert torch.equal(ang.cos(), cos) and torch.equal(ang.sin(), sin)


def test_positions_reject_bad_head_dim():
    with pytest.raises(AssertionError):
        rope_positions_2d([(1, 4, 4)], 70, 2, 10000.0, "cpu")


# ---- C ABI (no launch: plan queries and calls that fail validation) -------------------

def _args(n=9216, h=16, d=80, nseg=144, max_seqlen=64):
    a = _lib.FwdArgs()
    base = 1 << 20
    a.q, a.k, a.v, a.out = (base * (i + 1) for i in range(4))
    a.cos = a.sin = None
    a.cu_seqlens = base * 8
    a.q_stride_seq = a.k_stride_seq = a.v_stride_seq = a.out_stride_seq = h * d
    a.q_stride_head = a.k_stride_head = a.v_stride_head = a.out_stride_head = d
    a.total_seq, a.num_heads, a.head_dim = n, h, d
    a.num_seqs, a.max_seqlen = nseg, max_seqlen
    a.qkv_dtype, a.rope_dtype = _lib.FRA_DTYPE_BF16, _lib.FRA_DTYPE_F32
    a.rope_width = d // 2
    a.softmax_scale = d ** -0.5
    return a


def _rope():
    return _lib.RopePositions(1 << 24, 1 << 25)


def test_pos_plan_names_and_workspace():
    lib = _lib.load()
    pl = _lib.Plan()
    assert lib.fra_query_plan_pos(_args(), _rope(), pl) == _lib.FRA_OK
    assert pl.kernel == _lib.FRA_KERNEL_WINDOW and pl.name.decode() == "window_d80_bf16_ropepos"
    a = _args(nseg=1, max_seqlen=9216)
    nbytes = ctypes.c_int64(0)
    assert lib.fra_workspace_bytes_pos(a, _rope(), ctypes.byref(nbytes)) == _lib.FRA_OK
    assert nbytes.value >= 9216 * 16 * 80 * 2  # at least the rotated K
    a.workspace, a.workspace_bytes = 1 << 26, nbytes.value
    assert lib.fra_query_plan_pos(a, _rope(), pl) == _lib.FRA_OK
    assert pl.kernel == _lib.FRA_KERNEL_LONG and pl.name.decode() == "long_d80_bf16_ropepos"


def test_pos_long_without_workspace_is_unsupported():
    lib = _lib.load()
    rc = lib.fra_fwd_varlen_pos(_args(nseg=1, max_seqlen=9216), _rope(), None)
    assert rc == _lib.FRA_EUNSUPPORTED and "rotated-K" in _lib.last_error()


def test_pos_validation():
    lib = _lib.load()
    assert lib.fra_fwd_varlen_pos(_args(), None, None) == _lib.FRA_EINVAL
    assert lib.fra_fwd_varlen_pos(_args(), _lib.RopePositions(None, 1 << 25), None) == _lib.FRA_EINVAL
    assert lib.fra_fwd_varlen_pos(_args(d=70), _rope(), None) == _lib.FRA_EINVAL  # head_dim % 4
    assert lib.fra_fwd_varlen_pos(_args(), _lib.RopePositions((1 << 24) + 4, 1 << 25), None) == _lib.FRA_EUNSUPPORTED
    # cos/sin stay NULL for the position variant, but the table entry point needs them
    assert lib.fra_fwd_varlen(_args(), None) == _lib.FRA_EINVAL


def test_gather_plan_and_validation():
    lib = _lib.load()
    a = _args()
    a.cos, a.sin, a.rope_stride_seq = 1 << 24, 1 << 24, 40
    # long segments: no gather variant
    a.max_seqlen, a.num_seqs = 9216, 1
    rc = lib.fra_fwd_varlen_gather(a, None, 1 << 27, None)
    assert rc == _lib.FRA_EUNSUPPORTED and "window layers" in _lib.last_error()
    a.max_seqlen, a.num_seqs = 64, 144
    assert lib.fra_fwd_varlen_gather(a, None, None, None) == _lib.FRA_EINVAL
    assert lib.fra_fwd_varlen_gather(a, None, (1 << 27) + 2, None) == _lib.FRA_EINVAL  # alignment
    a.total_seq = 0  # nothing to launch: a valid plan returns OK without touching the GPU
    assert lib.fra_fwd_varlen_gather(a, None, 1 << 27, None) == _lib.FRA_OK
    assert lib.fra_fwd_varlen_gather(a, _rope(), 1 << 27, None) == _lib.FRA_OK
