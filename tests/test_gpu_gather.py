"""The window shuffle fused into the window kernel's addressing
(fra_fwd_varlen_gather, ``row_index=`` of the op): a window layer on
tensors kept in image order must give, bit for bit, what the reference's
route gives -- window_shuffle the inputs and tables (utils.py:105-126), run
the layer, window_unshuffle the output (utils.py:129-153) -- since every
window computes the same arithmetic on the same values, only fetched from
other rows.  Rows no window slot maps to stay untouched.
"""
import ctypes

import numpy as np
import pytest
import torch

from fused_rope_attn_amd import (_lib, compute_rope_2d, fused_rope_attention, fused_rope_attention_fwd,
                                 fused_rope_attention_pos, get_window_index, rope_positions_2d, window_row_index,
                                 window_shuffle, window_unshuffle)
from fused_rope_attn_amd.configs import WORKLOADS, image_order, make_inputs
from fused_rope_attn_amd.fused_attn import _build_args

pytestmark = pytest.mark.gpu


def _image_case(grids, h, d, seed, device, dtype=torch.bfloat16, rope_dtype=torch.float32, full=False):
    widx, cu = get_window_index(torch.tensor(grids))
    rows = window_row_index(widx).to(device)
    n = int(cu[-1])
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(n, h, d, generator=g).to(dtype).to(device) for _ in range(3))
    cos, sin = compute_rope_2d(grids, d, 2, 10000.0, device, rope_dtype)
    if full:
        cos, sin = torch.cat([cos, cos], 1), torch.cat([sin, sin], 1)
    return widx.to(device), cu.to(device), rows, q, k, v, cos, sin


def _shuffled_route(widx, cu, q, k, v, cos, sin):
    sh = lambda x: window_shuffle(x, widx)  # noqa: E731
    ms = int((cu[1:] - cu[:-1]).max())
    o = fused_rope_attention(sh(q), sh(k), sh(v), sh(cos), sh(sin), cu, ms)
    return window_unshuffle(o, widx)


@pytest.mark.parametrize("d,dtype,rope_dtype,full", [
    (80, torch.bfloat16, torch.float32, False),
    (64, torch.bfloat16, torch.float32, False),
    (72, torch.float16, torch.float32, False),
    (96, torch.bfloat16, torch.bfloat16, False),
    (80, torch.bfloat16, torch.float32, True),
    (80, torch.float16, torch.float16, False),
])
@pytest.mark.parametrize("heads", [None, 2, 4])
def test_gather_equals_shuffle_route(device, d, dtype, rope_dtype, full, heads, monkeypatch):
    # heads: the window kernel's form forced through FRA_WINDOW_HEADS for
    # both routes (None: the planner's choice)
    if heads is not None:
        monkeypatch.setenv("FRA_WINDOW_HEADS", str(heads))
    grids = [(1, 34, 46), (1, 16, 80), (1, 22, 66)]  # ragged edge windows
    widx, cu, rows, q, k, v, cos, sin = _image_case(grids, 6, d, d, device, dtype, rope_dtype, full)
    print(f"gather d={d} {dtype} tables {rope_dtype} full={full} tokens={q.shape[0]}", flush=True)
    ms = int((cu[1:] - cu[:-1]).max())
    got = fused_rope_attention(q, k, v, cos, sin, cu, ms, row_index=rows)
    want = _shuffled_route(widx, cu, q, k, v, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(got, want), float((got.float() - want.float()).abs().max())


def test_gather_positions_equal_shuffle_route(device):
    grids = [(1, 34, 46), (2, 8, 12)]
    widx, cu, rows, q, k, v, _, _ = _image_case(grids, 4, 80, 3, device)
    pos, inv = rope_positions_2d(grids, 80, 2, 10000.0, device)
    ms = int((cu[1:] - cu[:-1]).max())
    got = fused_rope_attention_pos(q, k, v, pos, inv, cu, ms, row_index=rows)
    sh = lambda x: window_shuffle(x, widx)  # noqa: E731
    want = window_unshuffle(fused_rope_attention_pos(sh(q), sh(k), sh(v), sh(pos), inv, cu, ms), widx)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_gather_lse_and_untouched_rows(device):
    """Through the C ABI: the log-sum-exp lands at the tensor rows, and rows
    no window covers (here the last image's windows are left out of
    cu_seqlens) keep their contents."""
    grids = [(1, 16, 16), (1, 8, 8)]
    widx, cu, rows, q, k, v, cos, sin = _image_case(grids, 2, 80, 9, device)
    n_first = 16 * 16
    ncu = int((cu <= n_first).sum())
    cu_part = cu[:ncu].contiguous()  # the first image's windows only
    out = torch.full_like(q, 7.0)
    lse = torch.full((q.shape[1], q.shape[0]), 3.0, dtype=torch.float32, device=device)
    a = _build_args(q, k, v, cos, sin, out, cu_part, 64, 80 ** -0.5)
    a.lse = lse.data_ptr()
    _lib.check(_lib.load().fra_fwd_varlen_gather(ctypes.byref(a), None, rows.data_ptr(),
                                                 torch.cuda.current_stream(device).cuda_stream))
    torch.cuda.synchronize()
    sh = lambda x: window_shuffle(x, widx)  # noqa: E731
    want, want_lse = fused_rope_attention_fwd(sh(q), sh(k), sh(v), sh(cos), sh(sin), cu, 64)
    want = window_unshuffle(want, widx)
    want_lse = window_unshuffle(want_lse.t().contiguous(), widx).t()
    covered = torch.zeros(q.shape[0], dtype=torch.bool, device=device)
    covered[rows[:n_first].long()] = True
    assert torch.equal(out[covered], want[covered])
    assert torch.equal(lse[:, covered], want_lse[:, covered])
    assert bool((out[~covered] == 7.0).all()) and bool((lse[:, ~covered] == 3.0).all())


@pytest.mark.parametrize("name", ["cfg2w", "cfg3"])
def test_gather_baseline_sizes(device, name):
    w = WORKLOADS[name]
    inp = make_inputs(w, seed=31, device=device)
    rows, cos_i, sin_i = image_order(w, device)
    inv = torch.empty_like(rows, dtype=torch.int64)
    inv[rows.long()] = torch.arange(rows.numel(), device=device)
    unsh = lambda x: x[inv]  # noqa: E731  (window order -> image order)
    q, k, v = (unsh(inp[x]) for x in ("q", "k", "v"))
    print(f"gather at {name}: {tuple(q.shape)}", flush=True)
    got = fused_rope_attention(q, k, v, cos_i, sin_i, inp["cu_seqlens"], inp["max_seqlen"], row_index=rows)
    want = fused_rope_attention(inp["q"], inp["k"], inp["v"], inp["cos"], inp["sin"], inp["cu_seqlens"],
                                inp["max_seqlen"])
    torch.cuda.synchronize()
    assert torch.equal(got, unsh(want))


def test_gather_value_errors(device):
    widx, cu, rows, q, k, v, cos, sin = _image_case([(1, 8, 8)], 2, 80, 1, device)
    with pytest.raises(ValueError, match=r"^row_index must be \[total_seq\]"):
        fused_rope_attention(q, k, v, cos, sin, cu, 64, row_index=rows[:-1])
    with pytest.raises(ValueError, match=r"^row_index must have an integer dtype"):
        fused_rope_attention(q, k, v, cos, sin, cu, 64, row_index=rows.float())
    with pytest.raises(ValueError, match=r"^row_index is for window layers"):
        fused_rope_attention(q, k, v, cos, sin, torch.tensor([0, 64], device=device), 64 + 1, row_index=rows)
    with pytest.raises(RuntimeError, match="forward only"):
        fused_rope_attention(q.clone().requires_grad_(True), k, v, cos, sin, cu, 64, row_index=rows)
