"""The position variant on the GPU (fra_fwd_varlen_pos through
``fused_rope_attention_pos``): the kernels evaluate cos/sin of
``[h * inv_freq || w * inv_freq]`` in registers instead of reading
``compute_rope_2d``'s table.

Bars: against the fp32 oracle fed the fp32 table of the same positions, the
north-star tolerance (max-abs <= 2e-2, mean-abs <= 2e-3); against the table
entry point on the same GPU, the two may differ only where the device's
sincosf and torch's table differ in the last fp32 bit and that flips the
bf16 rounding of a rotated element (max-abs <= 8e-3, mean-abs <= 1e-4).
"""
import numpy as np
import pytest
import torch

from fused_rope_attn_amd import (compute_rope_2d, fused_rope_attention, fused_rope_attention_pos, plan_pos,
                                 rope_positions_2d)
from fused_rope_attn_amd.configs import WORKLOADS, make_inputs, positions
from fused_rope_attn_amd.utils import get_window_index
from oracle import attention as A

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3
SAME_MAX, SAME_MEAN = 8e-3, 1e-4


def _tables(pos, inv):
    ang = torch.cat([pos[:, 0:1].float() * inv, pos[:, 1:2].float() * inv], dim=1)
    return ang.cos(), ang.sin()


def _case(lens, h, d, seed, dtype=torch.bfloat16, max_pos=100):
    g = torch.Generator().manual_seed(seed)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    n = int(cu[-1])
    q, k, v = (torch.randn(n, h, d, generator=g).to(dtype) for _ in range(3))
    pos = torch.randint(0, max_pos, (n, 2), generator=g, dtype=torch.int32)
    inv = 1.0 / (10000.0 ** (torch.arange(0, d // 2, 2, dtype=torch.float32) / (d // 2)))
    return q, k, v, pos, inv, cu


def _check(lens, h, d, seed, device, dtype=torch.bfloat16, want="window"):
    q, k, v, pos, inv, cu = _case(lens, h, d, seed, dtype)
    print(f"pos case lens={lens} heads={h} head_dim={d} {dtype}", flush=True)
    dq, dk, dv, dpos, dinv, dcu = (t.to(device) for t in (q, k, v, pos, inv, cu))
    ms = max(lens)
    assert plan_pos(dq, dk, dv, dpos, dinv, dcu, ms)["kernel"] == want
    out = fused_rope_attention_pos(dq, dk, dv, dpos, dinv, dcu, ms)
    cos_g, sin_g = _tables(dpos, dinv)
    ref_gpu = fused_rope_attention(dq, dk, dv, cos_g, sin_g, dcu, ms)
    torch.cuda.synchronize()
    o, rg = out.float().cpu().numpy(), ref_gpu.float().cpu().numpy()
    e = np.abs(o - rg)
    assert e.max() <= SAME_MAX and e.mean() <= SAME_MEAN, (lens, d, e.max(), e.mean())
    cos_c, sin_c = _tables(pos, inv)
    ref = A.fused_rope_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), cos_c.numpy(),
                                 sin_c.numpy(), cu.numpy())
    cov = ~np.isnan(ref)
    e = np.abs(o[cov] - ref[cov])
    assert np.isfinite(o[cov]).all()
    assert e.max() <= MAX_ABS and e.mean() <= MEAN_ABS, (lens, d, e.max(), e.mean())


@pytest.mark.parametrize("heads", [None, 2, 4])
@pytest.mark.parametrize("d", [64, 72, 80, 96])
def test_pos_window_kernel(device, d, heads, monkeypatch):
    # heads: the window kernel's form forced through FRA_WINDOW_HEADS (None:
    # the planner's, one head per workgroup for these few pairs)
    if heads is not None:
        monkeypatch.setenv("FRA_WINDOW_HEADS", str(heads))
    _check([64, 64, 17, 0, 33, 64, 5, 64], 4, d, 10 + d, device)


def test_pos_window_kernel_fp16_and_one_head(device):
    _check([64, 40, 64], 3, 80, 3, device, dtype=torch.float16)
    _check([64, 1, 63], 1, 64, 4, device)


@pytest.mark.parametrize("d", [72, 80, 128])
def test_pos_long_kernel(device, d):
    _check([300, 5, 700, 64], 2, d, 20 + d, device, want="long")


def test_pos_real_grid_with_window_order(device):
    # a ragged two-image batch in window order, as the HF encoder feeds it
    grids = [(1, 34, 46), (1, 16, 80)]
    widx, cu = get_window_index(torch.tensor(grids))
    pos, inv = rope_positions_2d(grids, 80, 2, 10000.0, device, window_idx=widx)
    cos, sin = compute_rope_2d(grids, 80, 2, 10000.0, device, torch.float32, window_idx=widx)
    n = pos.shape[0]
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(n, 16, 80, generator=g).to(torch.bfloat16).to(device) for _ in range(3))
    cu = cu.to(device)
    ms = int((cu[1:] - cu[:-1]).max())
    out = fused_rope_attention_pos(q, k, v, pos, inv, cu, ms)
    ref = fused_rope_attention(q, k, v, cos, sin, cu, ms)
    torch.cuda.synchronize()
    e = (out.float() - ref.float()).abs()
    assert float(e.max()) <= SAME_MAX and float(e.mean()) <= SAME_MEAN


@pytest.mark.parametrize("name", ["cfg2w", "cfg2f"])
def test_pos_baseline_sizes_match_tables(device, name):
    w = WORKLOADS[name]
    inp = make_inputs(w, seed=77, device=device)
    pos, inv = positions(w, device)
    cos, sin = _tables(pos, inv)
    # the workload's own tables are these, to the last bit (CPU-built there)
    assert torch.equal(cos.cpu(), inp["cos"].cpu()) or float((cos - inp["cos"]).abs().max()) <= 2e-6
    q, k, v, cu, ms = inp["q"], inp["k"], inp["v"], inp["cu_seqlens"], inp["max_seqlen"]
    print(f"pos at {name}: {tuple(q.shape)}", flush=True)
    out = fused_rope_attention_pos(q, k, v, pos, inv, cu, ms)
    ref = fused_rope_attention(q, k, v, cos, sin, cu, ms)
    torch.cuda.synchronize()
    e = (out.float() - ref.float()).abs()
    assert float(e.max()) <= SAME_MAX and float(e.mean()) <= SAME_MEAN, (float(e.max()), float(e.mean()))


def test_pos_value_errors(device):
    q, k, v, pos, inv, cu = (t.to(device) for t in _case([64, 64], 2, 80, 1))
    with pytest.raises(ValueError, match=r"^pos must be \[total_seq, 2\]"):
        fused_rope_attention_pos(q, k, v, pos[:, :1], inv, cu)
    with pytest.raises(ValueError, match=r"^pos must have an integer dtype"):
        fused_rope_attention_pos(q, k, v, pos.float(), inv, cu)
    with pytest.raises(ValueError, match=r"^inv_freq must be \[head_dim//4\]"):
        fused_rope_attention_pos(q, k, v, pos, inv[:-1], cu)
    with pytest.raises(ValueError, match=r"^inv_freq must be float32"):
        fused_rope_attention_pos(q, k, v, pos, inv.double(), cu)
    with pytest.raises(ValueError, match=r"^head_dim must be positive and divisible by 4"):
        fused_rope_attention_pos(q[..., :78], k[..., :78], v[..., :78], pos, inv, cu)
    with pytest.raises(RuntimeError, match="forward only"):
        fused_rope_attention_pos(q.clone().requires_grad_(True), k, v, pos, inv, cu)
