"""The op's argument checks: every ``ValueError`` branch of the reference
wrapper (reference ``fused_attn.py:159-201``) with its message text, the
drop-in contract of ``fused_rope_attention``, plus the checks this build
adds (head_dim above the kernels' limit, tensors on different devices).

Head dims the library has no kernel of its own for must still return the
reference's result (the reference pads any even head_dim to a power of two,
``fused_attn.py:167-168, 215-216``): forward and backward parity at such
head dims, against the fp32 oracle, with the north-star tolerance.
"""
import math
import re

import numpy as np
import pytest
import torch

from fused_rope_attn_amd import fused_rope_attention, fused_rope_attention_bwd, fused_rope_attention_fwd
from oracle import attention as A


def _args(device, n=10, h=2, d=8, dtype=torch.bfloat16, rope=torch.float32):
    q, k, v = (torch.randn(n, h, d, device=device).to(dtype) for _ in range(3))
    cos = torch.ones(n, d // 2, device=device, dtype=rope)
    sin = torch.zeros(n, d // 2, device=device, dtype=rope)
    cu = torch.tensor([0, 4, n], dtype=torch.int32, device=device)
    return q, k, v, cos, sin, cu


def _raises(msg, fn, *a, **kw):
    with pytest.raises(ValueError, match="^" + re.escape(msg) + "$"):
        fn(*a, **kw)


def test_q_must_be_on_cuda():
    # reference fused_attn.py:159-160 (the first check; no GPU needed)
    q, k, v, cos, sin, cu = _args("cpu")
    _raises("q must be on CUDA, got device=cpu", fused_rope_attention, q, k, v, cos, sin, cu)


@pytest.mark.gpu
def test_reference_value_errors(device):
    f = fused_rope_attention
    q, k, v, cos, sin, cu = _args(device)
    # :161-162
    _raises("q/k/v must have same shape, got q=(10, 2, 8) k=(10, 2, 6) v=(10, 2, 8)",
            f, q, k[..., :6].contiguous(), v, cos, sin, cu)
    _raises("q/k/v must have same shape, got q=(10, 2, 8) k=(10, 2, 8) v=(9, 2, 8)", f, q, k, v[:9], cos, sin, cu)
    # :163-164
    _raises("q/k/v must be [total_seq, num_heads, head_dim], got q.ndim=2",
            f, q[:, 0], k[:, 0], v[:, 0], cos, sin, cu)
    # :167-168
    q7 = torch.zeros(10, 2, 7, device=device, dtype=torch.bfloat16)
    _raises("head_dim must be positive and even, got 7", f, q7, q7, q7, cos, sin, cu)
    q0 = torch.zeros(10, 2, 0, device=device, dtype=torch.bfloat16)
    _raises("head_dim must be positive and even, got 0", f, q0, q0, q0, cos, sin, cu)
    # :170-173
    _raises("cos/sin must be [total_seq, head_dim//2]=(10, 4), got cos=(10, 3) sin=(10, 4)",
            f, q, k, v, cos[:, :3], sin, cu)
    _raises("cos/sin must be [total_seq, head_dim//2]=(10, 4), got cos=(10, 4) sin=(9, 4)",
            f, q, k, v, cos, sin[:9], cu)
    # :174-175
    _raises("cu_seqlens must be 1D with length >= 2, got (1,)", f, q, k, v, cos, sin, cu[:1])
    _raises("cu_seqlens must be 1D with length >= 2, got (1, 3)", f, q, k, v, cos, sin, cu[None])
    # :177-178
    qf = q.float()
    _raises("q dtype must be float16 or bfloat16, got torch.float32", f, qf, qf, qf, cos, sin, cu)
    # :179-180
    _raises("q/k/v must share dtype, got q=torch.bfloat16 k=torch.float16 v=torch.bfloat16",
            f, q, k.half(), v, cos, sin, cu)
    _raises("q/k/v must share dtype, got q=torch.bfloat16 k=torch.bfloat16 v=torch.float16",
            f, q, k, v.half(), cos, sin, cu)
    # :182-185
    _raises("cos dtype must be float16, bfloat16 or float32, got torch.float64", f, q, k, v, cos.double(), sin, cu)
    _raises("sin dtype must be float16, bfloat16 or float32, got torch.float64", f, q, k, v, cos, sin.double(), cu)
    # :197-201
    _raises("out must have shape (10, 2, 8), got (10, 2, 6)", f, q, k, v, cos, sin, cu,
            out=torch.empty(10, 2, 6, device=device, dtype=q.dtype))
    _raises(f"out must match q dtype/device, got out=torch.float16/{device} q=torch.bfloat16/{device}",
            f, q, k, v, cos, sin, cu, out=torch.empty(10, 2, 8, device=device, dtype=torch.float16))
    _raises(f"out must match q dtype/device, got out=torch.bfloat16/cpu q=torch.bfloat16/{device}",
            f, q, k, v, cos, sin, cu, out=torch.empty(10, 2, 8, dtype=torch.bfloat16))
    # the same checks guard the forward-with-lse and backward entry points
    _raises("q dtype must be float16 or bfloat16, got torch.float32", fused_rope_attention_fwd,
            qf, qf, qf, cos, sin, cu)


@pytest.mark.gpu
def test_build_specific_value_errors(device):
    f = fused_rope_attention
    q, k, v, cos, sin, cu = _args(device, d=130)
    _raises("head_dim must be <= 128 (the kernels keep a query row's rotated head_dim values in registers), got 130",
            f, q, k, v, cos, sin, cu)
    q, k, v, cos, sin, cu = _args(device)
    _raises(f"k must be on {q.device}, got cpu", f, q, k.cpu(), v, cos, sin, cu)
    _raises(f"sin must be on {q.device}, got cpu", f, q, k, v, cos, sin.cpu(), cu)


@pytest.mark.gpu
def test_valid_inputs_still_run(device):
    # the checks above do not reject the inputs they mutate from
    q, k, v, cos, sin, cu = _args(device)
    out = fused_rope_attention(q, k, v, cos, sin, cu)
    torch.cuda.synchronize()
    assert out.shape == q.shape and torch.isfinite(out.float()).all()


# --- head dims without a kernel of their own -----------------------------------

def _case(lens, h, d, seed, width_full=False):
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n = int(cu[-1]) + 2
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(n, h, d, generator=g).to(torch.bfloat16) for _ in range(4))
    w = d if width_full else d // 2
    ang = torch.rand(n, w, generator=g) * 2 * math.pi - math.pi
    return q, k, v, do, ang.cos(), ang.sin(), torch.from_numpy(cu)


@pytest.mark.gpu
@pytest.mark.parametrize("d", [6, 36, 40, 48, 50, 56, 88, 104, 112, 120, 126])
@pytest.mark.parametrize("lens", [[64, 17, 33], [150, 1, 70]], ids=["window", "long"])
def test_uncompiled_head_dims_match_oracle(device, d, lens):
    q, k, v, do, cos, sin, cu = _case(lens, 2, d, seed=d, width_full=(d % 4 == 2))
    dev = [t.to(device) for t in (q, k, v, cos, sin, cu)]
    qg, kg, vg = (t.clone().requires_grad_(True) for t in dev[:3])
    sentinel = torch.full(q.shape, 7.0, dtype=q.dtype, device=device)
    out_fixed = fused_rope_attention(*dev, max(lens), out=sentinel.clone())
    out = fused_rope_attention(qg, kg, vg, *dev[3:], max(lens))
    out.backward(do.to(device))
    torch.cuda.synchronize()
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    ref = A.fused_rope_attention(qn, kn, vn, cos.numpy(), sin.numpy(), cu.numpy())
    covered = ~np.isnan(ref)
    for got in (out, out_fixed):
        err = np.abs(got.detach().float().cpu().numpy()[covered] - ref[covered])
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, (d, lens, err.max(), err.mean())
    # rows outside every segment keep the caller's values
    tail = out_fixed[int(cu[-1]):].float().cpu()
    assert torch.equal(tail, torch.full_like(tail, 7.0))
    # gradients: the bounds of tests/test_gpu_bwd.py (check_grad)
    from test_gpu_bwd import check_grad
    grads = A.fused_rope_attention_bwd(do.float().numpy(), qn, kn, vn, cos.numpy(), sin.numpy(), cu.numpy())
    for name, got, rg in zip(("dq", "dk", "dv"), (qg.grad, kg.grad, vg.grad), grads):
        check_grad(got.float().cpu().numpy(), rg, f"d={d} lens={lens} {name}")
    # the functional backward agrees with autograd bit for bit
    o2, lse = fused_rope_attention_fwd(*dev, max(lens))
    dq, dk, dv = fused_rope_attention_bwd(do.to(device), *dev[:5], o2, lse, dev[5], max(lens))
    torch.cuda.synchronize()
    assert torch.equal(dq, qg.grad) and torch.equal(dk, kg.grad) and torch.equal(dv, vg.grad)
