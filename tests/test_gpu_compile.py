"""The op as torch.library custom ops (``fused_rope_attn_amd::fwd``,
``::fwd_out``, ``::bwd``): fake implementations and the autograd formula
pass torch's operator checks, and torch.compile traces the drop-in call in
one graph, forward and backward, with the eager results bit for bit."""
import pytest
import torch

from fused_rope_attn_amd import fused_rope_attention
from fused_rope_attn_amd.fused_attn import _fwd_op

pytestmark = pytest.mark.gpu


def _case(device, lens=(64, 64, 17), h=2, d=80, seed=0):
    g = torch.Generator().manual_seed(seed)
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0).tolist()), dtype=torch.int32, device=device)
    n = int(cu[-1])
    q, k, v = (torch.randn(n, h, d, generator=g).to(torch.bfloat16).to(device) for _ in range(3))
    ang = torch.rand(n, d // 2, generator=g) * 6.0
    return q, k, v, ang.cos().to(device), ang.sin().to(device), cu, max(lens)


@pytest.mark.parametrize("lens", [(64, 64, 17), (300, 5)])
def test_opcheck(device, lens):
    q, k, v, cos, sin, cu, ms = _case(device, lens)
    for with_lse in (False, True):
        args = (q, k, v, cos, sin, cu, ms, 80 ** -0.5, with_lse)
        torch.library.opcheck(_fwd_op, args, test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"))
    qg = q.clone().requires_grad_(True)
    torch.library.opcheck(_fwd_op, (qg, k, v, cos, sin, cu, ms, 80 ** -0.5, True),
                          test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


@pytest.mark.parametrize("lens", [(64, 64, 17), (300, 5)])
def test_torch_compile_forward_and_backward(device, lens):
    q, k, v, cos, sin, cu, ms = _case(device, lens, seed=1)

    def layer(q, k, v):
        return fused_rope_attention(q, k, v, cos, sin, cu, ms).float().square().sum()

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    with torch.no_grad():
        assert torch.equal(compiled(q, k, v), layer(q, k, v))
    grads = []
    for fn in (layer, compiled):
        qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
        fn(qg, kg, vg).backward()
        grads.append((qg.grad, kg.grad, vg.grad))
    torch.cuda.synchronize()
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_torch_compile_out_argument(device):
    q, k, v, cos, sin, cu, ms = _case(device, seed=2)
    out = torch.full_like(q, 3.0)

    def layer(q, k, v, out):
        return fused_rope_attention(q, k, v, cos, sin, cu, ms, out=out)

    got = torch.compile(layer, backend="aot_eager", fullgraph=True)(q, k, v, out)
    want = fused_rope_attention(q, k, v, cos, sin, cu, ms)
    torch.cuda.synchronize()
    assert torch.equal(out, want) and torch.equal(got, want)
