"""Parity of the log-sum-exp output and the backward (libfra.so through
``fused_rope_attention_fwd`` / ``fused_rope_attention_bwd`` and autograd)
with the CPU oracle on the same seeded inputs.

The reference is forward-only, so the oracle's gradients (pinned against
torch autograd in float64 and finite differences in ``test_oracle.py``)
are the target.  Tolerances, all against the fp32 oracle:

* lse (natural log, values ~5-8): max-abs <= 1e-2, mean-abs <= 1e-3.  The
  bf16 rounding of q_rot / k_rot alone moves it by up to 1.6e-3 (mean 4e-4)
  in the rounding-point model (oracle mode "bf16").
* dq, dk, dv in bf16 (magnitudes <= ~1.5 at head_dim 80, growing with
  head_dim): max-abs <= max(2e-2, 1e-2 x max |ref|) -- the forward's
  north-star bound, or the rounding-point model's own worst case below
  (storing a value x in bf16 alone errs by up to x * 2^-9; at head_dim 126
  the largest dk is ~4.4 and errs by ~0.73% of it) -- and mean-abs <= 2e-3
  and <= 1e-2 x mean |ref|.
  The rounding-point model of the kernels (q_rot/k_rot, P, dZ and the
  results rounded to bf16) sits at 3-4e-3 x mean |ref| and <= 1e-2 x max |ref|.

At full sizes, size-independent identities of the gradient cover what the
oracle cannot: per (segment, head), sum over keys of dv = sum over queries of
dout (rows of P sum to 1), and with cos = 1, sin = 0, sum over keys of dk = 0
(rows of dZ sum to 0).
"""
import math

import numpy as np
import pytest
import torch

from fused_rope_attn_amd import backward_plan, fused_rope_attention, fused_rope_attention_bwd, fused_rope_attention_fwd
from oracle import attention as A

pytestmark = pytest.mark.gpu

LSE_MAX, LSE_MEAN = 1e-2, 1e-3
G_MAX, G_MEAN, G_REL_MEAN, G_REL_MAX = 2e-2, 2e-3, 1e-2, 1e-2


def f32(t):
    return t.detach().float().cpu().numpy()


def make_case(lens, h, d, seed, dtype=torch.bfloat16, width=None, lead_rows=0, extra_rows=0):
    """Segments of the given lengths (0 allowed) starting at row lead_rows,
    with extra_rows rows after the last segment; random angles per token."""
    cu = (lead_rows + np.concatenate([[0], np.cumsum(lens)])).astype(np.int32)
    n = int(cu[-1]) + extra_rows
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(n, h, d, generator=g) for _ in range(4))
    w = d // 2 if width is None else width
    ang = torch.rand(n, w, generator=g) * 2 * math.pi - math.pi
    return {"q": q.to(dtype), "k": k.to(dtype), "v": v.to(dtype), "dout": do.to(dtype),
            "cos": ang.cos(), "sin": ang.sin(), "cu": torch.from_numpy(cu), "max_seqlen": int(max(lens))}


def on(case, device):
    return {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in case.items()}


def gpu_fwd_bwd(c):
    out, lse = fused_rope_attention_fwd(c["q"], c["k"], c["v"], c["cos"], c["sin"], c["cu"], c["max_seqlen"])
    dq, dk, dv = fused_rope_attention_bwd(c["dout"], c["q"], c["k"], c["v"], c["cos"], c["sin"], out, lse, c["cu"],
                                          c["max_seqlen"])
    torch.cuda.synchronize()
    return out, lse, dq, dk, dv


def check_grad(got, ref, what):
    covered = ~np.isnan(ref)
    assert covered.any()
    err = np.abs(got[covered] - ref[covered])
    assert np.isfinite(got[covered]).all(), f"{what}: non-finite gradient"
    mx, mn, rm = float(err.max()), float(err.mean()), float(np.abs(ref[covered]).mean())
    bound = max(G_MAX, G_REL_MAX * float(np.abs(ref[covered]).max()))
    assert mx <= bound and mn <= G_MEAN and mn <= G_REL_MEAN * rm, (
        f"{what}: max-abs {mx:.3e} (<= {bound:.3e}), mean-abs {mn:.3e} (<= {G_MEAN} and <= {G_REL_MEAN} x {rm:.3e})")
    # rows outside every segment: zero (freshly allocated results)
    assert np.all(got[~covered] == 0), f"{what}: rows outside the segments were written"


def check_lse(got, ref, what):
    covered = ~np.isnan(ref)
    err = np.abs(got[covered] - ref[covered])
    assert np.isfinite(got[covered]).all(), f"{what}: non-finite lse"
    mx, mn = float(err.max()), float(err.mean())
    assert mx <= LSE_MAX and mn <= LSE_MEAN, f"{what}: lse max-abs {mx:.3e} (<= {LSE_MAX}), mean {mn:.3e}"


CASES = [
    # (lens, heads, head_dim, width, dtype, lead_rows, extra_rows[, backward kernel on 256 CUs])
    ([64, 64, 40, 1], 2, 80, None, torch.bfloat16, 0, 0),      # window kernels (2 waves)
    ([64, 0, 17, 64], 3, 72, None, torch.bfloat16, 2, 3),      # window, empty segment, uncovered rows
    ([33, 64], 2, 64, 64, torch.float16, 0, 1),               # window, full-width tables, fp16
    ([300, 130], 2, 72, None, torch.bfloat16, 0, 0),          # long kernels (4 waves)
    ([65, 0, 257], 2, 80, None, torch.bfloat16, 5, 2),        # long, empty segment, uncovered rows
    ([200], 1, 96, 96, torch.bfloat16, 0, 0),                 # long, full-width tables
    ([150, 70], 2, 128, None, torch.float16, 0, 0),           # long, head_dim 128, fp16
    ([1000], 1, 80, None, torch.bfloat16, 0, 0),              # long, many key/query blocks
    # long, 10 (segment, head) pairs: more than eight, not a multiple of
    # eight, so the units' deal to the XCDs takes its general branch
    ([300, 1, 64, 0, 200], 2, 80, None, torch.bfloat16, 0, 2),
    # window grids of 768 < segments x heads <= 1024 (256 CUs): the variant
    # with V in registers, four workgroups per CU
    ([64] * 52 + [17, 0, 5, 33], 16, 80, None, torch.bfloat16, 0, 0, "bwd_window_vreg"),
    ([64] * 58 + [40, 2], 16, 72, 72, torch.float16, 0, 2, "bwd_window_vreg"),
    # head_dim 64: the staged kernel fits four workgroups per CU itself, so
    # the same grid runs it (no register-V instance is built there)
    ([64] * 49 + [1], 16, 64, None, torch.bfloat16, 3, 0, "bwd_window_d64"),
    # head_dim 96 window backward: half-width tables with the register-V
    # instance (grid in (3, 4] x CUs) and the staged one (below it); full
    # width (no register-V instance); head_dim 128 (the forward sends it to
    # the long kernel, the backward to the window kernel)
    ([64] * 60 + [33, 5], 13, 96, None, torch.bfloat16, 0, 1, "bwd_window_vreg"),
    ([64, 64, 21, 0, 64], 3, 96, None, torch.bfloat16, 1, 0, "bwd_window_d"),
    ([64, 9, 64], 2, 96, 96, torch.float16, 0, 0, "bwd_window_d"),
    ([64, 33, 64], 2, 128, None, torch.float16, 0, 2, "bwd_window_d"),
]


@pytest.mark.parametrize("ci", range(len(CASES)))
def test_lse_and_backward_match_oracle(device, ci):
    lens, h, d, width, dtype, lead, extra = CASES[ci][:7]
    case = make_case(lens, h, d, seed=500 + ci, dtype=dtype, width=width, lead_rows=lead, extra_rows=extra)
    print(f"case {ci}: lens={lens} h={h} d={d} width={width} dtype={dtype}", flush=True)
    c = on(case, device)
    if len(CASES[ci]) > 7 and torch.cuda.get_device_properties(device).multi_processor_count == 256:
        name = backward_plan(c["q"], c["k"], c["v"], c["cos"], c["sin"], c["cu"], c["max_seqlen"])["name"]
        assert name.startswith(CASES[ci][7]), (name, CASES[ci][7])
    out, lse, dq, dk, dv = gpu_fwd_bwd(c)
    q, k, v, do = (f32(case[x]) for x in ("q", "k", "v", "dout"))
    cos, sin, cu = f32(case["cos"]), f32(case["sin"]), case["cu"].numpy()
    ref_lse = A.softmax_lse(q, k, cos, sin, cu)
    check_lse(f32(lse), ref_lse, f"case {ci}")
    rq, rk, rv = A.fused_rope_attention_bwd(do, q, k, v, cos, sin, cu)
    what = f"case {ci} lens={lens} d={d}"
    check_grad(f32(dq), rq, what + " dq")
    check_grad(f32(dk), rk, what + " dk")
    check_grad(f32(dv), rv, what + " dv")


@pytest.mark.parametrize("lens,d", [([64, 64, 64], 80), ([513], 72)])
def test_autograd_matches_functional(device, lens, d):
    case = on(make_case(lens, 2, d, seed=600), device)
    q, k, v = (case[x].clone().requires_grad_(True) for x in ("q", "k", "v"))
    out = fused_rope_attention(q, k, v, case["cos"], case["sin"], case["cu"], case["max_seqlen"])
    out.backward(case["dout"])
    _, _, dq, dk, dv = gpu_fwd_bwd(case)
    out_ng = fused_rope_attention(case["q"], case["k"], case["v"], case["cos"], case["sin"], case["cu"],
                                  case["max_seqlen"])
    torch.cuda.synchronize()
    assert torch.equal(out.detach(), out_ng)
    assert torch.equal(q.grad, dq) and torch.equal(k.grad, dk) and torch.equal(v.grad, dv)


def test_forward_lse_does_not_change_output(device):
    # the lse write is an extra store; the output is bit-identical with or without it
    for lens, d in (([64, 40], 80), ([700], 80)):
        c = on(make_case(lens, 2, d, seed=610), device)
        out, _ = fused_rope_attention_fwd(c["q"], c["k"], c["v"], c["cos"], c["sin"], c["cu"], c["max_seqlen"])
        ref = fused_rope_attention(c["q"], c["k"], c["v"], c["cos"], c["sin"], c["cu"], c["max_seqlen"])
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


def test_backward_deterministic(device):
    c = on(make_case([1000, 64], 2, 80, seed=620), device)
    a = gpu_fwd_bwd(c)
    b = gpu_fwd_bwd(c)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def _segment_sums(x, cu):
    """[nseg, H, D] float64 sums of x's rows over each segment."""
    x = x.double()
    cs = torch.cat([torch.zeros_like(x[:1]), x.cumsum(0)])
    cu = cu.long()
    return cs[cu[1:]] - cs[cu[:-1]]


@pytest.mark.parametrize("nseg,L,h", [(144, 64, 16), (1, 9216, 2)])
def test_backward_identities_full_size(device, nseg, L, h):
    """BASELINE sizes (cfg2 window layer; cfg2 full layer at 2 of 16 heads):
    sum_keys dv = sum_queries dout per (segment, head); with the identity
    rotation, sum_keys dk = 0 per (segment, head)."""
    d = 80
    n = nseg * L
    g = torch.Generator(device=device).manual_seed(630)
    q, k, v, do = (torch.randn(n, h, d, generator=g, device=device).to(torch.bfloat16) for _ in range(4))
    cu = torch.arange(0, n + 1, L, dtype=torch.int32, device=device)
    cos = torch.ones(n, d // 2, device=device)
    sin = torch.zeros(n, d // 2, device=device)
    out, lse = fused_rope_attention_fwd(q, k, v, cos, sin, cu, L)
    dq, dk, dv = fused_rope_attention_bwd(do, q, k, v, cos, sin, out, lse, cu, L)
    torch.cuda.synchronize()
    for t in (lse, dq, dk, dv):
        assert torch.isfinite(t).all()
    sdv, sdo = _segment_sums(dv, cu), _segment_sums(do, cu)
    # dv rows are bf16-rounded sums of L products: compare at the scale of a row sum
    tol = 2e-2 * float(sdo.abs().mean()) + 1e-2
    assert float((sdv - sdo).abs().max()) <= tol * 4, float((sdv - sdo).abs().max())
    assert float((sdv - sdo).abs().mean()) <= tol, float((sdv - sdo).abs().mean())
    sdk = _segment_sums(dk, cu)
    dk_row = float(dk.double().abs().mean())
    assert float(sdk.abs().mean()) <= 0.05 * dk_row * math.sqrt(L), (float(sdk.abs().mean()), dk_row)


@pytest.mark.parametrize("lens,d", [([64, 64, 30], 80), ([300, 40], 72)])
def test_autograd_packed_qkv_views(device, lens, d):
    """HF's `qkv(x).reshape(n, 3, h, d).unbind(1)` views (non-contiguous,
    read in place): the gradient reaches the packed tensor and equals the
    gradient of contiguous inputs bit for bit."""
    c = on(make_case(lens, 2, d, seed=640), device)
    qkv = torch.stack([c["q"], c["k"], c["v"]], 1).requires_grad_(True)  # [n, 3, h, d]
    q, k, v = qkv.unbind(1)
    assert not q.is_contiguous()
    out = fused_rope_attention(q, k, v, c["cos"], c["sin"], c["cu"], c["max_seqlen"])
    out.backward(c["dout"])
    _, _, dq, dk, dv = gpu_fwd_bwd(c)
    torch.cuda.synchronize()
    assert torch.equal(qkv.grad[:, 0], dq) and torch.equal(qkv.grad[:, 1], dk) and torch.equal(qkv.grad[:, 2], dv)


def test_backward_bf16_tables_widened(device):
    """bf16 tables: the backward widens them to fp32 (exact), so the
    gradients equal those computed with the widened tables."""
    c = on(make_case([200, 64], 2, 80, seed=650), device)
    cb = dict(c, cos=c["cos"].to(torch.bfloat16), sin=c["sin"].to(torch.bfloat16))
    cf = dict(c, cos=cb["cos"].float(), sin=cb["sin"].float())
    a = gpu_fwd_bwd(cb)
    b = gpu_fwd_bwd(cf)
    for x, y in zip(a[2:], b[2:]):
        assert torch.equal(x, y)


def test_double_backward_raises(device):
    """The backward is not itself differentiable: a second derivative raises
    instead of silently being zero."""
    c = on(make_case([64], 1, 80, seed=660), device)
    q = c["q"].clone().requires_grad_(True)
    out = fused_rope_attention(q, c["k"], c["v"], c["cos"], c["sin"], c["cu"], c["max_seqlen"])
    (gq,) = torch.autograd.grad(out, q, c["dout"], create_graph=True)
    with pytest.raises(RuntimeError):
        gq.float().sum().backward()


@pytest.mark.parametrize("d,tdt", [(64, torch.bfloat16), (96, torch.float16), (72, torch.float32)])
def test_backward_long_table_dtypes(device, d, tdt):
    """Long segments at more head dims, with 16-bit tables (widened for the
    backward) and int64 cu_seqlens, against the oracle."""
    case = make_case([190, 70], 2, d, seed=670 + d)
    case["cos"], case["sin"] = case["cos"].to(tdt), case["sin"].to(tdt)
    case["cu"] = case["cu"].to(torch.int64)
    out, lse, dq, dk, dv = gpu_fwd_bwd(on(case, device))
    q, k, v, do = (f32(case[x]) for x in ("q", "k", "v", "dout"))
    cos, sin, cu = f32(case["cos"]), f32(case["sin"]), case["cu"].numpy()
    check_lse(f32(lse), A.softmax_lse(q, k, cos, sin, cu), f"d={d}")
    rq, rk, rv = A.fused_rope_attention_bwd(do, q, k, v, cos, sin, cu)
    check_grad(f32(dq), rq, f"d={d} dq")
    check_grad(f32(dk), rk, f"d={d} dk")
    check_grad(f32(dv), rv, f"d={d} dv")


def test_backward_noncontiguous_dout(device):
    """A dout that is a strided view (copied to the kernels' layout) gives the
    same gradients as its contiguous copy."""
    c = on(make_case([64, 50, 200], 2, 80, seed=690), device)
    wide = torch.zeros(c["dout"].shape[0], 2, c["dout"].shape[1], c["dout"].shape[2], dtype=c["dout"].dtype,
                       device=device)
    wide[:, 1] = c["dout"]
    strided = wide[:, 1]
    assert not strided.is_contiguous()
    out, lse = fused_rope_attention_fwd(c["q"], c["k"], c["v"], c["cos"], c["sin"], c["cu"], c["max_seqlen"])
    a = fused_rope_attention_bwd(strided, c["q"], c["k"], c["v"], c["cos"], c["sin"], out, lse, c["cu"], c["max_seqlen"])
    b = fused_rope_attention_bwd(c["dout"], c["q"], c["k"], c["v"], c["cos"], c["sin"], out, lse, c["cu"],
                                 c["max_seqlen"])
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)
