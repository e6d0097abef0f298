"""Pins of the CPU oracle (oracle/attention.py) against mathematics and
independent implementations -- not against a re-typed copy of its formula.

* float64 brute force written element by element (oracle.brute_force_f64);
* torch's scaled_dot_product_attention (a library routine) when the tables
  are cos=1, sin=0, i.e. no rotation;
* closed-form properties: rotation preserves each pair's norm and composes
  by adding angles; permuting tokens inside a segment permutes the output
  rows; a one-token segment returns V; identical keys return the mean of V;
  segments are independent; cu_seqlens are clamped;
* the HF rotate_half form (transformers apply_rotary_pos_emb_vision) for the
  full-width table layout.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import numerics as NUM


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def rand_tables(n, half, seed, width=None):
    ang = np.random.default_rng(seed).uniform(-math.pi, math.pi, (n, half)).astype(np.float32)
    c, s = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    if width == 2 * half:
        ang2 = np.random.default_rng(seed + 1).uniform(-math.pi, math.pi, (n, half)).astype(np.float32)
        c = np.concatenate([c, np.cos(ang2)], 1).astype(np.float32)
        s = np.concatenate([s, np.sin(ang2)], 1).astype(np.float32)
    return c, s


@pytest.mark.parametrize("d,width,cu", [
    (8, 4, [0, 3, 7]),
    (8, 8, [0, 5, 5, 9]),        # full-width tables, an empty segment
    (12, 6, [0, 1, 6, 6, 10]),   # L=1 segment, D/2 not a multiple of 4
    (16, 8, [2, 9]),             # rows outside every segment stay NaN
])
def test_oracle_vs_brute_force_f64(d, width, cu):
    n, h = 11, 2
    q, k, v = rand((n, h, d), 1), rand((n, h, d), 2), rand((n, h, d), 3)
    c, s = rand_tables(n, d // 2, 4, width)
    ref = A.brute_force_f64(q, k, v, c, s, cu)
    got = A.fused_rope_attention(q, k, v, c, s, cu, mode="fp32")
    covered = ~np.isnan(ref)
    assert np.array_equal(covered, ~np.isnan(got))
    np.testing.assert_allclose(got[covered], ref[covered], rtol=2e-5, atol=2e-5)


def test_oracle_scale_argument():
    n, h, d = 9, 1, 8
    q, k, v = rand((n, h, d), 5), rand((n, h, d), 6), rand((n, h, d), 7)
    c, s = rand_tables(n, d // 2, 8)
    ref = A.brute_force_f64(q, k, v, c, s, [0, 9], softmax_scale=0.7)
    got = A.fused_rope_attention(q, k, v, c, s, [0, 9], softmax_scale=0.7)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)


def test_identity_rotation_is_plain_attention_vs_torch_sdpa():
    n, h, d = 40, 3, 16
    cu = [0, 17, 40]
    q, k, v = rand((n, h, d), 9), rand((n, h, d), 10), rand((n, h, d), 11)
    c, s = np.ones((n, d // 2), np.float32), np.zeros((n, d // 2), np.float32)
    got = A.fused_rope_attention(q, k, v, c, s, cu)
    for a, b in zip(cu[:-1], cu[1:]):
        tq, tk, tv = (torch.from_numpy(x[a:b]).double().transpose(0, 1) for x in (q, k, v))
        ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv).transpose(0, 1).numpy()
        np.testing.assert_allclose(got[a:b], ref, rtol=1e-5, atol=1e-5)


def test_rotation_preserves_pair_norms_and_composes():
    n, h, d = 13, 2, 20
    x = rand((n, h, d), 12).astype(np.float64)
    a1 = np.random.default_rng(13).uniform(-3, 3, (n, d // 2))
    a2 = np.random.default_rng(14).uniform(-3, 3, (n, d // 2))
    r1 = A.rotate(x, np.cos(a1), np.sin(a1)).astype(np.float64)
    half = d // 2
    np.testing.assert_allclose(r1[..., :half] ** 2 + r1[..., half:] ** 2,
                               x[..., :half] ** 2 + x[..., half:] ** 2, rtol=1e-5)
    r12 = A.rotate(r1, np.cos(a2), np.sin(a2))
    direct = A.rotate(x, np.cos(a1 + a2), np.sin(a1 + a2))
    np.testing.assert_allclose(r12, direct, rtol=1e-4, atol=1e-5)
    # the sign convention: a pair (x0, x1) = (1, 0) rotated by +pi/2 is (0, 1)
    e = np.zeros((1, 1, 2), np.float32)
    e[..., 0] = 1
    out = A.rotate(e, np.array([[0.0]]), np.array([[1.0]]))
    np.testing.assert_allclose(out.reshape(-1), [0.0, 1.0], atol=1e-7)


def test_rotation_matches_hf_rotate_half_form():
    tf = pytest.importorskip("transformers.models.qwen2_5_vl.modeling_qwen2_5_vl")
    n, h, d = 7, 3, 16
    x = rand((n, h, d), 15)
    c, s = rand_tables(n, d // 2, 16, width=d)
    qe, _ = tf.apply_rotary_pos_emb_vision(torch.from_numpy(x), torch.from_numpy(x),
                                           torch.from_numpy(c), torch.from_numpy(s))
    np.testing.assert_allclose(A.rotate(x, c, s), qe.numpy(), rtol=1e-6, atol=1e-6)
    # the reference's half-width layout equals HF's with cat(t, t) tables
    c2, s2 = rand_tables(n, d // 2, 17)
    full_c, full_s = np.concatenate([c2, c2], 1), np.concatenate([s2, s2], 1)
    np.testing.assert_array_equal(A.rotate(x, c2, s2), A.rotate(x, full_c, full_s))


def test_permutation_inside_segment_permutes_rows():
    n, h, d = 24, 2, 8
    cu = [0, 10, 24]
    q, k, v = rand((n, h, d), 18), rand((n, h, d), 19), rand((n, h, d), 20)
    c, s = rand_tables(n, d // 2, 21)
    base = A.fused_rope_attention(q, k, v, c, s, cu)
    perm = np.concatenate([np.random.default_rng(22).permutation(10), 10 + np.random.default_rng(23).permutation(14)])
    got = A.fused_rope_attention(q[perm], k[perm], v[perm], c[perm], s[perm], cu)
    np.testing.assert_allclose(got, base[perm], rtol=1e-5, atol=1e-6)


def test_single_token_segment_returns_v_and_identical_keys_average_v():
    n, h, d = 9, 2, 8
    q, k, v = rand((n, h, d), 24), rand((n, h, d), 25), rand((n, h, d), 26)
    c, s = rand_tables(n, d // 2, 27)
    out = A.fused_rope_attention(q, k, v, c, s, [0, 1, 9])
    np.testing.assert_allclose(out[0], v[0], rtol=1e-6)
    # identical keys at identical positions: uniform weights
    k2 = np.broadcast_to(k[:1], k.shape).copy()
    c2, s2 = np.broadcast_to(c[:1], c.shape).copy(), np.broadcast_to(s[:1], s.shape).copy()
    out = A.fused_rope_attention(q, k2, v, c2, s2, [0, 9])
    np.testing.assert_allclose(out, np.broadcast_to(v.mean(0, keepdims=True), v.shape), rtol=1e-5, atol=1e-6)


def test_segments_independent_and_clamped():
    n, h, d = 20, 1, 8
    q, k, v = rand((n, h, d), 28), rand((n, h, d), 29), rand((n, h, d), 30)
    c, s = rand_tables(n, d // 2, 31)
    both = A.fused_rope_attention(q, k, v, c, s, [0, 8, 20])
    first = A.fused_rope_attention(q[:8], k[:8], v[:8], c[:8], s[:8], [0, 8])
    np.testing.assert_array_equal(both[:8], first)
    # bounds past the tensor are clamped to [0, n]
    clamped = A.fused_rope_attention(q, k, v, c, s, [-5, 8, 99])
    np.testing.assert_array_equal(clamped, both)
    assert A.segments([0, 4, 4, 2, 9], 8) == [(0, 4), (2, 8)]


def test_emulation_modes_close_to_fp32():
    n, h, d = 64, 2, 16
    q, k, v = (NUM.round_bf16(rand((n, h, d), i)) for i in (32, 33, 34))
    c, s = rand_tables(n, d // 2, 35)
    ref = A.fused_rope_attention(q, k, v, c, s, [0, 64])
    for mode, tol in (("bf16", 2e-2), ("f16", 3e-3)):
        got = A.fused_rope_attention(q, k, v, c, s, [0, 64], mode=mode)
        assert np.abs(got - ref).max() < tol


def test_round_bf16_matches_torch():
    x = np.concatenate([rand((4096,), 36) * 100, np.array([0.0, -0.0, 1.0, 3.0e38, -3.0e38, 1e-40,
                                                          np.inf, -np.inf], np.float32)]).astype(np.float32)
    # ties: values exactly half-way between two bf16 numbers
    ties = (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, -ties])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(NUM.round_bf16(x), ref)
    np.testing.assert_array_equal(NUM.from_bf16_bits(NUM.bf16_bits(x)), ref)
    assert np.isnan(NUM.round_bf16(np.array([np.nan], np.float32)))[0]


# ---- softmax statistics and gradients (the build's backward) ------------------


def _torch_f64_forward(q, k, v, c, s, cu, scale=None):
    """The unfused path in float64 torch ops (rotate_half form, per-segment
    softmax attention), differentiable by autograd: an implementation that
    shares no code with the oracle's backward."""
    d = q.shape[-1]
    half = d // 2
    c, s = torch.from_numpy(c).double(), torch.from_numpy(s).double()
    if c.shape[-1] == half:
        c, s = torch.cat([c, c], -1), torch.cat([s, s], -1)
    c, s = c[:, None, :], s[:, None, :]

    def rot(x):
        rh = torch.cat([-x[..., half:], x[..., :half]], -1)
        return x * c + rh * s

    qr, kr = rot(q), rot(k)
    scale = d ** -0.5 if scale is None else scale
    outs = []
    for a, b in A.segments(cu, q.shape[0]):
        p = torch.softmax(torch.einsum("ihd,jhd->hij", qr[a:b], kr[a:b]) * scale, -1)
        outs.append((a, b, torch.einsum("hij,jhd->ihd", p, v[a:b])))
    out = torch.zeros_like(q)
    for a, b, o in outs:
        out = out.index_copy(0, torch.arange(a, b), o)
    return out


@pytest.mark.parametrize("d,width,cu", [
    (8, 4, [0, 7, 7, 25, 40]),   # half-width tables, an empty segment
    (8, 8, [0, 13, 40]),         # full-width tables (second half rotates by its own angles)
    (12, 6, [3, 4, 30]),         # L=1 segment, rows outside every segment
])
def test_oracle_backward_vs_torch_autograd(d, width, cu):
    n, h = 40, 2
    q, k, v, g = (rand((n, h, d), 20 + i) for i in range(4))
    c, s = rand_tables(n, d // 2, 24, width)
    dq, dk, dv = A.fused_rope_attention_bwd(g, q, k, v, c, s, cu, softmax_scale=0.6)
    tq, tk, tv = (torch.from_numpy(x).double().requires_grad_(True) for x in (q, k, v))
    _torch_f64_forward(tq, tk, tv, c, s, cu, scale=0.6).backward(torch.from_numpy(g).double())
    covered = ~np.isnan(dq)
    rows = np.zeros(n, bool)
    for a, b in A.segments(cu, n):
        rows[a:b] = True
    assert np.array_equal(covered.all(axis=(1, 2)), rows)
    for got, ref in ((dq, tq.grad), (dk, tk.grad), (dv, tv.grad)):
        np.testing.assert_allclose(got[covered], ref.numpy()[covered], rtol=1e-4, atol=2e-6)


def test_oracle_backward_finite_differences_vs_brute_force():
    """Directional derivative of L = sum(dout * O) along random directions,
    O from the element-by-element float64 brute force, against the oracle's
    gradient."""
    n, h, d = 9, 1, 8
    cu = [0, 4, 9]
    q, k, v, g = (rand((n, h, d), 40 + i).astype(np.float64) for i in range(4))
    c, s = rand_tables(n, d // 2, 44, d)
    dq, dk, dv = A.fused_rope_attention_bwd(g, q, k, v, c, s, cu)
    eps = 1e-5
    for which, grad in ((0, dq), (1, dk), (2, dv)):
        direction = np.random.default_rng(50 + which).standard_normal((n, h, d))

        def loss(t):
            args = [q, k, v]
            args[which] = args[which] + t * direction
            return float((A.brute_force_f64(*args, c, s, cu) * g).sum())

        fd = (loss(eps) - loss(-eps)) / (2 * eps)
        assert abs(fd - float((grad * direction).sum())) <= 1e-4 * max(1.0, abs(fd)), (which, fd)


def test_softmax_lse_vs_scipy_logsumexp():
    from scipy.special import logsumexp
    n, h, d = 30, 2, 8
    cu = [0, 11, 11, 30]
    q, k = rand((n, h, d), 60), rand((n, h, d), 61)
    c, s = rand_tables(n, d // 2, 62)
    got = A.softmax_lse(q, k, c, s, cu, softmax_scale=0.8)
    qr, kr = A.rotate(q, c, s).astype(np.float64), A.rotate(k, c, s).astype(np.float64)
    for a, b in A.segments(cu, n):
        for hh in range(h):
            ref = logsumexp(qr[a:b, hh] @ kr[a:b, hh].T * 0.8, axis=1)
            np.testing.assert_allclose(got[hh, a:b], ref, rtol=1e-6, atol=1e-6)


def test_backward_identities():
    """Rows of P sum to 1, so per segment the sum over keys of dv equals the
    sum over queries of dout; rows of dZ sum to 0, so with the identity
    rotation the sum over keys of dk is 0; a one-token segment has dq = dk = 0
    and dv = dout."""
    n, h, d = 50, 2, 8
    cu = [0, 1, 20, 50]
    q, k, v, g = (rand((n, h, d), 70 + i) for i in range(4))
    c, s = np.ones((n, d // 2), np.float32), np.zeros((n, d // 2), np.float32)
    dq, dk, dv = A.fused_rope_attention_bwd(g, q, k, v, c, s, cu)
    for a, b in zip(cu[:-1], cu[1:]):
        np.testing.assert_allclose(dv[a:b].sum(0), g[a:b].sum(0), rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(dk[a:b].sum(0), 0.0, atol=1e-5)
    np.testing.assert_allclose(dq[0], 0.0, atol=1e-7)
    np.testing.assert_allclose(dv[0], g[0], atol=1e-7)


def test_backward_emulation_close_to_fp32():
    n, h, d = 128, 2, 16
    cu = [0, 64, 128]
    q, k, v, g = (NUM.round_bf16(rand((n, h, d), 80 + i)) for i in range(4))
    c, s = rand_tables(n, d // 2, 84)
    ref = A.fused_rope_attention_bwd(g, q, k, v, c, s, cu)
    emu = A.fused_rope_attention_bwd(g, q, k, v, c, s, cu, mode="bf16")
    for r, e in zip(ref, emu):
        assert np.abs(r - e).mean() <= 1e-2 * np.abs(r).mean()
        assert np.abs(r - e).max() <= 2e-2 * np.abs(r).max()
