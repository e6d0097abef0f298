"""The unfused RoPE + varlen attention path, restated in numpy.

Test infrastructure only (see ``oracle/__init__.py``).

Reference semantics restated here:

* split-half ("rotate_half", NeoX) rotation with per-token tables
  (reference ``fused_attn.py:319-345`` for Q, ``:364-390`` for K):
  ``x0' = x0*c - x1*s``, ``x1' = x0*s + x1*c`` with ``x0 = x[:D/2]``,
  ``x1 = x[D/2:]``, computed in fp32.  With full-width tables ``[N, D]``
  (the HF layout) the second half uses the second half of the tables,
  which is HF's ``q*cos + rotate_half(q)*sin``
  (transformers ``modeling_qwen2_5_vl.py:160-172``);
* per segment ``[cu[i], cu[i+1])`` non-causal softmax attention with
  scale ``1/sqrt(D)`` by default (``fused_attn.py:353-355``), keys of the
  same segment only (``:359-395``), empty segments skipped (``:295-296``);
* rows outside every segment are not written by the reference
  (``fused_attn.py:196``: ``empty_like``); the oracle returns NaN there.

Modes:

* ``"fp32"``: everything in fp32, no intermediate rounding -- the unfused
  path "evaluated in fp32", the official parity target.
* ``"bf16"`` / ``"f16"``: diagnostic model of the fused kernel's rounding
  points: Q_rot and K_rot rounded to the input dtype (``:344-345,
  389-390``), P rounded to V's dtype before PV (``:413``), the row sum taken
  from the unrounded P (``:400``), output rounded to the input dtype
  (``:423``).
"""
import math

import numpy as np

from .numerics import round_to


def rotate(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Split-half rotation of ``x [N, H, D]`` (fp32) by per-token tables.

    ``cos``/``sin`` are ``[N, D/2]`` (reference layout) or ``[N, D]`` (HF
    layout).  Products and the sum are each rounded to fp32, as separate
    elementwise torch ops do.
    """
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1]
    half = d // 2
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    c0, s0 = cos[:, None, :half], sin[:, None, :half]
    if cos.shape[-1] == d:
        c1, s1 = cos[:, None, half:], sin[:, None, half:]
    elif cos.shape[-1] == half:
        c1, s1 = c0, s0
    else:
        raise ValueError(f"cos/sin width must be D/2 or D, got {cos.shape[-1]} for D={d}")
    x0, x1 = x[..., :half], x[..., half:]
    r0 = (x0 * c0).astype(np.float32) - (x1 * s0).astype(np.float32)
    r1 = (x0 * s1).astype(np.float32) + (x1 * c1).astype(np.float32)
    return np.concatenate([r0, r1], axis=-1).astype(np.float32)


def _softmax_rows(s: np.ndarray) -> np.ndarray:
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    return p / p.sum(axis=-1, keepdims=True)


def segments(cu, total: int):
    """(start, end) pairs of the non-empty segments, clamped to [0, total]."""
    cu = np.asarray(cu, dtype=np.int64)
    out = []
    for i in range(cu.size - 1):
        a = int(min(max(cu[i], 0), total))
        b = int(min(max(cu[i + 1], 0), total))
        if b > a:
            out.append((a, b))
    return out


def _attend_fp32(qr, kr, v, segs, scale, out, row_chunk):
    """fp32 softmax(Qr Kr^T * scale) V per segment; batches equal lengths."""
    by_len = {}
    for a, b in segs:
        by_len.setdefault(b - a, []).append(a)
    h = qr.shape[1]
    for L, starts in by_len.items():
        starts = np.asarray(starts)
        per_seg = L * L * h * 4
        batch = max(1, min(len(starts), (256 << 20) // max(per_seg, 1)))
        if per_seg <= (256 << 20):
            idx = starts[:, None] + np.arange(L)[None, :]
            for i in range(0, len(starts), batch):
                sl = idx[i:i + batch]
                q = qr[sl].transpose(0, 2, 1, 3)      # [B, H, L, D]
                k = kr[sl].transpose(0, 2, 3, 1)      # [B, H, D, L]
                vv = v[sl].transpose(0, 2, 1, 3)      # [B, H, L, D]
                p = _softmax_rows(np.matmul(q, k) * np.float32(scale))
                o = np.matmul(p.astype(np.float32), vv)  # [B, H, L, D]
                out[sl] = o.transpose(0, 2, 1, 3)
        else:
            for a in starts:
                for hh in range(h):
                    k = np.ascontiguousarray(kr[a:a + L, hh].T)
                    vv = np.ascontiguousarray(v[a:a + L, hh])
                    for r0 in range(0, L, row_chunk):
                        r1 = min(L, r0 + row_chunk)
                        q = qr[a + r0:a + r1, hh]
                        p = _softmax_rows(np.matmul(q, k) * np.float32(scale))
                        out[a + r0:a + r1, hh] = np.matmul(p, vv)


def _attend_emulate(qr, kr, v, segs, scale_log2, dtype, out, row_chunk):
    """Model of the fused kernel's rounding: exp2 domain, P rounded to the
    value dtype before PV, row sum from the unrounded P."""
    h = qr.shape[1]
    for a, b in segs:
        L = b - a
        for hh in range(h):
            k = np.ascontiguousarray(kr[a:b, hh].T)
            vv = np.ascontiguousarray(v[a:b, hh])
            for r0 in range(0, L, row_chunk):
                r1 = min(L, r0 + row_chunk)
                s = np.matmul(qr[a + r0:a + r1, hh], k) * np.float32(scale_log2)
                m = s.max(axis=-1, keepdims=True)
                p = np.exp2(s - m).astype(np.float32)
                l = p.sum(axis=-1, keepdims=True, dtype=np.float32)
                acc = np.matmul(round_to(p, dtype), vv)
                out[a + r0:a + r1, hh] = acc / l


def fused_rope_attention(q, k, v, cos, sin, cu_seqlens, softmax_scale=None,
                         mode: str = "fp32", row_chunk: int = 2048):
    """Oracle of ``fused_rope_attention`` (reference fused_attn.py:139-232).

    ``q, k, v``: ``[N, H, D]`` arrays already holding the values the GPU
    sees (e.g. bf16-rounded and upcast to fp32).  Returns fp32 ``[N, H, D]``
    with NaN in rows not covered by any segment.
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    n, h, d = q.shape
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(d)
    qr = rotate(q, cos, sin)
    kr = rotate(k, cos, sin)
    out = np.full((n, h, d), np.nan, dtype=np.float32)
    segs = segments(cu_seqlens, n)
    if mode == "fp32":
        _attend_fp32(qr, kr, v, segs, softmax_scale, out, row_chunk)
        return out
    if mode in ("bf16", "f16"):
        qr = round_to(qr, mode)
        kr = round_to(kr, mode)
        scale_log2 = np.float32(softmax_scale) * np.float32(1.4426950408889634)
        _attend_emulate(qr, kr, v, segs, scale_log2, mode, out, row_chunk)
        covered = ~np.isnan(out)
        out[covered] = round_to(out[covered], mode)
        return out
    raise ValueError(f"unknown mode {mode!r}")


def brute_force_f64(q, k, v, cos, sin, cu_seqlens, softmax_scale=None):
    """Explicit-loop float64 evaluation for tiny inputs.

    Written element by element (no matrix products, no rotate helper) so it
    shares no code with the vectorised oracle above.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    cos = np.asarray(cos, dtype=np.float64)
    sin = np.asarray(sin, dtype=np.float64)
    n, h, d = q.shape
    half = d // 2
    full = cos.shape[-1] == d
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(d)

    def rot(x, t):
        y = [0.0] * d
        for j in range(half):
            c0, s0 = cos[t, j], sin[t, j]
            c1, s1 = (cos[t, j + half], sin[t, j + half]) if full else (c0, s0)
            y[j] = x[j] * c0 - x[j + half] * s0
            y[j + half] = x[j] * s1 + x[j + half] * c1
        return y

    out = np.full((n, h, d), np.nan)
    for a, b in segments(cu_seqlens, n):
        for hh in range(h):
            kr = [rot(k[t, hh], t) for t in range(a, b)]
            for i in range(a, b):
                qi = rot(q[i, hh], i)
                logits = [softmax_scale * sum(qi[j] * kr[t][j] for j in range(d)) for t in range(b - a)]
                mx = max(logits)
                w = [math.exp(x - mx) for x in logits]
                z = sum(w)
                for j in range(d):
                    out[i, hh, j] = sum(w[t] * v[a + t, hh, j] for t in range(b - a)) / z
    return out



# ---------------------------------------------------------------------------
# Softmax statistics and gradients (beyond the reference, which is
# forward-only: these restate the derivative of its arithmetic,
# fused_attn.py:316-423, for the build's backward).
# ---------------------------------------------------------------------------


def rotate_transpose(g: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Transpose of ``rotate`` applied to a gradient ``g [N, H, D]``: with
    ``x0' = x0 c0 - x1 s0`` and ``x1' = x0 s1 + x1 c1`` (``c1 = c0``,
    ``s1 = s0`` for half-width tables), ``g0 = g0' c0 + g1' s1`` and
    ``g1 = g1' c1 - g0' s0``."""
    g = np.asarray(g, dtype=np.float32)
    d = g.shape[-1]
    half = d // 2
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    c0, s0 = cos[:, None, :half], sin[:, None, :half]
    if cos.shape[-1] == d:
        c1, s1 = cos[:, None, half:], sin[:, None, half:]
    else:
        c1, s1 = c0, s0
    g0, g1 = g[..., :half], g[..., half:]
    return np.concatenate([g0 * c0 + g1 * s1, g1 * c1 - g0 * s0], axis=-1).astype(np.float32)


def softmax_lse(q, k, cos, sin, cu_seqlens, softmax_scale=None) -> np.ndarray:
    """Natural-log row sums ``lse[h, t] = log sum_j exp(scale * q_rot[t, h] .
    k_rot[j, h])`` over the keys of t's segment, ``[H, N]`` fp32, NaN for rows
    outside every segment (computed in float64)."""
    q = np.asarray(q, dtype=np.float32)
    n, h, d = q.shape
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(d)
    qr = rotate(q, cos, sin).astype(np.float64)
    kr = rotate(np.asarray(k, dtype=np.float32), cos, sin).astype(np.float64)
    out = np.full((h, n), np.nan, dtype=np.float64)
    for a, b in segments(cu_seqlens, n):
        for hh in range(h):
            s = (qr[a:b, hh] @ kr[a:b, hh].T) * softmax_scale
            m = s.max(axis=-1, keepdims=True)
            out[hh, a:b] = (m + np.log(np.exp(s - m).sum(axis=-1, keepdims=True)))[:, 0]
    return out.astype(np.float32)


def fused_rope_attention_bwd(dout, q, k, v, cos, sin, cu_seqlens, softmax_scale=None, mode: str = "fp32"):
    """Gradients ``(dq, dk, dv)`` of the oracle's forward at ``dout``.

    Per segment and head, with ``P = softmax(scale * q_rot k_rot^T)`` and
    ``O = P v``: ``dv = P^T dout``, ``dZ = P * (dout v^T - rowsum(dout * O))``,
    ``dq = rot^T(scale * dZ k_rot)``, ``dk = rot^T(scale * dZ^T q_rot)``.

    ``mode="fp32"``: all in fp32 from the inputs (the parity target).
    ``mode="bf16"``/``"f16"``: diagnostic model of the GPU kernels' rounding
    points: q_rot/k_rot rounded to the dtype, O rounded (the forward's
    output), P and dZ rounded before their products, results rounded.
    Rows outside every segment are NaN.
    """
    dout = np.asarray(dout, dtype=np.float32)
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    n, h, d = q.shape
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(d)
    scale = np.float32(softmax_scale)
    emulate = mode in ("bf16", "f16")
    if mode not in ("fp32", "bf16", "f16"):
        raise ValueError(f"unknown mode {mode!r}")
    rnd = (lambda x: round_to(x, mode)) if emulate else (lambda x: x)
    qr = rnd(rotate(q, cos, sin))
    kr = rnd(rotate(k, cos, sin))
    dqr = np.full((n, h, d), np.nan, dtype=np.float32)
    dkr = np.full((n, h, d), np.nan, dtype=np.float32)
    dv = np.full((n, h, d), np.nan, dtype=np.float32)
    for a, b in segments(cu_seqlens, n):
        for hh in range(h):
            qs, ks, vs, gs = qr[a:b, hh], kr[a:b, hh], v[a:b, hh], dout[a:b, hh]
            s = (qs @ ks.T) * scale
            p = _softmax_rows(s).astype(np.float32)
            o = rnd((p @ vs).astype(np.float32)) if not emulate else rnd(
                (round_to(p, mode) @ vs).astype(np.float32))
            dvec = (gs * o).sum(axis=-1, keepdims=True, dtype=np.float32)
            dp = (gs @ vs.T).astype(np.float32)
            dz = (p * (dp - dvec)).astype(np.float32)
            dv[a:b, hh] = rnd(p).T @ gs
            dqr[a:b, hh] = (rnd(dz) @ ks) * scale
            dkr[a:b, hh] = (rnd(dz).T @ qs) * scale
    dq = rotate_transpose(dqr, cos, sin)
    dk = rotate_transpose(dkr, cos, sin)
    if emulate:
        covered = ~np.isnan(dq)
        dq[covered] = round_to(dq[covered], mode)
        dk[covered] = round_to(dk[covered], mode)
        dv[covered] = round_to(dv[covered], mode)
    return dq, dk, dv
