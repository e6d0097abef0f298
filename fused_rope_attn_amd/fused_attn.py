"""Fused 2D-RoPE + varlen attention for vision encoders, on MI355X.

Drop-in for the reference module ``fused_attn.py``:

* ``fused_rope_attention`` -- reference ``fused_attn.py:139-232``; the
  device work runs in ``libfra.so`` (hand-written gfx950 HIP kernels behind
  the C ABI of ``include/fra.h``).  Same argument order, layout, dtype rules,
  validation messages and return value; ``max_seqlen`` and
  ``softmax_scale`` are optional extras after ``cu_seqlens``.
* ``compute_rope_2d`` -- reference ``fused_attn.py:33-136`` (with its LRU
  cache, ``:18-30``): the cos/sin tables the op consumes.
* ``next_pow2`` -- reference ``fused_attn.py:13-15``.
* ``rope_positions_2d`` / ``fused_rope_attention_pos`` -- beyond the
  reference: the same op with the rotation angles computed in the kernels
  from each token's (h, w) patch position and the inverse frequencies, so
  that no cos/sin table is built (``compute_rope_2d``) or read.

Beyond the reference (which is forward-only): ``fused_rope_attention``
records an autograd graph when q, k or v require grad, and
``fused_rope_attention_fwd`` / ``fused_rope_attention_bwd`` expose the
forward with its log-sum-exp and the gradients as plain functions.
"""
import contextlib
import ctypes
from collections import OrderedDict

import torch

from . import _lib

__all__ = ["fused_rope_attention", "fused_rope_attention_fwd", "fused_rope_attention_bwd",
           "compute_rope_2d", "next_pow2", "plan", "backward_plan",
           "rope_positions_2d", "fused_rope_attention_pos", "plan_pos"]


def next_pow2(n: int) -> int:
    """Smallest power of 2 >= n (1 for n <= 0), as reference fused_attn.py:13-15."""
    n = int(n)
    if n <= 1:
        return 1
    return 1 << (n - 1).bit_length()


# ---------------------------------------------------------------------------
# RoPE tables (reference fused_attn.py:18-136)
# ---------------------------------------------------------------------------

_rope_cache: "OrderedDict[tuple, tuple]" = OrderedDict()
_ROPE_CACHE_MAX = 32


def _device_key(device: torch.device) -> tuple:
    if device.type == "cuda":
        return ("cuda", device.index if device.index is not None else torch.cuda.current_device())
    return (device.type, device.index)


def _merge_order(h: int, w: int, merge: int, device) -> tuple:
    """(h, w) patch coordinates of an h x w grid listed block-major over
    merge x merge blocks: block row, block column, then the patches of the
    block row-major (reference fused_attn.py:86-94)."""
    if h % merge or w % merge:
        raise RuntimeError(f"grid h={h}, w={w} is not divisible by spatial_merge_size={merge}")
    mu = merge * merge
    n = torch.arange(h * w, device=device, dtype=torch.int64)
    blk, inner = n // mu, n % mu
    bw_count = w // merge
    hp = (blk // bw_count) * merge + inner // merge
    wp = (blk % bw_count) * merge + inner % merge
    return hp, wp


def compute_rope_2d(grid_thw, head_dim: int, spatial_merge_size: int, theta: float, device, dtype,
                    window_idx: "torch.Tensor | None" = None):
    """2D vision RoPE tables ``(cos, sin)``, each ``[total_seq, head_dim // 2]``.

    For every image ``(t, h, w)``: patch coordinates in spatial-merge block
    order, repeated ``t`` times; ``inv_freq = 1/theta**(arange(0, D/2, 2)/(D/2))``;
    ``emb = [h * inv_freq || w * inv_freq]``; ``cos(emb)``, ``sin(emb)`` cast
    to ``dtype``.  ``window_idx`` (a permutation of merge units, from
    ``get_window_index``) reorders the rows into window order.  Results are
    cached (32 entries, LRU) per (grids, head_dim, merge, theta, device,
    dtype), as in reference fused_attn.py:71-122.
    """
    assert head_dim > 0 and head_dim % 4 == 0, f"head_dim must be divisible by 4, got {head_dim}"
    rd = head_dim // 2
    merge = int(spatial_merge_size)
    device = torch.device(device)
    if isinstance(grid_thw, torch.Tensor):
        thw = [tuple(int(x) for x in row) for row in grid_thw.detach().cpu().tolist()]
    else:
        thw = [(int(t), int(h), int(w)) for t, h, w in grid_thw]

    key = (tuple(thw), int(head_dim), merge, float(theta), *_device_key(device), dtype)
    hit = _rope_cache.get(key)
    if hit is not None:
        _rope_cache.move_to_end(key)
        cos, sin = hit
    else:
        inv = 1.0 / (theta ** (torch.arange(0, rd, 2, device=device, dtype=torch.float32) / rd))
        hs, ws = [], []
        for t, h, w in thw:
            hp, wp = _merge_order(h, w, merge, device)
            hs.append(hp.repeat(t))
            ws.append(wp.repeat(t))
        hpos = torch.cat(hs).to(torch.float32)
        wpos = torch.cat(ws).to(torch.float32)
        emb = torch.cat([torch.outer(hpos, inv), torch.outer(wpos, inv)], dim=1)
        cos = emb.cos().to(dtype).contiguous()
        sin = emb.sin().to(dtype).contiguous()
        _rope_cache[key] = (cos, sin)
        while len(_rope_cache) > _ROPE_CACHE_MAX:
            _rope_cache.popitem(last=False)

    if window_idx is not None:
        mu = merge * merge
        widx = window_idx.to(device=device, dtype=torch.long)
        cos = cos.view(-1, mu, rd).index_select(0, widx).reshape(-1, rd)
        sin = sin.view(-1, mu, rd).index_select(0, widx).reshape(-1, rd)
    return cos.contiguous(), sin.contiguous()


# ---------------------------------------------------------------------------
# The op (reference fused_attn.py:139-232)
# ---------------------------------------------------------------------------

_QKV_CODE = {torch.bfloat16: _lib.FRA_DTYPE_BF16, torch.float16: _lib.FRA_DTYPE_F16}
_ROPE_CODE = {torch.bfloat16: _lib.FRA_DTYPE_BF16, torch.float16: _lib.FRA_DTYPE_F16,
              torch.float32: _lib.FRA_DTYPE_F32}


def _fits(t: torch.Tensor, ptr_align: int, stride_mult: int) -> bool:
    """True if the kernels can read ``t`` in place: unit stride on the last
    dim, base aligned to ``ptr_align`` bytes, outer strides multiples of
    ``stride_mult`` elements."""
    if t.stride(-1) != 1 and t.shape[-1] > 1:
        return False
    if t.data_ptr() % ptr_align:
        return False
    return all(s % stride_mult == 0 for s in t.stride()[:-1])


# The current stream of a device as a raw handle, without building a
# torch.cuda.Stream object per call (torch's own generated code reads it the
# same way); the public call where this build of torch lacks the binding.
_get_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _raw_stream(device: torch.device) -> int:
    if _get_raw_stream is not None:
        return _get_raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _on_device(device: torch.device):
    """``device`` current for the launch (the library queries the current
    device's CU count); no context switch when it already is."""
    if device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def _kernel_layout(t: torch.Tensor, ptr_align: int, stride_mult: int) -> torch.Tensor:
    return t if _fits(t, ptr_align, stride_mult) else t.contiguous()


def _build_args(q, k, v, cos, sin, out, cu, max_seqlen: int, scale: float) -> "_lib.FwdArgs":
    a = _lib.FwdArgs()
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.cos, a.sin, a.out = cos.data_ptr(), sin.data_ptr(), out.data_ptr()
    a.cu_seqlens = cu.data_ptr()
    a.q_stride_seq, a.q_stride_head = q.stride(0), q.stride(1)
    a.k_stride_seq, a.k_stride_head = k.stride(0), k.stride(1)
    a.v_stride_seq, a.v_stride_head = v.stride(0), v.stride(1)
    a.out_stride_seq, a.out_stride_head = out.stride(0), out.stride(1)
    a.rope_stride_seq = cos.stride(0)
    a.total_seq, a.num_heads, a.head_dim = q.shape
    a.num_seqs = cu.numel() - 1
    a.max_seqlen = int(max_seqlen)
    a.rope_width = cos.shape[1]
    a.qkv_dtype = _QKV_CODE[q.dtype]
    a.rope_dtype = _ROPE_CODE[cos.dtype]
    a.softmax_scale = float(scale)
    a.flags = 0
    return a


def _validate(q, k, v, cos, sin, cu_seqlens, out) -> None:
    """The reference's checks and messages (fused_attn.py:159-185, 195-201),
    with cos/sin also accepted at width head_dim (HF cat(emb, emb) layout)."""
    if q.device.type != "cuda":
        raise ValueError(f"q must be on CUDA, got device={q.device}")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q/k/v must have same shape, got q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    if q.ndim != 3:
        raise ValueError(f"q/k/v must be [total_seq, num_heads, head_dim], got q.ndim={q.ndim}")
    total_seq, num_heads, head_dim = (int(q.shape[0]), int(q.shape[1]), int(q.shape[2]))
    if head_dim <= 0 or head_dim % 2 != 0:
        raise ValueError(f"head_dim must be positive and even, got {head_dim}")
    if head_dim > MAX_HEAD_DIM:
        raise ValueError(f"head_dim must be <= {MAX_HEAD_DIM} (the kernels keep a query row's rotated "
                         f"head_dim values in registers), got {head_dim}")
    widths = ((total_seq, head_dim // 2), (total_seq, head_dim))
    if tuple(cos.shape) not in widths or tuple(sin.shape) != tuple(cos.shape):
        raise ValueError(
            f"cos/sin must be [total_seq, head_dim//2]={total_seq, head_dim // 2}, "
            f"got cos={tuple(cos.shape)} sin={tuple(sin.shape)}")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError(f"cu_seqlens must be 1D with length >= 2, got {tuple(cu_seqlens.shape)}")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"q dtype must be float16 or bfloat16, got {q.dtype}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q/k/v must share dtype, got q={q.dtype} k={k.dtype} v={v.dtype}")
    if cos.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"cos dtype must be float16, bfloat16 or float32, got {cos.dtype}")
    if sin.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"sin dtype must be float16, bfloat16 or float32, got {sin.dtype}")
    if out is not None:
        if out.shape != q.shape:
            raise ValueError(f"out must have shape {tuple(q.shape)}, got {tuple(out.shape)}")
        if out.dtype != q.dtype or out.device != q.device:
            raise ValueError(f"out must match q dtype/device, got out={out.dtype}/{out.device} q={q.dtype}/{q.device}")
    for name, t in (("k", k), ("v", v), ("cos", cos), ("sin", sin)):
        if t.device != q.device:
            raise ValueError(f"{name} must be on {q.device}, got {t.device}")


# ---------------------------------------------------------------------------
# head_dim coverage.  The reference takes any even head_dim and pads it to a
# power of two inside its kernel (fused_attn.py:167-168, 215-216).  Here the
# library has kernels for a fixed set of head dims (fra_supports_head_dim);
# any other even head_dim up to MAX_HEAD_DIM runs at the next compiled one
# with zero-padded inputs, which changes no result: the padded dims add 0 to
# every dot product and the padded value columns are dropped.
# ---------------------------------------------------------------------------

MAX_HEAD_DIM = 128

_kernel_dims: "dict[int, int]" = {}


def _kernel_head_dim(d: int) -> int:
    """The head_dim the kernels run ``d`` at (``d`` itself when compiled)."""
    dp = _kernel_dims.get(d)
    if dp is None:
        if d > MAX_HEAD_DIM:
            raise ValueError(f"head_dim must be <= {MAX_HEAD_DIM} (the kernels keep a query row's rotated "
                             f"head_dim values in registers), got {d}")
        lib = _lib.load()
        dp = next((c for c in range(d, MAX_HEAD_DIM + 1) if c % 8 == 0 and lib.fra_supports_head_dim(c)), None)
        if dp is None:
            raise ValueError(f"head_dim={d} has no kernel at or above it in this build of libfra.so")
        _kernel_dims[d] = dp
    return dp


def _pad_halves(x: torch.Tensor, d: int, dp: int) -> torch.Tensor:
    """``[..., d]`` -> ``[..., dp]`` keeping the rotation's split-half pairs:
    ``x[..., :d/2]`` at ``[0, d/2)`` and ``x[..., d/2:]`` at
    ``[dp/2, dp/2 + d/2)``; zeros elsewhere."""
    y = x.new_zeros(*x.shape[:-1], dp)
    y[..., : d // 2] = x[..., : d // 2]
    y[..., dp // 2: dp // 2 + d // 2] = x[..., d // 2:]
    return y


def _unpad_halves(y: torch.Tensor, d: int, dp: int) -> torch.Tensor:
    return torch.cat([y[..., : d // 2], y[..., dp // 2: dp // 2 + d // 2]], dim=-1)


def _pad_tail(x: torch.Tensor, d: int, dp: int) -> torch.Tensor:
    """``[..., d]`` -> ``[..., dp]`` with zeros after the first d values."""
    y = x.new_zeros(*x.shape[:-1], dp)
    y[..., :d] = x
    return y


def _pad_table(t: torch.Tensor, d: int, dp: int) -> torch.Tensor:
    """cos/sin of width d/2 -> dp/2 (zeros after), width d -> dp (halves
    split as in ``_pad_halves``)."""
    return _pad_tail(t, d // 2, dp // 2) if t.shape[-1] == d // 2 else _pad_halves(t, d, dp)


def _uses_long_kernel(max_seqlen: int, head_dim: int) -> bool:
    """The library's kernel choice: segments of at most 64 tokens at
    head_dim <= 96 go to the window kernel, everything else to the long one."""
    return not (max_seqlen <= 64 and head_dim <= 96)


def _prepare_cu(cu_seqlens, device):
    cu = cu_seqlens
    if cu.dtype != torch.int32 or cu.device != device or not cu.is_contiguous():
        cu = cu.to(device=device, dtype=torch.int32).contiguous()
    return cu


def _prepare(q, k, v, cos, sin, long_kernel: bool):
    """Kernel-readable views: strided q/k/v are used in place when their
    last dim is contiguous and aligned (packed qkv views from a fused qkv
    projection qualify); anything else is copied, as the reference copies
    non-contiguous inputs (fused_attn.py:187-193).  The long kernel moves K,
    V and table rows in 16-byte chunks: K must then be 16-byte aligned and
    table rows whole chunks (16-bit tables whose rows are not, e.g. head_dim
    72 at width 36, are widened to float32, which is exact)."""
    q = _kernel_layout(q, 8, 4)
    k = _kernel_layout(k, 16, 8) if long_kernel else _kernel_layout(k, 8, 4)
    v = _kernel_layout(v, 16, 8)
    if cos.dtype != sin.dtype:
        # One table dtype per call: widening bf16/f16 to fp32 is exact.
        cos, sin = cos.float(), sin.float()
    if long_kernel and (cos.shape[1] * cos.element_size()) % 16:
        cos, sin = cos.float(), sin.float()
    ra = 16 if (cos.dtype == torch.float32 or long_kernel) else 8
    sm = 16 // cos.element_size() if long_kernel else 4
    if not (_fits(cos, ra, sm) and _fits(sin, ra, sm) and cos.stride(0) == sin.stride(0)):
        cos, sin = cos.contiguous(), sin.contiguous()
    return q, k, v, cos, sin


def _workspace_bytes(lib, args) -> int:
    """Bytes of the long kernel's optional workspace: rotated K and the split
    scratch (0 for the window kernel)."""
    total = ctypes.c_int64(0)
    _lib.check(lib.fra_workspace_bytes(args, ctypes.byref(total)))
    return int(total.value)


def plan(q, k, v, cos, sin, cu_seqlens, max_seqlen: int, softmax_scale=None) -> dict:
    """Which kernel ``fused_rope_attention`` launches for these inputs
    (no launch): ``{"kernel", "name", "grid", "block", "block_q",
    "block_kv", "lds_bytes", ...}``; for a head_dim without kernels of its
    own, the plan of the zero-padded call that runs instead."""
    d = q.shape[2]
    dp = _kernel_head_dim(d)
    if dp != d:
        scale = d ** -0.5 if softmax_scale is None else softmax_scale
        return plan(_pad_halves(q, d, dp), _pad_halves(k, d, dp), _pad_tail(v, d, dp), _pad_table(cos, d, dp),
                    _pad_table(sin, d, dp), cu_seqlens, max_seqlen, scale)
    cu = _prepare_cu(cu_seqlens, q.device)
    q2, k2, v2, cos2, sin2 = _prepare(q, k, v, cos, sin, _uses_long_kernel(int(max_seqlen), q.shape[2]))
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    scale = q.shape[2] ** -0.5 if softmax_scale is None else softmax_scale
    a = _build_args(q2, k2, v2, cos2, sin2, out, cu, max_seqlen, scale)
    lib = _lib.load()
    a.workspace_bytes = _workspace_bytes(lib, a)  # as fused_rope_attention provides it
    pl = _lib.Plan()
    _lib.check(lib.fra_query_plan(a, pl))
    return {"kernel": {_lib.FRA_KERNEL_WINDOW: "window", _lib.FRA_KERNEL_LONG: "long"}.get(pl.kernel, "none"),
            "name": pl.name.decode(), "grid": pl.grid, "block": pl.block, "block_q": pl.block_q,
            "block_kv": pl.block_kv, "lds_bytes": pl.lds_bytes, "workspace_bytes": a.workspace_bytes,
            "split_units": pl.split_units, "split_parts": pl.split_parts}


def fused_rope_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: "int | None" = None,
    softmax_scale: "float | None" = None,
    *,
    out: "torch.Tensor | None" = None,
    row_index: "torch.Tensor | None" = None,
) -> torch.Tensor:
    """Fused split-half RoPE on Q and K + non-causal attention over packed
    segments (reference fused_attn.py:139-232).

    Shapes:
      - q, k, v: ``[total_seq, num_heads, head_dim]``, float16 or bfloat16;
        any outer strides with a contiguous last dim are read in place.
      - cos, sin: ``[total_seq, head_dim // 2]`` (reference layout) or
        ``[total_seq, head_dim]`` (HF ``cat(emb, emb)`` layout); float32,
        bfloat16 or float16.
      - cu_seqlens: ``[num_segments + 1]`` cumulative token offsets (any int
        dtype; converted to int32 on q's device).
      - max_seqlen: longest segment.  ``None`` computes it on the device and
        synchronises once (as the reference always does); passing it keeps
        the call free of host synchronisation (graph-capturable).
      - softmax_scale: defaults to ``head_dim ** -0.5``.
      - out: optional ``[total_seq, num_heads, head_dim]`` result buffer.
      - row_index: optional ``[total_seq]`` integer tensor (beyond the
        reference): the window shuffle fused into the kernel's addressing.
        q, k, v, cos, sin and out stay in image order; ``cu_seqlens``
        describes the windows over window-order slots and slot i uses row
        ``row_index[i]`` (``utils.window_row_index``).  Window layers only
        (segments of at most 64 tokens, head_dim <= 96); forward only.

    Rows outside every segment are left unwritten, as in the reference.
    Returns ``out``.
    """
    _validate(q, k, v, cos, sin, cu_seqlens, out)
    rows = _prepare_rows(row_index, q)
    cu = _prepare_cu(cu_seqlens, q.device)
    if max_seqlen is None:
        max_seqlen = int((cu[1:] - cu[:-1]).max().item())
    max_seqlen = int(max_seqlen)
    scale = q.shape[2] ** -0.5 if softmax_scale is None else float(softmax_scale)
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        if out is not None:
            raise RuntimeError("fused_rope_attention(): out= does not support automatic differentiation "
                               "(q, k or v requires grad)")
        if rows is not None:
            raise RuntimeError("fused_rope_attention(): row_index is forward only (q, k or v requires grad)")
        return torch.ops.fused_rope_attn_amd.fwd(q, k, v, cos, sin, cu, max_seqlen, scale, True)[0]
    if torch.compiler.is_compiling() and rows is None:
        # traced (torch.compile / export): through the custom ops
        if out is None:
            return torch.ops.fused_rope_attn_amd.fwd(q, k, v, cos, sin, cu, max_seqlen, scale, False)[0]
        torch.ops.fused_rope_attn_amd.fwd_out(q, k, v, cos, sin, cu, max_seqlen, scale, out)
        return out
    # eager: straight to the library (the dispatcher round trip of a custom
    # op costs host time a back-to-back stream of layers then waits on)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    return _forward(q, k, v, cos, sin, cu, max_seqlen, scale, out, None, rows)


def _prepare_rows(row_index, q):
    """``row_index`` as contiguous int32 on q's device (None stays None)."""
    if row_index is None:
        return None
    if row_index.ndim != 1 or row_index.numel() != q.shape[0]:
        raise ValueError(f"row_index must be [total_seq]={q.shape[0],}, got {tuple(row_index.shape)}")
    if row_index.dtype.is_floating_point or row_index.dtype.is_complex or row_index.dtype == torch.bool:
        raise ValueError(f"row_index must have an integer dtype, got {row_index.dtype}")
    return row_index.to(device=q.device, dtype=torch.int32).contiguous()


def _forward(q, k, v, cos, sin, cu, max_seqlen: int, scale: float, out, lse, rows=None):
    """One forward launch into ``out`` (and ``lse`` if given, [heads, tokens]
    fp32); inputs already validated, ``cu`` int32 on q's device; ``rows``
    the optional int32 row gather."""
    if max_seqlen <= 0 or q.shape[0] == 0:
        if lse is not None:
            lse.fill_(float("-inf"))
        return out.zero_()
    d = q.shape[2]
    dp = _kernel_head_dim(d)
    if dp != d:
        # The padded output starts as a copy of ``out`` so that rows outside
        # every segment come back unchanged.
        outp = _pad_tail(out, d, dp)
        _forward(_pad_halves(q, d, dp), _pad_halves(k, d, dp), _pad_tail(v, d, dp), _pad_table(cos, d, dp),
                 _pad_table(sin, d, dp), cu, max_seqlen, scale, outp, lse, rows)
        return out.copy_(outp[..., :d])
    if rows is not None and _uses_long_kernel(max_seqlen, d):
        raise ValueError(f"row_index is for window layers (segments of at most 64 tokens, head_dim <= 96), "
                         f"got max_seqlen={max_seqlen}, head_dim={d}")
    qk, kk, vk, cosk, sink = _prepare(q, k, v, cos, sin, _uses_long_kernel(max_seqlen, q.shape[2]))
    dst = out if _fits(out, 8, 4) else torch.empty(q.shape, dtype=q.dtype, device=q.device)

    lib = _lib.load()
    args = _build_args(qk, kk, vk, cosk, sink, dst, cu, max_seqlen, scale)
    if lse is not None:
        args.lse = lse.data_ptr()
    ws = None
    with _on_device(q.device):
        # The long kernel's workspace (scratch, per call, from torch's
        # caching allocator: stream-ordered reuse keeps it alive for the
        # kernels that use it) holds K rotated once per call and, where a
        # partly filled last round of workgroups is split along the key
        # range, the parts' partial rows.  The window kernel takes none.
        nbytes = _workspace_bytes(lib, args) if _uses_long_kernel(max_seqlen, d) else 0
        if nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
            args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
        stream = _raw_stream(q.device)
        if rows is not None:
            _lib.check(lib.fra_fwd_varlen_gather(args, None, rows.data_ptr(), stream))
        else:
            _lib.check(lib.fra_fwd_varlen(args, stream))
    if dst is not out:
        out.copy_(dst)
    return out


def fused_rope_attention_fwd(q, k, v, cos, sin, cu_seqlens, max_seqlen=None, softmax_scale=None, *, out=None):
    """Forward with the softmax statistics: returns ``(out, lse)``, where
    ``lse[h, t] = log(sum_j exp(softmax_scale * q_rot[t, h] . k_rot[j, h]))``
    over the keys of t's segment (float32, ``[num_heads, total_seq]``; the
    natural-log convention of flash-attn's varlen ``softmax_lse``).  Entries
    of rows outside every segment are unspecified.  No counterpart in the
    reference, which keeps these statistics in registers
    (fused_attn.py:347-355, 398-405)."""
    _validate(q, k, v, cos, sin, cu_seqlens, out)
    cu = _prepare_cu(cu_seqlens, q.device)
    if max_seqlen is None:
        max_seqlen = int((cu[1:] - cu[:-1]).max().item())
    scale = q.shape[2] ** -0.5 if softmax_scale is None else float(softmax_scale)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((q.shape[1], q.shape[0]), dtype=torch.float32, device=q.device)
    _forward(q, k, v, cos, sin, cu, int(max_seqlen), scale, out, lse)
    return out, lse


def _bwd_layout(t: torch.Tensor) -> torch.Tensor:
    return _kernel_layout(t, 16, 8)


def _bwd_args(dout, q, k, v, cos, sin, out, lse, cu, max_seqlen: int, scale: float, dq, dk, dv):
    """``fra_bwd_args`` of one backward call, and the tensors it points to
    (kept alive by the caller until the launch)."""
    q2, k2, v2, o2, do2 = (_bwd_layout(t) for t in (q, k, v, out, dout))
    # The backward reads float32 tables (widening is exact).
    cos2 = cos.float().contiguous()
    sin2 = sin.float().contiguous()
    lse2 = lse.contiguous()
    a = _lib.BwdArgs()
    for name, t in (("q", q2), ("k", k2), ("v", v2), ("out", o2), ("dout", do2), ("dq", dq), ("dk", dk), ("dv", dv)):
        setattr(a, name, t.data_ptr())
        setattr(a, f"{name}_stride_seq", t.stride(0))
        setattr(a, f"{name}_stride_head", t.stride(1))
    a.cos, a.sin, a.lse, a.cu_seqlens = cos2.data_ptr(), sin2.data_ptr(), lse2.data_ptr(), cu.data_ptr()
    a.rope_stride_seq = cos2.stride(0)
    a.total_seq, a.num_heads, a.head_dim = q.shape
    a.num_seqs = cu.numel() - 1
    a.max_seqlen = int(max_seqlen)
    a.rope_width = cos2.shape[1]
    a.qkv_dtype = _QKV_CODE[q.dtype]
    a.rope_dtype = _lib.FRA_DTYPE_F32
    a.softmax_scale = float(scale)
    a.flags = 0
    return a, (q2, k2, v2, o2, do2, cos2, sin2, lse2)


def backward_plan(q, k, v, cos, sin, cu_seqlens, max_seqlen: int) -> dict:
    """Which main kernel the backward of these inputs launches (no launch):
    ``{"kernel", "name", "grid", "block"}``; for a head_dim without kernels
    of its own, the plan of the zero-padded call that runs instead."""
    d = q.shape[2]
    dp = _kernel_head_dim(d)
    if dp != d:
        return backward_plan(_pad_halves(q, d, dp), _pad_halves(k, d, dp), _pad_tail(v, d, dp),
                             _pad_table(cos, d, dp), _pad_table(sin, d, dp), cu_seqlens, max_seqlen)
    cu = _prepare_cu(cu_seqlens, q.device)
    z = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((q.shape[1], q.shape[0]), dtype=torch.float32, device=q.device)
    a, _keep = _bwd_args(z, q, k, v, cos, sin, z, lse, cu, max_seqlen, q.shape[2] ** -0.5, z, z, z)
    pl = _lib.Plan()
    _lib.check(_lib.load().fra_bwd_query_plan(a, pl))
    return {"kernel": {_lib.FRA_KERNEL_WINDOW: "window", _lib.FRA_KERNEL_LONG: "long"}.get(pl.kernel, "none"),
            "name": pl.name.decode(), "grid": pl.grid, "block": pl.block}


def _backward(dout, q, k, v, cos, sin, out, lse, cu, max_seqlen: int, scale: float, dq, dk, dv):
    """One backward launch (``fra_bwd_varlen``) writing dq, dk, dv."""
    if max_seqlen <= 0 or q.shape[0] == 0:
        return dq, dk, dv
    d = q.shape[2]
    dp = _kernel_head_dim(d)
    if dp != d:
        dqp, dkp, dvp = _pad_halves(dq, d, dp), _pad_halves(dk, d, dp), _pad_tail(dv, d, dp)
        _backward(_pad_tail(dout, d, dp), _pad_halves(q, d, dp), _pad_halves(k, d, dp), _pad_tail(v, d, dp),
                  _pad_table(cos, d, dp), _pad_table(sin, d, dp), _pad_tail(out, d, dp), lse, cu, max_seqlen,
                  scale, dqp, dkp, dvp)
        dq.copy_(_unpad_halves(dqp, d, dp))
        dk.copy_(_unpad_halves(dkp, d, dp))
        dv.copy_(dvp[..., :d])
        return dq, dk, dv
    lib = _lib.load()
    dsts = [t if _fits(t, 16, 8) else torch.empty(q.shape, dtype=q.dtype, device=q.device) for t in (dq, dk, dv)]
    a, _keep = _bwd_args(dout, q, k, v, cos, sin, out, lse, cu, max_seqlen, scale, *dsts)
    with _on_device(q.device):
        nbytes = ctypes.c_int64(0)
        _lib.check(lib.fra_bwd_workspace_bytes(a, ctypes.byref(nbytes)))
        ws = torch.empty(max(int(nbytes.value), 16), dtype=torch.uint8, device=q.device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        _lib.check(lib.fra_bwd_varlen(a, _raw_stream(q.device)))
    for dst, t in zip(dsts, (dq, dk, dv)):
        if dst is not t:
            t.copy_(dst)
    return dq, dk, dv


def fused_rope_attention_bwd(dout, q, k, v, cos, sin, out, lse, cu_seqlens, max_seqlen=None, softmax_scale=None,
                             *, dq=None, dk=None, dv=None):
    """Gradients ``(dq, dk, dv)`` of ``fused_rope_attention`` given ``dout``
    and the forward's ``out`` and ``lse`` (from ``fused_rope_attention_fwd``
    with the same inputs).  cos/sin get no gradient.  Rows outside every
    segment of freshly allocated results are zero.  No counterpart in the
    reference (forward-only); the arithmetic is the derivative of its kernel
    (fused_attn.py:316-423), with the rotation's rounding taken as the
    identity."""
    _validate(q, k, v, cos, sin, cu_seqlens, out)
    if dout.shape != q.shape or dout.dtype != q.dtype or dout.device != q.device:
        raise ValueError(f"dout must match q shape/dtype/device, got {tuple(dout.shape)} {dout.dtype} {dout.device}")
    if lse.shape != (q.shape[1], q.shape[0]) or lse.dtype != torch.float32:
        raise ValueError(f"lse must be float32 [num_heads, total_seq]={q.shape[1], q.shape[0]}, "
                         f"got {tuple(lse.shape)} {lse.dtype}")
    cu = _prepare_cu(cu_seqlens, q.device)
    if max_seqlen is None:
        max_seqlen = int((cu[1:] - cu[:-1]).max().item())
    scale = q.shape[2] ** -0.5 if softmax_scale is None else float(softmax_scale)
    dq = torch.zeros_like(q, memory_format=torch.contiguous_format) if dq is None else dq
    dk = torch.zeros_like(k, memory_format=torch.contiguous_format) if dk is None else dk
    dv = torch.zeros_like(v, memory_format=torch.contiguous_format) if dv is None else dv
    return _backward(dout, q, k, v, cos, sin, out, lse, cu, int(max_seqlen), scale, dq, dk, dv)


# ---------------------------------------------------------------------------
# torch.library registration: the op as custom ops with fake (meta)
# implementations and an autograd formula, so that torch.compile and
# torch.export trace through it (the ctypes call is opaque to them).
# ---------------------------------------------------------------------------

@torch.library.custom_op("fused_rope_attn_amd::fwd", mutates_args=(), device_types="cuda")
def _fwd_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
            cu: torch.Tensor, max_seqlen: int, scale: float, with_lse: bool) -> "tuple[torch.Tensor, torch.Tensor]":
    """Forward into a fresh ``out`` (and ``lse`` [heads, tokens] fp32 when
    ``with_lse``; else an empty tensor).  Inputs validated by the caller."""
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((q.shape[1], q.shape[0]) if with_lse else (0,), dtype=torch.float32, device=q.device)
    _forward(q, k, v, cos, sin, cu, max_seqlen, scale, out, lse if with_lse else None)
    return out, lse


@_fwd_op.register_fake
def _fwd_fake(q, k, v, cos, sin, cu, max_seqlen, scale, with_lse):
    return (q.new_empty(q.shape),
            q.new_empty((q.shape[1], q.shape[0]) if with_lse else (0,), dtype=torch.float32))


@torch.library.custom_op("fused_rope_attn_amd::fwd_out", mutates_args=("out",), device_types="cuda")
def _fwd_out_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                cu: torch.Tensor, max_seqlen: int, scale: float, out: torch.Tensor) -> None:
    """Forward into the caller's ``out`` (rows outside every segment keep
    their contents)."""
    _forward(q, k, v, cos, sin, cu, max_seqlen, scale, out, None)


@_fwd_out_op.register_fake
def _fwd_out_fake(q, k, v, cos, sin, cu, max_seqlen, scale, out):
    return None


@torch.library.custom_op("fused_rope_attn_amd::bwd", mutates_args=(), device_types="cuda")
def _bwd_op(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
            sin: torch.Tensor, out: torch.Tensor, lse: torch.Tensor, cu: torch.Tensor, max_seqlen: int,
            scale: float) -> "tuple[torch.Tensor, torch.Tensor, torch.Tensor]":
    """Gradients of ``fwd`` (zero in rows outside every segment).  Has no
    autograd formula itself: a double backward raises."""
    dq = torch.zeros(q.shape, dtype=q.dtype, device=q.device)
    dk = torch.zeros(q.shape, dtype=q.dtype, device=q.device)
    dv = torch.zeros(q.shape, dtype=q.dtype, device=q.device)
    _backward(dout, q, k, v, cos, sin, out, lse, cu, max_seqlen, scale, dq, dk, dv)
    return dq, dk, dv


@_bwd_op.register_fake
def _bwd_fake(dout, q, k, v, cos, sin, out, lse, cu, max_seqlen, scale):
    return q.new_empty(q.shape), q.new_empty(q.shape), q.new_empty(q.shape)


def _fwd_setup_context(ctx, inputs, output):
    q, k, v, cos, sin, cu, max_seqlen, scale, _with_lse = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, cos, sin, out, lse, cu)
    ctx.max_seqlen, ctx.scale = max_seqlen, scale
    ctx.mark_non_differentiable(lse)


def _fwd_backward(ctx, dout, _dlse):
    """cos/sin and cu_seqlens get no gradient."""
    q, k, v, cos, sin, out, lse, cu = ctx.saved_tensors
    dq, dk, dv = torch.ops.fused_rope_attn_amd.bwd(dout, q, k, v, cos, sin, out, lse, cu, ctx.max_seqlen, ctx.scale)
    return dq, dk, dv, None, None, None, None, None, None


_fwd_op.register_autograd(_fwd_backward, setup_context=_fwd_setup_context)


# ---------------------------------------------------------------------------
# RoPE from positions (beyond the reference: compute_rope_2d's table is never
# built; the kernels compute its angles, cosines and sines in registers)
# ---------------------------------------------------------------------------

def rope_positions_2d(grid_thw, head_dim: int, spatial_merge_size: int, theta: float, device,
                      window_idx: "torch.Tensor | None" = None):
    """``(pos, inv_freq)`` for ``fused_rope_attention_pos``: ``pos`` int32
    ``[total_seq, 2]`` holds the (h, w) patch position of every row of
    ``compute_rope_2d``'s tables (merge-block order, ``t`` repeats, the
    ``window_idx`` reorder), ``inv_freq`` float32 ``[head_dim // 4]`` is
    ``1/theta**(arange(0, D/2, 2)/(D/2))``.  Row t of the table is then
    ``[pos[t, 0] * inv_freq || pos[t, 1] * inv_freq]`` (reference
    fused_attn.py:78-116)."""
    assert head_dim > 0 and head_dim % 4 == 0, f"head_dim must be divisible by 4, got {head_dim}"
    rd = head_dim // 2
    merge = int(spatial_merge_size)
    device = torch.device(device)
    if isinstance(grid_thw, torch.Tensor):
        thw = [tuple(int(x) for x in row) for row in grid_thw.detach().cpu().tolist()]
    else:
        thw = [(int(t), int(h), int(w)) for t, h, w in grid_thw]
    inv = 1.0 / (theta ** (torch.arange(0, rd, 2, device=device, dtype=torch.float32) / rd))
    hs, ws = [], []
    for t, h, w in thw:
        hp, wp = _merge_order(h, w, merge, device)
        hs.append(hp.repeat(t))
        ws.append(wp.repeat(t))
    pos = torch.stack([torch.cat(hs), torch.cat(ws)], dim=1).to(torch.int32)
    if window_idx is not None:
        mu = merge * merge
        widx = window_idx.to(device=device, dtype=torch.long)
        pos = pos.view(-1, mu, 2).index_select(0, widx).reshape(-1, 2)
    return pos.contiguous(), inv.contiguous()


def _validate_pos(q, k, v, pos, inv_freq, cu_seqlens, out) -> None:
    """The op's checks with the tables replaced by positions."""
    if q.device.type != "cuda":
        raise ValueError(f"q must be on CUDA, got device={q.device}")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q/k/v must have same shape, got q={tuple(q.shape)} k={tuple(k.shape)} v={tuple(v.shape)}")
    if q.ndim != 3:
        raise ValueError(f"q/k/v must be [total_seq, num_heads, head_dim], got q.ndim={q.ndim}")
    total_seq, head_dim = int(q.shape[0]), int(q.shape[2])
    if head_dim <= 0 or head_dim % 4 != 0:
        raise ValueError(f"head_dim must be positive and divisible by 4 for rope positions, got {head_dim}")
    if not _lib.load().fra_supports_head_dim(head_dim):
        raise ValueError(f"head_dim={head_dim} has no kernel in this build of libfra.so (rope positions run "
                         f"only at compiled head dims)")
    if tuple(pos.shape) != (total_seq, 2):
        raise ValueError(f"pos must be [total_seq, 2]={total_seq, 2}, got {tuple(pos.shape)}")
    if pos.dtype.is_floating_point or pos.dtype.is_complex or pos.dtype == torch.bool:
        raise ValueError(f"pos must have an integer dtype, got {pos.dtype}")
    if tuple(inv_freq.shape) != (head_dim // 4,):
        raise ValueError(f"inv_freq must be [head_dim//4]={head_dim // 4,}, got {tuple(inv_freq.shape)}")
    if inv_freq.dtype != torch.float32:
        raise ValueError(f"inv_freq must be float32, got {inv_freq.dtype}")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError(f"cu_seqlens must be 1D with length >= 2, got {tuple(cu_seqlens.shape)}")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"q dtype must be float16 or bfloat16, got {q.dtype}")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"q/k/v must share dtype, got q={q.dtype} k={k.dtype} v={v.dtype}")
    if out is not None:
        if out.shape != q.shape:
            raise ValueError(f"out must have shape {tuple(q.shape)}, got {tuple(out.shape)}")
        if out.dtype != q.dtype or out.device != q.device:
            raise ValueError(f"out must match q dtype/device, got out={out.dtype}/{out.device} q={q.dtype}/{q.device}")
    for name, t in (("k", k), ("v", v), ("pos", pos), ("inv_freq", inv_freq)):
        if t.device != q.device:
            raise ValueError(f"{name} must be on {q.device}, got {t.device}")


def _pos_args(q, k, v, pos, inv_freq, out, cu, max_seqlen: int, scale: float):
    """(FwdArgs, RopePositions, kept tensors) of one position call."""
    qk, kk, vk = _prepare_qkv(q, k, v, _uses_long_kernel(max_seqlen, q.shape[2]))
    pos = pos.to(dtype=torch.int32).contiguous()
    inv_freq = inv_freq.contiguous()
    a = _lib.FwdArgs()
    a.q, a.k, a.v, a.out = qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), out.data_ptr()
    a.cos = a.sin = None
    a.cu_seqlens = cu.data_ptr()
    a.q_stride_seq, a.q_stride_head = qk.stride(0), qk.stride(1)
    a.k_stride_seq, a.k_stride_head = kk.stride(0), kk.stride(1)
    a.v_stride_seq, a.v_stride_head = vk.stride(0), vk.stride(1)
    a.out_stride_seq, a.out_stride_head = out.stride(0), out.stride(1)
    a.rope_stride_seq = 0
    a.total_seq, a.num_heads, a.head_dim = q.shape
    a.num_seqs = cu.numel() - 1
    a.max_seqlen = int(max_seqlen)
    a.rope_width = q.shape[2] // 2
    a.qkv_dtype = _QKV_CODE[q.dtype]
    a.rope_dtype = _lib.FRA_DTYPE_F32
    a.softmax_scale = float(scale)
    a.flags = 0
    rope = _lib.RopePositions(pos.data_ptr(), inv_freq.data_ptr())
    return a, rope, (qk, kk, vk, pos, inv_freq)


def _prepare_qkv(q, k, v, long_kernel: bool):
    q = _kernel_layout(q, 8, 4)
    k = _kernel_layout(k, 16, 8) if long_kernel else _kernel_layout(k, 8, 4)
    v = _kernel_layout(v, 16, 8)
    return q, k, v


def plan_pos(q, k, v, pos, inv_freq, cu_seqlens, max_seqlen: int, softmax_scale=None) -> dict:
    """``plan`` of a ``fused_rope_attention_pos`` call (no launch)."""
    cu = _prepare_cu(cu_seqlens, q.device)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    scale = q.shape[2] ** -0.5 if softmax_scale is None else softmax_scale
    a, rope, _keep = _pos_args(q, k, v, pos, inv_freq, out, cu, max_seqlen, scale)
    lib = _lib.load()
    nbytes = ctypes.c_int64(0)
    _lib.check(lib.fra_workspace_bytes_pos(a, rope, ctypes.byref(nbytes)))
    a.workspace_bytes = int(nbytes.value)
    pl = _lib.Plan()
    _lib.check(lib.fra_query_plan_pos(a, rope, pl))
    return {"kernel": {_lib.FRA_KERNEL_WINDOW: "window", _lib.FRA_KERNEL_LONG: "long"}.get(pl.kernel, "none"),
            "name": pl.name.decode(), "grid": pl.grid, "block": pl.block, "lds_bytes": pl.lds_bytes,
            "workspace_bytes": a.workspace_bytes, "split_units": pl.split_units, "split_parts": pl.split_parts}


def fused_rope_attention_pos(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    pos: torch.Tensor,
    inv_freq: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: "int | None" = None,
    softmax_scale: "float | None" = None,
    *,
    out: "torch.Tensor | None" = None,
    row_index: "torch.Tensor | None" = None,
) -> torch.Tensor:
    """``fused_rope_attention`` with the rotation computed from positions:
    for token t, ``cos``/``sin`` row t of ``compute_rope_2d`` is evaluated in
    the kernels as ``cos/sin([pos[t, 0] * inv_freq || pos[t, 1] *
    inv_freq])`` (fp32 products, the device library's sincosf), so no table
    is built or read.  ``pos`` and ``inv_freq`` come from
    ``rope_positions_2d`` with the arguments ``compute_rope_2d`` would take.
    Forward only; head_dim must be a multiple of 4 with its own kernels.
    ``row_index`` as in ``fused_rope_attention`` (``pos`` then in image
    order too).  Returns ``out``."""
    _validate_pos(q, k, v, pos, inv_freq, cu_seqlens, out)
    rows = _prepare_rows(row_index, q)
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        raise RuntimeError("fused_rope_attention_pos() is forward only; use fused_rope_attention with "
                           "compute_rope_2d tables for gradients")
    cu = _prepare_cu(cu_seqlens, q.device)
    if max_seqlen is None:
        max_seqlen = int((cu[1:] - cu[:-1]).max().item())
    max_seqlen = int(max_seqlen)
    scale = q.shape[2] ** -0.5 if softmax_scale is None else float(softmax_scale)
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if max_seqlen <= 0 or q.shape[0] == 0:
        return out.zero_()
    dst = out if _fits(out, 8, 4) else torch.empty(q.shape, dtype=q.dtype, device=q.device)
    a, rope, _keep = _pos_args(q, k, v, pos, inv_freq, dst, cu, max_seqlen, scale)
    lib = _lib.load()
    ws = None
    with _on_device(q.device):
        nbytes = ctypes.c_int64(0)
        _lib.check(lib.fra_workspace_bytes_pos(a, rope, ctypes.byref(nbytes)))
        if nbytes.value:
            ws = torch.empty(int(nbytes.value), dtype=torch.uint8, device=q.device)
            a.workspace, a.workspace_bytes = ws.data_ptr(), int(nbytes.value)
        stream = _raw_stream(q.device)
        if rows is not None:
            if _uses_long_kernel(max_seqlen, q.shape[2]):
                raise ValueError(f"row_index is for window layers (segments of at most 64 tokens, head_dim <= "
                                 f"96), got max_seqlen={max_seqlen}, head_dim={q.shape[2]}")
            _lib.check(lib.fra_fwd_varlen_gather(a, rope, rows.data_ptr(), stream))
        else:
            _lib.check(lib.fra_fwd_varlen_pos(a, rope, stream))
    if dst is not out:
        out.copy_(dst)
    return out
