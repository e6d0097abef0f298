"""The allocation-free forward entry point ``fra_fwd_varlen_static``
(include/fra.h; no counterpart in the reference) against
``fra_fwd_varlen`` with a workspace, both called through the C ABI.

The two share their kernels; the static entry point rotates K inside the
long kernel (the workspace path rotates it once per call into the
workspace, which gives bit-identical rotated values) and keeps a split last
round's partial rows in the library's static device array.  So the outputs
and the log-sum-exp must agree bit for bit.  Two calls in a row: the first
with a split needing 22 MB of scratch, the second with a smaller one (2.8
MB), which must not see the first call's leftovers; a third at head_dim 72;
then a window layer (no scratch).
"""
import ctypes

import numpy as np
import pytest
import torch

from fused_rope_attn_amd import _lib
from fused_rope_attn_amd.fused_attn import _build_args

pytestmark = pytest.mark.gpu


def _case(device, lens, h, d, seed):
    g = torch.Generator().manual_seed(seed)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32)
    n = int(cu[-1])
    q, k, v = (torch.randn(n, h, d, generator=g).to(torch.bfloat16).to(device) for _ in range(3))
    ang = torch.rand(n, d // 2, generator=g) * 6.0
    return q, k, v, ang.cos().to(device), ang.sin().to(device), cu.to(device), max(lens)


def _run(lib, device, case, static):
    q, k, v, cos, sin, cu, ms = case
    out = torch.full(q.shape, float("nan"), dtype=q.dtype, device=device)
    lse = torch.full((q.shape[1], q.shape[0]), float("nan"), dtype=torch.float32, device=device)
    a = _build_args(q, k, v, cos, sin, out, cu, ms, q.shape[2] ** -0.5)
    a.lse = lse.data_ptr()
    stream = torch.cuda.current_stream(device).cuda_stream
    ws = None
    pl = _lib.Plan()
    if static:
        rc = lib.fra_fwd_varlen_static(ctypes.byref(a), stream)
    else:
        nbytes = ctypes.c_int64(0)
        _lib.check(lib.fra_workspace_bytes(ctypes.byref(a), ctypes.byref(nbytes)))
        ws = torch.empty(max(int(nbytes.value), 16), dtype=torch.uint8, device=device)
        a.workspace, a.workspace_bytes = ws.data_ptr(), int(nbytes.value)
        _lib.check(lib.fra_query_plan(ctypes.byref(a), ctypes.byref(pl)))
        rc = lib.fra_fwd_varlen(ctypes.byref(a), stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return out, lse, pl


def test_static_entry_point_matches_workspace_entry_point(device):
    lib = _lib.load()
    cases = [
        # one 9216-token segment x 16 heads: 576 units, the last 64 split in 4 parts (22 MB of scratch)
        ([9216], 16, 80, 1, 4),
        # one 1024-token segment x 4 heads: 16 units split in 2 parts (2.8 MB)
        ([1024], 4, 80, 2, 2),
        # ragged long segments at head_dim 72 (48 units, split in 3 parts)
        ([700, 3, 64, 1500], 2, 72, 3, 3),
    ]
    for lens, h, d, seed, parts in cases:
        print(f"static vs workspace: lens={lens} heads={h} head_dim={d}", flush=True)
        case = _case(device, lens, h, d, seed)
        o_ws, l_ws, pl = _run(lib, device, case, static=False)
        o_st, l_st, _ = _run(lib, device, case, static=True)
        if torch.cuda.get_device_properties(device).multi_processor_count == 256:
            assert pl.split_parts == parts, (lens, pl.split_parts)  # the scratch is in use
        assert not torch.isnan(o_ws.float()).any()
        assert torch.equal(o_st, o_ws), (lens, float((o_st.float() - o_ws.float()).abs().max()))
        assert torch.equal(l_st, l_ws), (lens, float((l_st - l_ws).abs().max()))


def test_static_entry_point_window_layer(device):
    # window layers use no scratch: the static entry point runs the same launch
    lib = _lib.load()
    case = _case(device, [64, 64, 17], 4, 80, 5)
    o_ws, l_ws, _ = _run(lib, device, case, static=False)
    o_st, l_st, _ = _run(lib, device, case, static=True)
    assert torch.equal(o_st, o_ws) and torch.equal(l_st, l_ws)
