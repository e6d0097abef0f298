"""Parity of the HIP path (libfra.so through fused_rope_attention) with the
CPU oracle on the same seeded inputs.

Bar (north star): per call in bf16, max-abs error <= 2e-2 and mean-abs error
<= 2e-3 against the unfused path evaluated in fp32 (oracle mode "fp32").  A
second, tighter check compares with the oracle that rounds where the kernel
rounds (Q_rot/K_rot and P to the input dtype): max-abs <= 8e-3,
mean-abs <= 5e-4.  At full BASELINE sizes the oracle covers a subset of heads
and a size-independent property (head permutation) covers the rest.
"""
import math

import numpy as np
import pytest
import torch

from fused_rope_attn_amd import _lib, fused_rope_attention, plan
from fused_rope_attn_amd.configs import WORKLOADS, make_inputs
from oracle import attention as A

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 2e-3            # vs fp32 unfused path (north star)
EMU_MAX_ABS, EMU_MEAN_ABS = 8e-3, 5e-4    # vs the rounding-point model of the kernel


def f32(t):
    return t.detach().float().cpu().numpy()


def assert_close(out, ref, max_abs, mean_abs, what=""):
    covered = ~np.isnan(ref)
    assert covered.any()
    err = np.abs(out[covered] - ref[covered])
    assert np.isfinite(out[covered]).all(), f"{what}: non-finite output"
    mx, mn = float(err.max()), float(err.mean())
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3e} (<= {max_abs}), mean-abs {mn:.3e} (<= {mean_abs})"


def random_case(lens, h, d, seed, dtype=torch.bfloat16, rope_dtype=torch.float32, width=None, extra_rows=0):
    """Segments of the given lengths (0 allowed), random angles per token."""
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    n = int(cu[-1]) + extra_rows
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(n, h, d, generator=g) for _ in range(3))
    half = d // 2
    w = half if width is None else width
    ang = torch.rand(n, w, generator=g) * 2 * math.pi - math.pi
    cos, sin = ang.cos().to(rope_dtype), ang.sin().to(rope_dtype)
    return {"q": q.to(dtype), "k": k.to(dtype), "v": v.to(dtype), "cos": cos, "sin": sin,
            "cu_seqlens": torch.from_numpy(cu), "max_seqlen": int(max(lens)) if lens else 0}


def run_gpu(case, device, **kw):
    args = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in case.items()}
    out = fused_rope_attention(args["q"], args["k"], args["v"], args["cos"], args["sin"], args["cu_seqlens"],
                               kw.pop("max_seqlen", args["max_seqlen"]), **kw)
    torch.cuda.synchronize()
    return out


def oracle(case, mode="fp32", heads=None, scale=None):
    q, k, v = f32(case["q"]), f32(case["k"]), f32(case["v"])
    if heads is not None:
        q, k, v = q[:, heads], k[:, heads], v[:, heads]
    return A.fused_rope_attention(q, k, v, f32(case["cos"]), f32(case["sin"]), case["cu_seqlens"].numpy(),
                                  softmax_scale=scale, mode=mode)


def emu_mode(dtype):
    return "bf16" if dtype == torch.bfloat16 else "f16"


# --- window kernel: every segment <= 64 tokens ------------------------------

WINDOW_LENS = [
    [64, 64, 64],
    [1, 4, 12, 16, 49, 56, 63, 64],
    [0, 64, 0, 0, 33, 0],          # empty segments
    [2, 31, 32, 33],
]


@pytest.mark.parametrize("heads", [None, 1, 2, 4])
@pytest.mark.parametrize("d", [64, 72, 80, 96])
@pytest.mark.parametrize("li", range(len(WINDOW_LENS)))
def test_window_kernel_ragged(device, d, li, heads, monkeypatch):
    # heads: the window kernel's form forced through FRA_WINDOW_HEADS (None:
    # the planner's choice, which for these few (segment, head) pairs is one
    # head per workgroup with its query tiles split over two wavefronts;
    # head_dim 72 has no such instance: the planner then takes two heads, a
    # forced one-head form four).  Three heads leave a partial last group in
    # the two-head form and a partial one in the four.
    if heads is not None:
        monkeypatch.setenv("FRA_WINDOW_HEADS", str(heads))
    lens = WINDOW_LENS[li]
    case = random_case(lens, h=3, d=d, seed=100 + li, extra_rows=5)
    pl = plan(*(case[x].to(device) for x in ("q", "k", "v", "cos", "sin", "cu_seqlens")), max_seqlen=case["max_seqlen"])
    assert pl["kernel"] == "window"
    form = heads if heads is not None else 1
    if form == 1 and d == 72:
        form = 4 if heads == 1 else 2
    assert pl["grid"] == len(lens) * -(-3 // form), (pl, form)
    out = f32(run_gpu(case, device))
    assert_close(out, oracle(case), MAX_ABS, MEAN_ABS, f"window d={d} lens={lens} heads={heads}")
    assert_close(out, oracle(case, "bf16"), EMU_MAX_ABS, EMU_MEAN_ABS, f"window d={d} lens={lens} heads={heads} (emulated)")


# --- long kernel --------------------------------------------------------------

LONG_LENS = [
    [65],
    [128, 129],
    [300, 1, 64, 0, 200],
    [1000],
]


@pytest.mark.parametrize("d", [64, 72, 80, 96, 128])
@pytest.mark.parametrize("li", range(len(LONG_LENS)))
def test_long_kernel_ragged(device, d, li):
    lens = LONG_LENS[li]
    case = random_case(lens, h=2, d=d, seed=200 + li, extra_rows=3)
    out = f32(run_gpu(case, device))
    assert_close(out, oracle(case), MAX_ABS, MEAN_ABS, f"long d={d} lens={lens}")
    assert_close(out, oracle(case, "bf16"), EMU_MAX_ABS, EMU_MEAN_ABS, f"long d={d} lens={lens} (emulated)")


@pytest.mark.parametrize("d", [72, 80])
@pytest.mark.parametrize("lens", [[320, 384], [448, 512], [1024, 321], [383, 640]])
def test_long_kernel_block_counts(device, d, lens):
    """Segments of 5 to 16 key blocks, full or partial last block: the
    steady loop runs through the second-to-last block when the last one is
    full (an even or odd number of its iterations), else stops three
    blocks earlier, and the generic loop takes the rest."""
    case = random_case(lens, h=2, d=d, seed=1500 + sum(lens) + d)
    print(f"long block counts lens={lens} head_dim={d}", flush=True)
    assert plan(*(case[k].to(device) for k in ("q", "k", "v", "cos", "sin", "cu_seqlens")),
                case["max_seqlen"])["kernel"] == "long"
    assert_close(f32(run_gpu(case, device)), oracle(case), MAX_ABS, MEAN_ABS, f"lens={lens} d={d}")


@pytest.mark.parametrize("d", [72, 80, 96, 128])
@pytest.mark.parametrize("rope_dtype", [torch.float32, torch.bfloat16])
def test_long_kernel_full_width_tables(device, d, rope_dtype):
    # width-head_dim tables: the long kernel stages twice the table bytes (one
    # raw buffer instead of two at d >= 96 with float32 tables); bf16 tables of
    # rows that are not whole 16-byte chunks are widened to float32 by the op.
    lens = [700, 63, 0, 129]
    case = random_case(lens, h=2, d=d, seed=250 + d, rope_dtype=rope_dtype, width=d)
    out = f32(run_gpu(case, device))
    assert_close(out, oracle(case), MAX_ABS, MEAN_ABS, f"long d={d} full-width {rope_dtype}")
    assert_close(out, oracle(case, "bf16"), EMU_MAX_ABS, EMU_MEAN_ABS, f"long d={d} full-width {rope_dtype} (emulated)")
    half = dict(case, cos=case["cos"][:, : d // 2].contiguous(), sin=case["sin"][:, : d // 2].contiguous())
    out_h = f32(run_gpu(half, device))
    assert_close(out_h, oracle(half), MAX_ABS, MEAN_ABS, f"long d={d} half-width {rope_dtype}")


def test_long_kernel_serves_short_segments(device):
    # max_seqlen above 64 routes every segment, short ones too, to the long kernel
    lens = [64, 5, 64, 17]
    case = random_case(lens, h=2, d=80, seed=300)
    out = f32(run_gpu(case, device, max_seqlen=200))
    assert_close(out, oracle(case), MAX_ABS, MEAN_ABS, "long kernel on short segments")
    win = f32(run_gpu(case, device))
    assert_close(win, out, 8e-3, 5e-4, "window vs long kernel")


# --- dtypes, table layouts, arguments -----------------------------------------

@pytest.mark.parametrize("lens", [[64, 40], [150, 7]])
def test_fp16(device, lens):
    case = random_case(lens, h=2, d=80, seed=400, dtype=torch.float16)
    out = run_gpu(case, device)
    assert out.dtype == torch.float16
    out = f32(out)
    assert_close(out, oracle(case), MAX_ABS, MEAN_ABS, "fp16")
    assert_close(out, oracle(case, "f16"), 4e-3, 2e-4, "fp16 (emulated)")


@pytest.mark.parametrize("rope_dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("full", [False, True])
@pytest.mark.parametrize("lens", [[64, 23], [130]])
def test_rope_table_dtypes_and_widths(device, rope_dtype, full, lens):
    d = 72
    case = random_case(lens, h=2, d=d, seed=500, rope_dtype=rope_dtype, width=d if full else d // 2)
    out = f32(run_gpu(case, device))
    assert_close(out, oracle(case), MAX_ABS, MEAN_ABS, f"rope {rope_dtype} full={full}")
    assert_close(out, oracle(case, "bf16"), EMU_MAX_ABS, EMU_MEAN_ABS, f"rope {rope_dtype} full={full} (emulated)")


def test_full_width_duplicated_tables_equal_half_width(device):
    case = random_case([64, 64, 100], h=2, d=80, seed=501)
    a = run_gpu(case, device)
    full = dict(case, cos=torch.cat([case["cos"]] * 2, 1), sin=torch.cat([case["sin"]] * 2, 1))
    b = run_gpu(full, device)
    assert torch.equal(a, b)


def test_mixed_cos_sin_dtypes(device):
    case = random_case([64], h=2, d=80, seed=502)
    mixed = dict(case, sin=case["sin"].to(torch.bfloat16))
    out = f32(run_gpu(mixed, device))
    assert_close(out, oracle(mixed), MAX_ABS, MEAN_ABS, "cos f32 / sin bf16")


@pytest.mark.parametrize("lens", [[64, 64], [200]])
def test_softmax_scale_and_max_seqlen_none(device, lens):
    case = random_case(lens, h=2, d=80, seed=600)
    out = f32(run_gpu(case, device, softmax_scale=0.05))
    assert_close(out, oracle(case, scale=0.05), MAX_ABS, MEAN_ABS, "softmax_scale")
    a = run_gpu(case, device, max_seqlen=None)
    b = run_gpu(case, device)
    assert torch.equal(a, b)


def test_out_argument_and_strided_views(device):
    n, h, d = 64 * 3 + 20, 4, 80
    lens = [64, 64, 64, 20]
    base = random_case(lens, h=h, d=d, seed=700)
    qkv = torch.stack([base["q"], base["k"], base["v"]], dim=1).to(device)  # [N, 3, H, D]
    q, k, v = qkv.unbind(1)
    assert not q.is_contiguous()
    cos, sin, cu = base["cos"].to(device), base["sin"].to(device), base["cu_seqlens"].to(device)
    out = torch.empty(n, h, d, dtype=q.dtype, device=device)
    res = fused_rope_attention(q, k, v, cos, sin, cu, out=out)
    assert res is out
    ref = run_gpu(base, device)
    assert torch.equal(out, ref)
    # a strided output buffer (every other head of a wider tensor)
    wide = torch.zeros(n, 2 * h, d, dtype=q.dtype, device=device)
    view = wide[:, ::2]
    fused_rope_attention(q, k, v, cos, sin, cu, out=view)
    assert torch.equal(view, ref)
    assert torch.count_nonzero(wide[:, 1::2]) == 0


@pytest.mark.parametrize("lens", [[64, 64, 64], [64, 40, 64]])
def test_window_input_head_strides(device, lens):
    # q/k/v whose head stride is not head_dim (every other head of a wider
    # tensor) take the window kernel's general addressing path, also for full
    # windows of four heads; the result must equal that of contiguous inputs
    base = random_case(lens, h=4, d=80, seed=710 + len(lens) + lens[1])
    ref = run_gpu(base, device)

    def every_other_head(x):
        wide = torch.zeros(x.shape[0], 2 * x.shape[1], x.shape[2], dtype=x.dtype, device=device)
        wide[:, ::2] = x.to(device)
        return wide[:, ::2]

    q, k, v = (every_other_head(base[x]) for x in ("q", "k", "v"))
    assert q.stride(1) == 2 * 80
    cos, sin, cu = (base[x].to(device) for x in ("cos", "sin", "cu_seqlens"))
    assert plan(q, k, v, cos, sin, cu, max_seqlen=64)["kernel"] == "window"
    out = fused_rope_attention(q, k, v, cos, sin, cu, 64)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_rows_outside_segments_untouched_and_zero_path(device):
    case = random_case([10, 20], h=2, d=80, seed=800)
    q = case["q"].to(device)
    cu = torch.tensor([5, 15, 25], dtype=torch.int32)  # rows 0-4 and 25-29 outside
    out = torch.full_like(q, 7.0)
    fused_rope_attention(q, case["k"].to(device), case["v"].to(device), case["cos"].to(device),
                         case["sin"].to(device), cu.to(device), out=out)
    torch.cuda.synchronize()
    assert torch.all(out[:5] == 7.0) and torch.all(out[25:] == 7.0)
    ref = oracle(dict(case, cu_seqlens=cu))
    assert_close(f32(out), ref, MAX_ABS, MEAN_ABS, "offset segments")
    # all segments empty: max_seqlen 0 -> zeros (reference fused_attn.py:212-213)
    z = fused_rope_attention(q, case["k"].to(device), case["v"].to(device), case["cos"].to(device),
                             case["sin"].to(device), torch.tensor([3, 3], device=device))
    assert torch.count_nonzero(z) == 0


def test_deterministic(device):
    case = random_case([64] * 8 + [500], h=4, d=80, seed=900)
    a = run_gpu(case, device)
    b = run_gpu(case, device)
    assert torch.equal(a, b)


def test_graph_capture_replays(device):
    # 700 tokens: the long kernel with K rotated into the captured workspace
    # and the ping-pong loop; K changes between replays, so a stale rotated
    # K would show
    case = random_case([64, 64, 30, 700], h=4, d=80, seed=1000)
    st = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in case.items()}
    out = torch.empty_like(st["q"])
    ms = case["max_seqlen"]

    def call():
        fused_rope_attention(st["q"], st["k"], st["v"], st["cos"], st["sin"], st["cu_seqlens"], ms, out=out)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    g = torch.Generator().manual_seed(1001)
    for _ in range(4):
        for x in ("q", "k", "v"):
            st[x].copy_(torch.randn(st[x].shape, generator=g).to(st[x].dtype))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = fused_rope_attention(st["q"], st["k"], st["v"], st["cos"], st["sin"], st["cu_seqlens"], ms)
        torch.cuda.synchronize()
        assert torch.equal(got, eager)


# --- BASELINE workloads at full size --------------------------------------------

WORKLOAD_HEADS = {  # heads checked against the oracle at full size
    "cfg0": None, "cfg1": None, "cfg2w": None, "cfg3": None,
    "cfg2f": [0, 15], "cfg3f": [0, 11], "cfg4v": [0, 9], "cfg4s": [5],
}


@pytest.mark.parametrize("name", list(WORKLOAD_HEADS))
def test_workload_parity(device, name):
    w = WORKLOADS[name]
    case = make_inputs(w, seed=1234 + list(WORKLOADS).index(name))
    out = run_gpu(case, device)
    heads = WORKLOAD_HEADS[name]
    got = f32(out if heads is None else out[:, heads])
    ref = oracle(case, heads=heads)
    assert_close(got, ref, MAX_ABS, MEAN_ABS, name)
    # every head: permuting heads of the inputs permutes heads of the output --
    # bit for bit, except where the long kernel splits the units of its last
    # round along the key range (which units those are moves with the heads,
    # and a split sums the keys in a different order: within 2 bf16 ulps)
    perm = torch.randperm(w.heads, generator=torch.Generator().manual_seed(7))
    pc = dict(case, q=case["q"][:, perm], k=case["k"][:, perm], v=case["v"][:, perm])
    out_p = run_gpu(pc, device)
    want = out[:, perm.to(out.device)]
    pl = plan(*(case[x].to(device) for x in ("q", "k", "v", "cos", "sin", "cu_seqlens")),
              max_seqlen=case["max_seqlen"])
    if pl["split_parts"] > 1:
        diff = (out_p.float() - want.float()).abs()
        assert float(diff.max()) <= 2 * 2 ** -8 * float(want.float().abs().max()), name
    else:
        assert torch.equal(out_p, want)


def _call_abi(case, device, workspace):
    """fra_fwd_varlen through the C ABI, with the long kernel's whole
    workspace (True), none (False: K rotated in the kernel, no unit split),
    or "krot": only the rotated-K part (no split)."""
    import ctypes

    from fused_rope_attn_amd.fused_attn import _build_args, _workspace_bytes
    args_t = {x: case[x].to(device) for x in ("q", "k", "v", "cos", "sin")}
    cu = case["cu_seqlens"].to(device=device, dtype=torch.int32)
    out = torch.full_like(args_t["q"], float("nan"))
    a = _build_args(args_t["q"], args_t["k"], args_t["v"], args_t["cos"], args_t["sin"], out, cu,
                    case["max_seqlen"], case["q"].shape[2] ** -0.5)
    lib = _lib.load()
    ws = None
    nbytes = _workspace_bytes(lib, a)
    if workspace == "krot":
        nbytes = (a.total_seq * a.num_heads * a.head_dim * 2 + 255) // 256 * 256
    if workspace and nbytes:
        ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device=device)  # scratch: any contents
        a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    pl = _lib.Plan()
    _lib.check(lib.fra_query_plan(a, pl))
    _lib.check(lib.fra_fwd_varlen(a, ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)))
    torch.cuda.synchronize()
    return out, pl


@pytest.mark.parametrize("lens,h,d", [([2000], 3, 80), ([700, 1500, 64, 1], 2, 72), ([9216], 16, 80)])
def test_long_kernel_split_last_round(device, lens, h, d):
    # the split path (parts of the key range merged by split_merge_kernel) against the
    # unsplit kernel and the oracle
    case = random_case(lens, h=h, d=d, seed=260 + d)
    split, pl = _call_abi(case, device, workspace=True)
    whole, pl0 = _call_abi(case, device, workspace=False)
    assert pl.split_parts > 1 and pl0.split_parts == 0
    assert pl.grid == pl0.grid - pl.split_units + pl.split_units * pl.split_parts
    assert_close(f32(split), f32(whole), 8e-3, 5e-4, f"split vs whole {lens}")
    heads = [0] if h > 3 else None
    ref = oracle(case, heads=heads)
    got = f32(split if heads is None else split[:, heads])
    assert_close(got, ref, MAX_ABS, MEAN_ABS, f"split {lens}")


@pytest.mark.parametrize("lens,h,d,rope_dtype,full", [
    ([300, 5], 4, 80, torch.float32, False),
    ([700, 1500, 64, 1], 2, 72, torch.float32, True),
    ([520, 130], 3, 64, torch.bfloat16, False),
    ([333], 2, 128, torch.float16, True),
    # 5, 7, 8, 9 and 16 key blocks: 2, 4, 5, 6 and 13 steady iterations (the
    # ping-pong loop runs them in pairs, the rest go to the generic loop)
    ([257, 385, 449, 513, 1024, 3], 2, 80, torch.float32, False),
])
def test_long_kernel_rotated_k_workspace(device, lens, h, d, rope_dtype, full):
    # K rotated once per call into the workspace (a separate kernel) and then
    # staged by the ping-pong loop, against K rotated per block inside the
    # kernel by the lockstep loop: both round the same fp32 rotation to the
    # storage dtype and sum in the same order, so the outputs are identical
    case = random_case(lens, h=h, d=d, seed=270 + d, rope_dtype=rope_dtype, width=d if full else d // 2)
    pre, pl = _call_abi(case, device, workspace="krot")
    inkernel, pl0 = _call_abi(case, device, workspace=False)
    assert pl.kernel == _lib.FRA_KERNEL_LONG and pl.split_parts == 0 and pl0.split_parts == 0
    assert torch.equal(pre, inkernel), f"rotated-K workspace vs in-kernel rotation {lens}"
    assert_close(f32(pre), oracle(case), MAX_ABS, MEAN_ABS, f"rotated-K workspace {lens}")


# ---- known answers (tests/golden/attention_kat.npz, float64 from the definition) ----

_KAT = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "attention_kat.npz"))


@pytest.mark.parametrize("name", sorted({k.split("/")[0] for k in _KAT.files}))
def test_known_answers(device, name):
    case = {x: torch.from_numpy(_KAT[f"{name}/{x}"]) for x in ("q", "k", "v", "cos", "sin", "cu_seqlens")}
    for x in ("q", "k", "v"):
        case[x] = case[x].to(torch.bfloat16)   # the fixture values are bf16-representable
    cu = _KAT[f"{name}/cu_seqlens"]
    case["max_seqlen"] = int((cu[1:] - cu[:-1]).max())
    out = run_gpu(case, device, softmax_scale=float(_KAT[f"{name}/scale"][0]))
    assert torch.equal(case["q"].float(), torch.from_numpy(_KAT[f"{name}/q"]))
    assert_close(f32(out), _KAT[f"{name}/out"], MAX_ABS, MEAN_ABS, name)
    emu = A.fused_rope_attention(*(_KAT[f"{name}/{x}"] for x in ("q", "k", "v", "cos", "sin", "cu_seqlens")),
                                 softmax_scale=float(_KAT[f"{name}/scale"][0]), mode="bf16")
    assert_close(f32(out), emu, EMU_MAX_ABS, EMU_MEAN_ABS, name + " vs bf16 model")
