"""The C ABI of libfra.so without a GPU: the library loads, exports every
symbol include/fra.h declares, its structs match the ctypes mirrors, and the
dispatcher's validation and kernel choice behave (no kernel is launched:
every call here fails validation, or has total_seq == 0, or is a plan query)."""
import ctypes
import os
import re

import pytest

from fused_rope_attn_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fra.h")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z0-9_]+\s*\*?\s*(fra_[a-z0-9_]+)\s*\(", text, re.M)))


def test_header_declares_what_the_binding_types():
    syms = header_symbols()
    assert syms, "no declarations parsed"
    assert set(syms) == set(_lib.SIGNATURES), (syms, sorted(_lib.SIGNATURES))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in header_symbols():
        assert hasattr(lib, name), name
    assert lib.fra_abi_version() == _lib.ABI_VERSION
    assert lib.fra_sizeof_args() == ctypes.sizeof(_lib.FwdArgs)
    assert lib.fra_sizeof_plan() == ctypes.sizeof(_lib.Plan)
    assert b"gfx950" in lib.fra_version()


def make_args(**kw):
    a = _lib.FwdArgs()
    n, h, d = kw.get("n", 1024), kw.get("h", 16), kw.get("d", 80)
    base = 1 << 20  # fake, aligned device addresses: nothing is launched
    a.q, a.k, a.v, a.cos, a.sin, a.out = (base * (i + 1) for i in range(6))
    a.cu_seqlens = base * 8
    a.q_stride_seq = a.k_stride_seq = a.v_stride_seq = a.out_stride_seq = h * d
    a.q_stride_head = a.k_stride_head = a.v_stride_head = a.out_stride_head = d
    a.rope_stride_seq = d // 2
    a.total_seq, a.num_heads, a.head_dim = n, h, d
    a.num_seqs = kw.get("nseg", 16)
    a.max_seqlen = kw.get("max_seqlen", 64)
    a.rope_width = d // 2
    a.qkv_dtype, a.rope_dtype = _lib.FRA_DTYPE_BF16, _lib.FRA_DTYPE_F32
    a.softmax_scale = d ** -0.5
    a.flags = 0
    for key, val in kw.items():
        if key not in ("n", "h", "d", "nseg"):
            setattr(a, key, val)
    return a


def plan_of(a):
    p = _lib.Plan()
    rc = _lib.load().fra_query_plan(a, p)
    return rc, p


def test_plan_window_and_long(monkeypatch):
    monkeypatch.delenv("FRA_WINDOW_HEADS", raising=False)
    rc, p = plan_of(make_args())
    assert rc == _lib.FRA_OK
    # One workgroup per (window, group of hw heads).  hw = 1 (two wavefronts
    # splitting the head's queries) when there are no more (window, head)
    # pairs than CUs (256 assumed without a GPU); else hw = 2 when that grid
    # runs in one round of resident workgroups (5 per CU), else 4.
    assert p.kernel == _lib.FRA_KERNEL_WINDOW and p.block == 128
    assert p.grid == 16 * 16
    rc, p = plan_of(make_args(n=2048, nseg=32))  # 512 pairs: two heads a workgroup
    assert rc == _lib.FRA_OK and p.block == 128 and p.grid == 32 * 8
    rc, p = plan_of(make_args(n=4096, nseg=64, h=6))  # 384 pairs, a partial head group
    assert rc == _lib.FRA_OK and p.grid == 64 * 3
    # FRA_WINDOW_HEADS forces a form
    for heads, block, grid in (("1", 128, 256), ("2", 128, 128), ("4", 256, 64)):
        monkeypatch.setenv("FRA_WINDOW_HEADS", heads)
        rc, p = plan_of(make_args())
        assert rc == _lib.FRA_OK and (p.block, p.grid) == (block, grid), heads
    monkeypatch.setenv("FRA_WINDOW_HEADS", "1")  # head_dim 72 has no one-head form: four
    rc, p = plan_of(make_args(d=72))
    assert rc == _lib.FRA_OK and (p.block, p.grid) == (256, 64)
    monkeypatch.delenv("FRA_WINDOW_HEADS")
    rc, p = plan_of(make_args(n=9216, nseg=144))  # 1152 two-head workgroups fit 1280 slots
    assert rc == _lib.FRA_OK and p.block == 128 and p.grid == 144 * 8
    rc, p = plan_of(make_args(n=11968, nseg=187))  # 1496 do not: four heads
    assert rc == _lib.FRA_OK and p.block == 256 and p.grid == 187 * 4
    assert p.name.decode() == "window_d80_bf16_ropef32"
    rc, p = plan_of(make_args(max_seqlen=9216, num_seqs=1, n=9216))
    assert rc == _lib.FRA_OK and p.kernel == _lib.FRA_KERNEL_LONG
    assert p.grid == 16 * ((9216 + p.block_q - 1) // p.block_q)
    rc, p = plan_of(make_args(d=128, max_seqlen=64))
    assert rc == _lib.FRA_OK and p.kernel == _lib.FRA_KERNEL_LONG  # window kernel is for D <= 96
    rc, p = plan_of(make_args(d=72, max_seqlen=64, qkv_dtype=_lib.FRA_DTYPE_F16, rope_dtype=_lib.FRA_DTYPE_BF16))
    assert rc == _lib.FRA_OK and p.name.decode() == "window_d72_f16_ropebf16"


@pytest.mark.parametrize("field,value,code,msg", [
    ("q", 0, _lib.FRA_EINVAL, "NULL"),
    ("cu_seqlens", 0, _lib.FRA_EINVAL, "NULL"),
    ("num_heads", 0, _lib.FRA_EINVAL, "num_heads"),
    ("head_dim", 81, _lib.FRA_EINVAL, "even"),
    ("head_dim", 0, _lib.FRA_EINVAL, "even"),
    ("num_seqs", 0, _lib.FRA_EINVAL, "num_seqs"),
    ("max_seqlen", 0, _lib.FRA_EINVAL, "max_seqlen"),
    ("qkv_dtype", _lib.FRA_DTYPE_F32, _lib.FRA_EINVAL, "qkv_dtype"),
    ("rope_dtype", 7, _lib.FRA_EINVAL, "rope_dtype"),
    ("rope_width", 33, _lib.FRA_EINVAL, "rope_width"),
    ("softmax_scale", 0.0, _lib.FRA_EINVAL, "softmax_scale"),
    ("softmax_scale", float("nan"), _lib.FRA_EINVAL, "softmax_scale"),
    ("flags", 1, _lib.FRA_EINVAL, "flags"),
    ("q_stride_seq", -1280, _lib.FRA_EINVAL, "strides"),
    ("v", (1 << 20) + 8, _lib.FRA_EUNSUPPORTED, "aligned"),
    ("q", (1 << 20) + 4, _lib.FRA_EUNSUPPORTED, "aligned"),
    ("v_stride_seq", 1284, _lib.FRA_EUNSUPPORTED, "multiples"),
    ("q_stride_head", 82, _lib.FRA_EUNSUPPORTED, "multiples"),
])
def test_validation_errors(field, value, code, msg):
    a = make_args(**{field: value})
    lib = _lib.load()
    rc, _ = plan_of(a)
    assert rc == code
    assert msg in lib.fra_last_error().decode()
    assert lib.fra_fwd_varlen(a, None) == code  # fails before any launch


def test_unsupported_head_dim():
    lib = _lib.load()
    for d in (64, 72, 80, 96, 128):
        assert lib.fra_supports_head_dim(d) == 1
    for d in (2, 66, 88, 256):
        assert lib.fra_supports_head_dim(d) == 0
        a = make_args(d=d)
        assert lib.fra_fwd_varlen(a, None) == _lib.FRA_EUNSUPPORTED
        assert "head_dim" in lib.fra_last_error().decode()


def test_null_args_and_empty_problem():
    lib = _lib.load()
    assert lib.fra_fwd_varlen(None, None) == _lib.FRA_EINVAL
    assert lib.fra_query_plan(make_args(), None) == _lib.FRA_EINVAL
    # total_seq == 0 validates and returns without launching
    assert lib.fra_fwd_varlen(make_args(n=0), None) == _lib.FRA_OK
    assert lib.fra_last_error() == b""


def test_forward_lse_pointer_alignment():
    lib = _lib.load()
    a = make_args(lse=(1 << 20) * 9 + 2)
    assert lib.fra_fwd_varlen(a, None) == _lib.FRA_EINVAL
    assert "lse" in lib.fra_last_error().decode()


def test_forward_workspace_size_and_alignment():
    lib = _lib.load()
    nbytes = ctypes.c_int64(-1)
    assert lib.fra_workspace_bytes(make_args(), ctypes.byref(nbytes)) == _lib.FRA_OK
    assert nbytes.value == 0  # window kernel: no workspace
    n, h, d = 9216, 16, 80
    a = make_args(n=n, nseg=1, max_seqlen=n, num_seqs=1)
    assert lib.fra_workspace_bytes(a, ctypes.byref(nbytes)) == _lib.FRA_OK
    krot = (n * h * d * 2 + 255) // 256 * 256  # K rotated once per call, then the split scratch
    assert nbytes.value > krot
    a.workspace, a.workspace_bytes = (1 << 20) * 10, nbytes.value
    rc, p = plan_of(a)
    assert rc == _lib.FRA_OK and p.split_parts > 1
    a.workspace_bytes = krot  # rotated K only: no split
    rc, p = plan_of(a)
    assert rc == _lib.FRA_OK and p.split_parts == 0 and p.grid == h * ((n + p.block_q - 1) // p.block_q)
    a.workspace = (1 << 20) * 10 + 8
    assert lib.fra_fwd_varlen(a, None) == _lib.FRA_EINVAL
    assert "workspace" in lib.fra_last_error().decode()


@pytest.mark.parametrize("total,nseg,max_seqlen,parts", [
    # six unequal images as full-attention segments (10493 tokens): the grid
    # has 11 query blocks for every (segment, head), 1056 units, but at most
    # 16 x (41 + 6) = 752 hold queries -- three rounds, no split
    (10493, 6, 2736, 0),
    # the same segment count with every segment full: 1056 real units, the
    # last round of 32 split in 5 parts (43 key blocks, at least 8 a part)
    (6 * 2736, 6, 2736, 5),
])
def test_split_plan_counts_query_blocks_that_exist(total, nseg, max_seqlen, parts):
    lib = _lib.load()
    a = make_args(n=total, nseg=nseg, max_seqlen=max_seqlen, num_seqs=nseg)
    nbytes = ctypes.c_int64(0)
    assert lib.fra_workspace_bytes(a, ctypes.byref(nbytes)) == _lib.FRA_OK
    a.workspace, a.workspace_bytes = (1 << 20) * 10, nbytes.value
    rc, p = plan_of(a)
    assert rc == _lib.FRA_OK and p.kernel == _lib.FRA_KERNEL_LONG
    assert p.split_parts == parts
    assert p.grid >= 16 * nseg * (-(-max_seqlen // 256))


@pytest.mark.parametrize("seglen,nseg,parts", [
    (9216, 1, 4),   # 576 units: a last round of 64 on 256 CUs, 144 key blocks per unit
    (2304, 8, 2),   # 1152 units: 128 left over, 2 parts of 18 key blocks
    (512, 18, 0),   # 576 units, but 8 key blocks per unit: parts of 4 or 2 blocks lose
    (256, 36, 0),
])
def test_split_plan_needs_eight_key_blocks_per_part(seglen, nseg, parts):
    # CU count assumed 256 without a GPU; the workspace holds everything asked for
    lib = _lib.load()
    n = seglen * nseg
    a = make_args(n=n, nseg=nseg, max_seqlen=seglen, num_seqs=nseg)
    nbytes = ctypes.c_int64(0)
    assert lib.fra_workspace_bytes(a, ctypes.byref(nbytes)) == _lib.FRA_OK
    a.workspace, a.workspace_bytes = (1 << 20) * 10, nbytes.value
    rc, p = plan_of(a)
    assert rc == _lib.FRA_OK and p.kernel == _lib.FRA_KERNEL_LONG
    assert p.split_parts == parts
    if parts:
        assert p.split_units == (16 * nseg * (seglen // 256)) % 256


def make_bwd_args(**kw):
    a = _lib.BwdArgs()
    n, h, d = kw.get("n", 1024), kw.get("h", 16), kw.get("d", 80)
    base = 1 << 20  # fake, aligned device addresses: nothing is launched
    names = ("q", "k", "v", "cos", "sin", "out", "dout", "lse", "cu_seqlens", "dq", "dk", "dv")
    for i, name in enumerate(names):
        setattr(a, name, base * (i + 1))
    for t in ("q", "k", "v", "out", "dout", "dq", "dk", "dv"):
        setattr(a, f"{t}_stride_seq", h * d)
        setattr(a, f"{t}_stride_head", d)
    a.rope_stride_seq = d // 2
    a.total_seq, a.num_heads, a.head_dim = n, h, d
    a.num_seqs = kw.get("nseg", 16)
    a.max_seqlen = kw.get("max_seqlen", 64)
    a.rope_width = d // 2
    a.qkv_dtype, a.rope_dtype = _lib.FRA_DTYPE_BF16, _lib.FRA_DTYPE_F32
    a.softmax_scale = d ** -0.5
    a.flags = 0
    for key, val in kw.items():
        if key not in ("n", "h", "d", "nseg"):
            setattr(a, key, val)
    return a


def test_bwd_struct_and_workspace_size():
    lib = _lib.load()
    assert lib.fra_sizeof_bwd_args() == ctypes.sizeof(_lib.BwdArgs)
    nbytes = ctypes.c_int64(-1)
    a = make_bwd_args(n=9216, h=16, max_seqlen=9216, nseg=1)
    assert lib.fra_bwd_workspace_bytes(a, ctypes.byref(nbytes)) == _lib.FRA_OK
    # one fp32 per (head, token) for the rows' dout . out (256-byte padded),
    # then q and k rotated once ([N, H, D], 2 bytes each)
    assert nbytes.value == (9216 * 16 * 4 + 255) // 256 * 256 + 2 * 9216 * 16 * 80 * 2
    # segments of at most 64 tokens take the one-pass kernel, which needs no scratch
    assert lib.fra_bwd_workspace_bytes(make_bwd_args(n=9216, nseg=144), ctypes.byref(nbytes)) == _lib.FRA_OK
    assert nbytes.value == 0
    # total_seq == 0 validates and returns without launching (no workspace needed)
    assert lib.fra_bwd_varlen(make_bwd_args(n=0), None) == _lib.FRA_OK


@pytest.mark.parametrize("field,value,code,msg", [
    ("dout", 0, _lib.FRA_EINVAL, "NULL"),
    ("lse", 0, _lib.FRA_EINVAL, "NULL"),
    ("dk", 0, _lib.FRA_EINVAL, "NULL"),
    ("d", 88, _lib.FRA_EUNSUPPORTED, "head_dim"),
    ("rope_dtype", _lib.FRA_DTYPE_BF16, _lib.FRA_EUNSUPPORTED, "float32"),
    ("dq", (1 << 20) * 10 + 8, _lib.FRA_EUNSUPPORTED, "16-byte aligned"),
    ("dout_stride_head", 84, _lib.FRA_EUNSUPPORTED, "multiples of 8"),
    ("cos", (1 << 20) * 4 + 8, _lib.FRA_EUNSUPPORTED, "cos/sin"),
    ("lse", (1 << 20) * 8 + 2, _lib.FRA_EINVAL, "lse"),
    ("flags", 2, _lib.FRA_EINVAL, "flags"),
    ("max_seqlen", 0, _lib.FRA_EINVAL, "max_seqlen"),
])
def test_bwd_validation_errors(field, value, code, msg):
    lib = _lib.load()
    a = make_bwd_args(**{field: value})
    nbytes = ctypes.c_int64(0)
    assert lib.fra_bwd_workspace_bytes(a, ctypes.byref(nbytes)) == code
    assert msg in lib.fra_last_error().decode()
    assert lib.fra_bwd_varlen(a, None) == code  # fails before any launch


def test_bwd_requires_workspace():
    lib = _lib.load()
    a = make_bwd_args(max_seqlen=1000, nseg=1)
    assert lib.fra_bwd_varlen(a, None) == _lib.FRA_EINVAL  # no workspace: fails before any launch
    assert "workspace" in lib.fra_last_error().decode()
    a.workspace, a.workspace_bytes = (1 << 20) * 20, 1024 * 16 * 4 + 2 * 1024 * 16 * 80 * 2 - 4
    assert lib.fra_bwd_varlen(a, None) == _lib.FRA_EINVAL
