"""CPU tests of the C ABI (include/chia_attn.h) -- no GPU calls.

The host-only entry points (chia_attn_plan, chia_attn_tile_map,
chia_attn_query_intervals) run the same mask functions the kernel runs
(chia_proj_amd/csrc/mask.h), so checking them against the oracle's masks pins
the kernel's mask reduction, tile classification and FLOP accounting on the CPU.
"""
import ctypes
import itertools
import re
from pathlib import Path

import numpy as np
import pytest

import oracle
from chia_proj_amd import _lib, make_args

HEADER = Path(__file__).resolve().parent.parent / "include" / "chia_attn.h"


def test_library_exports_every_declared_symbol(lib_built):
    text = HEADER.read_text()
    declared = set(re.findall(r"\b(chia_attn_[a-z0-9_]+)\s*\(", text))
    assert declared == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib_built, name), name


def _c_struct_fields(text, name):
    body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), text, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        names = decl.split()[-1] if "," not in decl else decl
        for part in re.split(r",", decl):
            tok = part.strip().split()[-1].lstrip("*")
            fields.append(re.sub(r"\[.*\]", "", tok))
    return fields


@pytest.mark.parametrize("cname,pyclass", [("chia_attn_args", _lib.AttnArgs), ("chia_attn_plan_info", _lib.PlanInfo),
                                           ("chia_attn_bwd_args", _lib.BwdArgs), ("chia_attn_fp8_args", _lib.Fp8Args)])
def test_ctypes_mirrors_header_struct(cname, pyclass):
    fields = _c_struct_fields(HEADER.read_text(), cname)
    assert fields == [f[0] for f in pyclass._fields_]


def test_status_strings_and_version(lib_built):
    assert lib_built.chia_attn_abi_version() == _lib.ABI_VERSION
    for st in (0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10):
        assert _lib.status_string(st)
    assert "unknown" in _lib.status_string(-99)


def _plan_status(**kw):
    a = make_args(batch=1, heads=1, seqlen=128, head_dim=64)
    for k, v in kw.items():
        setattr(a, k, v)
    info = _lib.PlanInfo()
    return _lib.lib().chia_attn_plan(ctypes.byref(a), ctypes.byref(info))


def test_validation_codes(lib_built):
    assert _plan_status() == 0
    assert _plan_status(head_dim=96) == -3
    assert _plan_status(seqlen=0) == -2
    assert _plan_status(batch=0) == -2
    assert _plan_status(dilation=0) == -4
    assert _plan_status(window=-1) == -4
    assert _plan_status(dilation=2, prefix=4) == -4
    assert _plan_status(scale=0.0) == -5
    assert _plan_status(scale=float("nan")) == -5
    assert _plan_status(softcap=-1.0) == -5
    assert _plan_status(norm=7) == -6
    assert _plan_status(struct_size=12) == -8
    # grouped-query K/V: kv_heads must divide heads
    assert _plan_status(heads=8, kv_heads=2) == 0
    assert _plan_status(heads=8, kv_heads=1) == 0
    assert _plan_status(heads=8, kv_heads=3) == -2
    assert _plan_status(heads=8, kv_heads=-1) == -2
    a = make_args(batch=1, heads=1, seqlen=128, head_dim=64)
    a.reserved[1] = 1
    assert lib_built.chia_attn_plan(ctypes.byref(a), ctypes.byref(_lib.PlanInfo())) == -8


def test_fwd_rejects_bad_arguments_without_launching(lib_built):
    # null tensors and misaligned pointers are host-side errors: no GPU is touched
    a = make_args(batch=1, heads=1, seqlen=64, head_dim=64)
    assert lib_built.chia_attn_fwd(ctypes.byref(a), None) == -1
    a.q = a.k = a.v = a.o = 0x1000
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        st = getattr(a, name)
        st[0], st[1], st[2] = 64 * 64, 64 * 64, 64
    a.o = 0x1008  # not 16-byte aligned
    assert lib_built.chia_attn_fwd(ctypes.byref(a), None) == -7
    a.o = 0x1000
    a.q_stride[2] = 60  # row stride not a multiple of 8 elements
    assert lib_built.chia_attn_fwd(ctypes.byref(a), None) == -7
    a.q_stride[2] = 64
    # K/V rows are addressed with 32-bit offsets within a tile: negative or
    # huge sequence strides are rejected
    a.k_stride[2] = -64
    assert lib_built.chia_attn_fwd(ctypes.byref(a), None) == -2
    a.k_stride[2] = 64
    a.v_stride[2] = 1 << 25
    assert lib_built.chia_attn_fwd(ctypes.byref(a), None) == -2
    a.v_stride[2] = 1 << 24
    a.dilation = 2
    assert lib_built.chia_attn_fwd(ctypes.byref(a), None) == -2
    assert lib_built.chia_attn_fwd(None, None) == -1


MASKS = [
    dict(causal=c, window=w, dilation=d, block=b, prefix=p)
    for c, w, d, b, p in itertools.product([True, False], [0, 5, 64, 300], [1, 2, 3], [0, 33, 128], [0, 40])
    if not (d > 1 and p)
]


@pytest.mark.parametrize("S", [1, 63, 200, 513])
def test_plan_pairs_match_oracle_mask(S, lib_built):
    for kw in MASKS:
        a = make_args(batch=2, heads=3, seqlen=S, head_dim=64, **kw)
        got = _lib.plan(a)["pairs_visible"]
        want = 6 * oracle.visible_mask(S, **kw).sum().item()
        assert got == want, (S, kw)


@pytest.mark.parametrize("S", [77, 300, 700])
def test_intervals_and_tile_classes_match_oracle(S, lib_built):
    for kw in MASKS:
        a = make_args(batch=1, heads=1, seqlen=S, head_dim=64, **kw)
        full = oracle.visible_mask(S, **kw).numpy()
        dil = kw["dilation"]
        for r in range(min(dil, S)):
            sub = full[r::dil, r::dil]
            n = sub.shape[0]
            # pairs across residue classes are never visible when dilation > 1
            if dil > 1:
                off = full.copy()
                off[r::dil, r::dil] = False
                assert not off[r::dil].any()
            jlo, jhi, pre = _lib.query_intervals(a, r, n)
            jj = np.arange(n)
            rebuilt = (jj[None, :] < pre) | ((jj[None, :] >= jlo[:, None]) & (jj[None, :] <= jhi[:, None]))
            assert (rebuilt == sub).all(), (kw, r)
            for rows in (32, 64, 128):
                tm = _lib.tile_map(a, r, rows)
                for qb, kt in itertools.product(range(tm.shape[0]), range(tm.shape[1])):
                    blk = sub[qb * rows:(qb + 1) * rows, kt * 64:(kt + 1) * 64]
                    if tm[qb, kt] == 0:
                        assert not blk.any(), (kw, r, rows, qb, kt)
                    elif tm[qb, kt] == 1:
                        assert blk.shape[1] == 64 and blk.all(), (kw, r, rows, qb, kt)


def test_plan_geometry(lib_built):
    # causal sigmoid without a window pairs row blocks (i, n-1-i); every pair is one workgroup
    p = _lib.plan(make_args(batch=4, heads=16, seqlen=2048, head_dim=64, norm="sigmoid", causal=True))
    assert p["waves"] == 4 and p["block_m"] == 256 and p["workgroups"] == 4 * 16 * 8
    # so does causal softmax on fewer than 64 (batch, head) slices of 4096 rows,
    # on rows longer than 4096, and on a grid too small for two one-block
    # workgroups per CU (the pairs then have 2 wavefronts)
    p = _lib.plan(make_args(batch=2, heads=16, seqlen=4096, head_dim=64, causal=True))
    assert (p["waves"], p["block_m"], p["workgroups"]) == (4, 256, 2 * 16 * 16)
    p = _lib.plan(make_args(batch=4, heads=16, seqlen=8192, head_dim=64, causal=True))
    assert (p["waves"], p["block_m"]) == (4, 256)
    p = _lib.plan(make_args(batch=1, heads=8, seqlen=2048, head_dim=64, causal=True))
    assert (p["waves"], p["block_m"], p["workgroups"]) == (2, 128, 8 * 16)
    # a window or block mask, causal rows with a prefix (whose block work
    # zigzag pairs do not balance), and causal softmax on 64 slices or on 2-wavefront
    # pairs' grids with at least 512 blocks run the one-block core: 128-row
    # blocks, one per workgroup, 32-key steps
    for kw in (dict(causal=True, window=256), dict(causal=False, block=256), dict(causal=True, window=129),
               dict(causal=True, prefix=1024), dict(causal=True), dict(causal=True, softcap=50.0, alibi=True)):
        p = _lib.plan(make_args(batch=4, heads=16, seqlen=2048, head_dim=64, **kw))
        assert (p["waves"], p["block_m"], p["block_n"], p["workgroups"]) == (4, 128, 32, 4 * 16 * 16)
    for b, h, s in ((4, 16, 1024), (1, 16, 4096), (4, 16, 4096)):
        p = _lib.plan(make_args(batch=b, heads=h, seqlen=s, head_dim=64, causal=True))
        assert (p["waves"], p["block_m"], p["block_n"], p["workgroups"]) == (4, 128, 32, b * h * s // 128)
    # full rows stay on the paired core
    p = _lib.plan(make_args(batch=4, heads=16, seqlen=4096, head_dim=64, causal=False))
    assert (p["waves"], p["block_m"], p["block_n"]) == (4, 256, 64)
    # every visible pair is inside a computed 32 x block_n step
    for kw in (dict(causal=True), dict(causal=True, window=256), dict(causal=False, block=256),
               dict(causal=True, dilation=2, window=1024), dict(causal=True, prefix=1024)):
        p = _lib.plan(make_args(batch=1, heads=1, seqlen=4096, head_dim=64, **kw))
        assert p["block_n"] == (32 if ("window" in kw or "block" in kw or "prefix" in kw) else 64)
        assert p["wave_tiles_visited"] * 32 * p["block_n"] >= p["pairs_visible"]
        assert p["wave_tiles_partial"] <= p["wave_tiles_visited"]


def test_plan_geometry_head_dim_128(lib_built):
    # head_dim 128 runs the one-block core: 128-row blocks, one per workgroup
    # step, computed in 32-key steps (block_n 32); causal pairs blocks (i, n-1-i)
    p = _lib.plan(make_args(batch=2, heads=32, seqlen=2048, head_dim=128, causal=True))
    assert (p["waves"], p["block_m"], p["block_n"]) == (4, 128, 32)
    assert p["workgroups"] == 2 * 32 * 8
    # full rows below 2048 keys: one block per workgroup
    p = _lib.plan(make_args(batch=4, heads=16, seqlen=1024, head_dim=128, norm="sigmoid", causal=False))
    assert (p["block_m"], p["block_n"], p["workgroups"]) == (128, 32, 4 * 16 * 8)
    # dense full rows: every 32 x 32 step of every block is computed
    assert p["wave_tiles_visited"] == p["tiles_total"] * 4 == 4 * 16 * (1024 // 32) * (1024 // 32)
    # sigmoid / ReLU on full rows of 2048+ keys without a score modifier: the paired core
    for S in (2048, 4096):
        for norm in ("sigmoid", "relu"):
            p = _lib.plan(make_args(batch=4, heads=16, seqlen=S, head_dim=128, norm=norm, causal=False))
            assert (p["waves"], p["block_m"], p["block_n"]) == (4, 256, 64)
        # softmax there runs the one-block core (no paired softmax kernel at head_dim 128)
        p = _lib.plan(make_args(batch=4, heads=16, seqlen=S, head_dim=128, norm="softmax", causal=False))
        assert (p["waves"], p["block_m"], p["block_n"]) == (4, 128, 32)
    # ... but with a softcap (or too few workgroups for two per CU) the one-block core
    p = _lib.plan(make_args(batch=4, heads=16, seqlen=4096, head_dim=128, softcap=30.0, causal=False))
    assert (p["block_m"], p["block_n"]) == (128, 32)
    p = _lib.plan(make_args(batch=1, heads=4, seqlen=4096, head_dim=128, norm="relu", causal=False))
    assert (p["block_m"], p["block_n"]) == (128, 32)
    # every visible pair lies inside a computed 32 x block_n step, and the steps
    # are fewer than with 64-key tiles on a band
    for kw in (dict(causal=True), dict(causal=True, window=256), dict(causal=False, block=256),
               dict(causal=True, dilation=2, window=1024), dict(causal=True, prefix=1024)):
        p = _lib.plan(make_args(batch=1, heads=1, seqlen=4096, head_dim=128, **kw))
        assert p["block_n"] == 32
        assert p["wave_tiles_visited"] * 32 * 32 >= p["pairs_visible"]
        assert p["wave_tiles_partial"] <= p["wave_tiles_visited"]
        p64 = _lib.plan(make_args(batch=1, heads=1, seqlen=4096, head_dim=64, **kw))
        assert p["wave_tiles_visited"] * 32 <= p64["wave_tiles_visited"] * p64["block_n"]
        assert p64["pairs_visible"] == p["pairs_visible"]


def _bwd_ready_args(norm="softmax", **kw):
    """Forward args with fake (aligned, never dereferenced) device pointers."""
    a = make_args(batch=1, heads=4, seqlen=128, head_dim=64, norm=norm)
    a.q = a.k = a.v = a.o = 0x10000
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        st = getattr(a, name)
        st[0], st[1], st[2] = 4 * 128 * 64, 128 * 64, 64
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _bwd_status(a, **kw):
    b = _lib.BwdArgs(fwd=ctypes.pointer(a), dout=0x20000, dq=0x30000, dk=0x40000, dv=0x50000, lse=0x60000,
                     workspace=0x70000, workspace_bytes=1 << 30)
    for name in ("dout_stride", "dq_stride", "dk_stride", "dv_stride"):
        st = getattr(b, name)
        st[0], st[1], st[2] = 4 * 128 * 64, 128 * 64, 64
    for k, v in kw.items():
        setattr(b, k, v)
    return _lib.lib().chia_attn_bwd(ctypes.byref(b), None)


def test_bwd_workspace_size(lib_built):
    # softmax: lse log2 e and delta per (b, h, residue, row padded to 64 rows), fp32
    a = make_args(batch=2, heads=3, seqlen=100, head_dim=64)
    assert lib_built.chia_attn_bwd_workspace_size(ctypes.byref(a)) == 2 * 2 * 3 * 128 * 4
    a = make_args(batch=2, heads=3, seqlen=100, head_dim=64, dilation=3)  # residues of 34, 33, 33 rows
    assert lib_built.chia_attn_bwd_workspace_size(ctypes.byref(a)) == 2 * 2 * 3 * 3 * 64 * 4
    for norm in ("sigmoid", "relu"):
        a = make_args(batch=2, heads=3, seqlen=100, head_dim=64, norm=norm)
        assert lib_built.chia_attn_bwd_workspace_size(ctypes.byref(a)) == 0
    a = make_args(batch=1, heads=1, seqlen=100, head_dim=96)
    assert lib_built.chia_attn_bwd_workspace_size(ctypes.byref(a)) == -3


def test_bwd_rejects_bad_arguments_without_launching(lib_built):
    assert lib_built.chia_attn_bwd(None, None) == -1
    a = _bwd_ready_args()
    assert _bwd_status(a, struct_size=8) == -8
    assert _bwd_status(a, reserved0=1) == -8
    assert _bwd_status(a, dq=None) == -1
    assert _bwd_status(a, dk=0x40008) == -7          # misaligned
    assert _bwd_status(a, lse=None) == -1            # softmax needs the forward's lse
    assert _bwd_status(a, workspace=None) == -9
    assert _bwd_status(a, workspace_bytes=8) == -9
    b = _bwd_ready_args(head_dim=96)
    assert _bwd_status(b) == -3
    c = _bwd_ready_args(norm="relu")
    assert _bwd_status(c, lse=None, workspace=None, workspace_bytes=0, dq=None) == -1
    d = _bwd_ready_args(heads=512, kv_heads=1)       # more than 256 query heads per K/V head
    assert _bwd_status(d) == -2


def test_bwd_noalloc_rejects_without_launching(lib_built):
    """The allocation-free backward checks its arguments as chia_attn_bwd does (the
    workspace fields aside) and refuses statistics beyond its static scratch."""
    assert lib_built.chia_attn_bwd_noalloc(None, None) == -1
    a = _bwd_ready_args()
    b = _lib.BwdArgs(fwd=ctypes.pointer(a), dout=0x20000, dq=0x30000, dk=0x40000, dv=None, lse=0x60000)
    assert lib_built.chia_attn_bwd_noalloc(ctypes.byref(b), None) == -1
    big = _bwd_ready_args(batch=16, heads=16, seqlen=8192)
    assert lib_built.chia_attn_bwd_workspace_size(ctypes.byref(big)) == 2 * 16 * 16 * 8192 * 4
    b = _lib.BwdArgs(fwd=ctypes.pointer(big), dout=0x20000, dq=0x30000, dk=0x40000, dv=0x50000, lse=0x60000)
    for name in ("dout_stride", "dq_stride", "dk_stride", "dv_stride"):
        st = getattr(b, name)
        st[0], st[1], st[2] = 4 * 128 * 64, 128 * 64, 64
    assert lib_built.chia_attn_bwd_noalloc(ctypes.byref(b), None) == -10
    assert "scratch" in _lib.status_string(-10)


def test_fp8_rejects_bad_arguments_without_launching(lib_built):
    a = make_args(batch=1, heads=1, seqlen=64, head_dim=64)
    a.q = a.k = a.v = a.o = 0x1000
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        st = getattr(a, name)
        st[0], st[1], st[2] = 64 * 64, 64 * 64, 64
    f = _lib.Fp8Args(attn=ctypes.pointer(a))
    call = lambda: lib_built.chia_attn_fwd_fp8(ctypes.byref(f), None)  # noqa: E731
    assert lib_built.chia_attn_fwd_fp8(None, None) == -1
    f.format = 2
    assert call() == -8                      # e4m3 (0) or e5m2 (1) only
    f.format = 0
    f.reserved[4] = 1
    assert call() == -8
    f.reserved[4] = 0
    f.v_descale = 0.0
    assert call() == -5
    f.v_descale = float("inf")
    assert call() == -5
    f.v_descale = 1.0
    a.q_stride[2] = 72                       # a multiple of 8 elements, not of 16 bytes
    assert call() == -7
    a.q_stride[2] = 64
    a.cu_seqlens = 0x2002                    # packed sequences: offsets must be 4-byte aligned
    assert call() == -7
