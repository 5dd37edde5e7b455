"""C-ABI: both libraries load without a GPU, export every function declared in
include/*.h, the ctypes descriptor mirrors the C struct byte for byte, and
host-side validation turns bad input into error codes (no GPU call is made)."""

import ctypes
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

from tensorpack_amd import _abi, _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def _declared(header):
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(mtc_[a-z_0-9]+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def hip():
    return _native.hip_lib()


def test_every_declared_symbol_is_exported(hip):
    rd = _native.rd_lib()
    for header, lib in (("mtc_hip.h", hip), ("mtc_rd.h", rd)):
        names = _declared(header)
        assert names, header
        for n in names:
            assert hasattr(lib, n), f"{n} declared in {header} but not exported"
    assert set(_abi.EXPORTED) == set(_declared("mtc_hip.h"))
    assert hip.mtc_abi_version() == _abi.ABI_VERSION
    assert rd.mtc_rd_abi_version() == 1


def test_descriptor_layout_matches_c():
    fields = [f[0] for f in _abi.MtcStreamDesc._fields_]
    src = "#include <stddef.h>\n#include <stdio.h>\n#include \"mtc_hip.h\"\nint main(void){\n"
    src += 'printf("%zu\\n", sizeof(mtc_stream_desc));\n'
    for f in fields:
        src += f'printf("%zu\\n", offsetof(mtc_stream_desc, {f}));\n'
    src += "return 0;}\n"
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "t.c"), os.path.join(d, "t")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", INCLUDE, c, "-o", exe], check=True)
        out = [int(x) for x in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    assert out[0] == ctypes.sizeof(_abi.MtcStreamDesc)
    assert out[1:] == [getattr(_abi.MtcStreamDesc, f).offset for f in fields]


def _desc(**kw):
    d = _abi.MtcStreamDesc()
    d.abi_version = _abi.ABI_VERSION
    d.K, d.N, d.chunk_rows = 256, 64, 128
    d.n_panels, d.n_chunks = 2, 2
    d.n_buckets, d.max_unit_words, d.max_unit_words4 = 4, 100, 100
    d.n_leaves, d.payload_dwords = 4, 64
    dummy = 0x1000
    d.payload = d.buckets = d.unit_hdr = d.leaf_word = d.steps = dummy
    d.n_steps = 8
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def test_descriptor_validation(hip):
    ok = _desc()
    assert hip.mtc_check_desc(ctypes.byref(ok)) == 0
    cases = {
        "abi_version": (99, -7), "N": (60, -2), "K": (0, -2), "chunk_rows": (48, -2),
        "n_panels": (3, -2), "n_chunks": (1, -2), "unit_hdr": (None, -1), "payload": (None, -1),
        "max_unit_words4": (50, -2), "steps": (None, -1), "n_steps": (0, -1),
        "fixed_steps": (20, -2), "reserved": (1, -2),
    }
    for field, (val, code) in cases.items():
        assert hip.mtc_check_desc(ctypes.byref(_desc(**{field: val}))) == code, field
        assert hip.mtc_last_error()
    assert hip.mtc_check_desc(None) == -1
    # fp32-scale flag and table must agree
    assert hip.mtc_check_desc(ctypes.byref(_desc(flags=_abi.MTC_FLAG_FP32_SCALES))) == -1
    assert hip.mtc_check_desc(ctypes.byref(_desc(leaf_scale=0x2000))) == -2
    # the fixed record area of the 8 decode blocks plus the null record must be present
    assert hip.mtc_check_desc(ctypes.byref(_desc(fixed_steps=16, n_steps=129))) == 0
    assert hip.mtc_check_desc(ctypes.byref(_desc(fixed_steps=16, n_steps=128))) == -2
    # arrays the kernels would address past 2 GiB with their 32-bit byte offsets are rejected
    lim = 0x7FFFFFFF
    assert hip.mtc_check_desc(ctypes.byref(_desc(payload_dwords=lim // 4))) == 0
    assert hip.mtc_check_desc(ctypes.byref(_desc(payload_dwords=lim // 4 + 1))) == -2
    assert hip.mtc_check_desc(ctypes.byref(_desc(n_leaves=lim // 4 + 1))) == -2
    assert hip.mtc_check_desc(ctypes.byref(_desc(n_steps=lim // 32))) == 0          # 8-word records
    assert hip.mtc_check_desc(ctypes.byref(_desc(n_steps=lim // 32 + 1))) == -2


def test_entry_points_reject_bad_arguments_before_any_gpu_call(hip):
    d = _desc()
    ref = ctypes.byref(d)
    assert hip.mtc_gemv_f32(ref, None, 256, 0x10, 64, 1, None, 0, None) == -1
    assert hip.mtc_gemv_f32(ref, 0x10, 256, 0x10, 64, 0, None, 0, None) == -3
    assert hip.mtc_gemv_f32(ref, 0x10, 100, 0x10, 64, 1, None, 0, None) == -3
    need = hip.mtc_gemv_workspace_bytes(ref, 1)
    assert need > 0                                             # two chunks -> split-K workspace
    assert hip.mtc_gemv_f32(ref, 0x10, 256, 0x10, 64, 1, None, 0, None) == -5
    assert hip.mtc_gemv_f32(ref, 0x10, 256, 0x10, 64, 1, 0x20, need - 1, None) == -5
    assert hip.mtc_dequant(ref, None, None) == -1
    t = ctypes.byref(_tdesc())
    assert hip.mtc_gemm_bf16(t, 0x10, 5, 256, 0x10, 0, 300, 4, None, 0, None) == -4
    assert hip.mtc_gemm_bf16(t, 0x10, 1, 256, 0x10, 9, 300, 4, None, 0, None) == -4
    assert hip.mtc_gemm_bf16(t, None, 1, 256, 0x10, 0, 300, 4, None, 0, None) == -1
    assert hip.mtc_gemm_bf16(t, 0x10, 1, 100, 0x10, 0, 300, 4, None, 0, None) == -3
    assert hip.mtc_gemm_bf16(t, 0x10, 1, 256, 0x10, 0, 300, 0, None, 0, None) == -3
    assert hip.mtc_gemm_bf16(t, 0x10, 1, 260, 0x10, 0, 300, 4, None, 0, None) == -3      # unaligned bf16 rows
    need = hip.mtc_gemm_workspace_bytes(t, 4, 0)
    # fp32 X adds the staged bf16 copy (M x K x 2 bytes) to whatever the K splits need
    assert need - hip.mtc_gemm_workspace_bytes(t, 4, 1) == 4 * 256 * 2
    assert hip.mtc_gemm_bf16(t, 0x10, 0, 256, 0x10, 0, 300, 4, 0x20, need - 1, None) == -5
    tp = ctypes.byref(_tdesc(row_perm=0x3000))
    assert hip.mtc_gemm_workspace_bytes(tp, 4, 1) - hip.mtc_gemm_workspace_bytes(t, 4, 1) == 4 * 256 * 2   # a row permutation stages bf16 X too


def test_group_entry_rejects_bad_arguments_before_any_gpu_call(hip):
    one = _desc(chunk_rows=256, n_chunks=1)                     # single-chunk streams group
    two = _desc()                                               # two row chunks: not groupable
    D = _abi.DescP
    descs = lambda *ds: (D * len(ds))(*[ctypes.pointer(x) for x in ds])
    ys = lambda n: (ctypes.c_void_p * n)(*([0x10] * n))
    lds = lambda n, v=64: (ctypes.c_int64 * n)(*([v] * n))
    f = hip.mtc_gemv_f32_group
    assert f(None, 1, 0x10, 256, ys(1), lds(1), 1, None) == -1
    assert f(descs(one), 0, 0x10, 256, ys(1), lds(1), 1, None) == -3
    assert f(descs(*[one] * 5), 5, 0x10, 256, ys(5), lds(5), 1, None) == -3      # more than MTC_MAX_GROUP
    assert _abi.MAX_GROUP == 4
    assert f(descs(one), 1, None, 256, ys(1), lds(1), 1, None) == -1
    assert f(descs(one), 1, 0x10, 256, ys(1), lds(1), 0, None) == -3
    assert f(descs(one, two), 2, 0x10, 256, ys(2), lds(2), 1, None) == -3        # split-K member
    assert b"row chunks" in hip.mtc_last_error()
    other_k = _desc(K=512, chunk_rows=512, n_chunks=1)
    assert f(descs(one, other_k), 2, 0x10, 512, ys(2), lds(2), 1, None) == -3     # different K
    assert f(descs(one, _desc(chunk_rows=256, n_chunks=1, row_perm=0x2000)), 2, 0x10, 256, ys(2), lds(2), 1,
             None) == -3                                                          # permutation presence
    assert f(descs(one), 1, 0x10, 100, ys(1), lds(1), 1, None) == -3             # ldx < K
    assert f(descs(one), 1, 0x10, 256, ys(1), lds(1, 10), 1, None) == -3         # ldy < N
    assert f(descs(one), 1, 0x10, 256, (ctypes.c_void_p * 1)(None), lds(1), 1, None) == -1
    assert f(descs(_desc(chunk_rows=256, n_chunks=1, abi_version=3)), 1, 0x10, 256, ys(1), lds(1), 1, None) == -7


def test_group_prefill_entry_rejects_bad_arguments_before_any_gpu_call(hip):
    a, b = _tdesc(), _tdesc(N=544, n_col_tiles=3)
    D = _abi.TileDescP
    descs = lambda *ds: (D * len(ds))(*[ctypes.pointer(x) for x in ds])
    ys = lambda n: (ctypes.c_void_p * n)(*([0x10] * n))
    lds = lambda n, v=600: (ctypes.c_int64 * n)(*([v] * n))
    f = hip.mtc_gemm_bf16_group
    assert f(None, 1, 0x10, 1, 256, ys(1), 0, lds(1), 4, None, 0, None) == -1
    assert f(descs(a), 0, 0x10, 1, 256, ys(1), 0, lds(1), 4, None, 0, None) == -3
    assert f(descs(*[a] * 5), 5, 0x10, 1, 256, ys(5), 0, lds(5), 4, None, 0, None) == -3
    assert f(descs(a), 1, None, 1, 256, ys(1), 0, lds(1), 4, None, 0, None) == -1
    assert f(descs(a), 1, 0x10, 5, 256, ys(1), 0, lds(1), 4, None, 0, None) == -4               # x dtype
    assert f(descs(a), 1, 0x10, 1, 256, ys(1), 9, lds(1), 4, None, 0, None) == -4               # y dtype
    assert f(descs(a), 1, 0x10, 1, 256, ys(1), 0, lds(1), 0, None, 0, None) == -3               # M
    other_k = _tdesc(K=512, n_ksteps=8)
    assert f(descs(a, other_k), 2, 0x10, 1, 512, ys(2), 0, lds(2), 4, None, 0, None) == -3      # different K
    assert f(descs(a, _tdesc(flags=_abi.MTC_FLAG_FP32_SCALES)), 2, 0x10, 1, 256, ys(2), 0, lds(2), 4, None, 0,
             None) == -3                                                                          # scale format
    assert f(descs(a, b), 2, 0x10, 1, 100, ys(2), 0, lds(2), 4, None, 0, None) == -3           # ldx < K
    assert f(descs(a, b), 2, 0x10, 1, 256, ys(2), 0, lds(2, 300), 4, None, 0, None) == -3      # ldy < N
    assert f(descs(a), 1, 0x10, 1, 260, ys(1), 0, lds(1), 4, None, 0, None) == -3              # unaligned bf16 rows
    need = hip.mtc_gemm_group_workspace_bytes(descs(a, b), 2, 4, 0)                             # fp32 X: staged per member
    assert need - hip.mtc_gemm_group_workspace_bytes(descs(a, b), 2, 4, 1) == 2 * 4 * 256 * 2
    assert need == hip.mtc_gemm_workspace_bytes(ctypes.byref(a), 4, 0) + hip.mtc_gemm_workspace_bytes(ctypes.byref(b), 4, 0)
    assert f(descs(a, b), 2, 0x10, 0, 256, ys(2), 0, lds(2), 4, 0x20, need - 1, None) == -5    # workspace too small
    assert f(descs(a, b), 2, 0x10, 0, 256, ys(2), 0, lds(2), 4, 0x20, need, None) == -5        # unaligned workspace
    assert hip.mtc_gemm_group_workspace_bytes(None, 2, 4, 1) == 0


def test_decode_once_workspace_by_shape(hip):
    """Prefill with at least max(512, K / 8) rows of X, 2^28 multiply-adds and no output column
    permutation takes the decode-once path: its workspace holds W_hat in bf16 (N x 64 * n_ksteps)
    and the staged X (the GEMM needs none), or the tile kernel's needs if those are larger (the
    call falls back to it without hipBLASLt). The shape alone decides."""
    big = _tdesc(K=1024, N=4096, n_ksteps=16, n_col_tiles=16)
    wt = 4096 * 1024 * 2
    ws = lambda d, M, xdt: hip.mtc_gemm_workspace_bytes(ctypes.byref(d), M, xdt)
    assert ws(big, 4096, 1) == wt                                         # bf16 X read in place, 256 tiles: no split
    assert ws(big, 4096, 0) == wt + 4096 * 1024 * 2                       # fp32 X staged as bf16
    part = lambda d, M, b: b % (M * d.N * 4) == 0 and 1 <= b // (M * d.N * 4) <= 64   # split-K partials only
    assert ws(big, 512, 1) >= wt
    assert part(big, 511, ws(big, 511, 1))                                # below 512 rows: the tile kernel
    deep = _tdesc(K=8192, N=2048, n_ksteps=128, n_col_tiles=8)           # K / 8 = 1024 rows
    assert ws(deep, 1024, 1) >= 2048 * 8192 * 2
    assert part(deep, 1023, ws(deep, 1023, 1))
    narrow = _tdesc(K=1024, N=256, n_ksteps=16, n_col_tiles=1)            # 2^28 multiply-adds from 1024 rows
    assert ws(narrow, 1024, 1) >= 256 * 1024 * 2
    assert part(narrow, 1023, ws(narrow, 1023, 1))
    rows = _tdesc(K=1024, N=4096, n_ksteps=16, n_col_tiles=16, row_perm=0x2000)
    assert ws(rows, 4096, 1) == wt + 4096 * 1024 * 2                      # a row permutation: X staged
    cols = _tdesc(K=1024, N=4096, n_ksteps=16, n_col_tiles=16, row_perm=0x2000, col_perm=0x3000)
    assert ws(cols, 4096, 1) == 4096 * 1024 * 2                           # a column permutation: tile kernel
    D = _abi.TileDescP
    small = _tdesc(K=1024, n_ksteps=16, row_perm=0x2000, col_perm=0x3000)
    descs = (D * 2)(ctypes.pointer(small), ctypes.pointer(big))
    assert hip.mtc_gemm_group_workspace_bytes(descs, 2, 4096, 1) == ws(small, 4096, 1) + wt
    # the fp32 path (mtc_gemm_f32): from 256 rows and 2^32 multiply-adds, the exact W_hat in fp32
    f32ws = lambda d, M: hip.mtc_gemm_f32_workspace_bytes(ctypes.byref(d), M)
    assert f32ws(big, 1024) == 4096 * 1024 * 4                           # 1024 x 1024 x 4096 = 2^32
    assert f32ws(rows, 1024) == 4096 * 1024 * 4 + 1024 * 1024 * 4         # and X gathered through row_perm
    assert f32ws(big, 1023) == 0                                          # below: the tile kernel (1024 tiles, no split)
    assert f32ws(cols, 1024) == 1024 * 1024 * 4                           # a column permutation: tile kernel, X gathered
    assert hip.mtc_set_prefill_decode_once(-1) == 1
    assert hip.mtc_set_prefill_decode_once(0) == 1
    assert hip.mtc_set_prefill_decode_once(-1) == 0
    assert ws(big, 4096, 1) == wt                                         # sizes do not follow the switch
    assert hip.mtc_set_prefill_decode_once(1) == 0


def _tdesc(**kw):
    d = _abi.MtcTileDesc()
    d.abi_version = _abi.ABI_VERSION
    d.K, d.N, d.n_ksteps, d.n_col_tiles = 256, 288, 4, 2
    d.payload_dwords = 64
    d.cells = d.step_off = d.payload = 0x1000
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def test_tile_descriptor_layout_and_validation(hip):
    fields = [f[0] for f in _abi.MtcTileDesc._fields_]
    src = "#include <stddef.h>\n#include <stdio.h>\n#include \"mtc_hip.h\"\nint main(void){\n"
    src += 'printf("%zu\\n", sizeof(mtc_tile_desc));\n'
    for f in fields:
        src += f'printf("%zu\\n", offsetof(mtc_tile_desc, {f}));\n'
    src += "return 0;}\n"
    with tempfile.TemporaryDirectory() as d:
        c, exe = os.path.join(d, "t.c"), os.path.join(d, "t")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I", INCLUDE, c, "-o", exe], check=True)
        out = [int(x) for x in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    assert out[0] == ctypes.sizeof(_abi.MtcTileDesc)
    assert out[1:] == [getattr(_abi.MtcTileDesc, f).offset for f in fields]
    assert hip.mtc_check_tile_desc(ctypes.byref(_tdesc())) == 0
    cases = {"abi_version": (4, -7), "N": (100, -2), "K": (252, -2), "n_ksteps": (3, -2), "n_col_tiles": (1, -2),
             "flags": (8, -2), "cells": (None, -1), "payload": (None, -1), "step_off": (None, -1)}
    for field, (val, code) in cases.items():
        assert hip.mtc_check_tile_desc(ctypes.byref(_tdesc(**{field: val}))) == code, field
    assert hip.mtc_check_tile_desc(None) == -1
    # gathered columns: bf16 scales and no col_perm only
    g = _abi.MTC_FLAG_COLS_GATHERED
    assert hip.mtc_check_tile_desc(ctypes.byref(_tdesc(flags=g))) == 0
    assert hip.mtc_check_tile_desc(ctypes.byref(_tdesc(flags=g | _abi.MTC_FLAG_FP32_SCALES))) == -2
    assert hip.mtc_check_tile_desc(ctypes.byref(_tdesc(flags=g, col_perm=0x2000))) == -2
    # payload past 2 GiB (32-bit byte offsets) is rejected
    assert hip.mtc_check_tile_desc(ctypes.byref(_tdesc(payload_dwords=0x7FFFFFFF // 4))) == 0
    assert hip.mtc_check_tile_desc(ctypes.byref(_tdesc(payload_dwords=0x7FFFFFFF // 4 + 1))) == -2


def test_rd_search_rejects_bad_block_size():
    rd = _native.rd_lib()
    F, D = _native.c_f32p, _native.c_f64p
    z = np.zeros(16, np.float32)
    hd = np.zeros(16, np.float64)
    out_d = np.zeros(4, np.float64)
    out_s = np.zeros(4, np.float32)
    rc = rd.mtc_rd_search(_native.ptr(z, F), _native.ptr(hd, D), _native.ptr(z, F), 1, 3, -2.0, 1.0, 2.0,
                          _native.ptr(z, F), 1, _native.ptr(z, F), 1, 0, 1, _native.ptr(out_d, D),
                          _native.ptr(out_s, F))
    assert rc == -1


def test_gpu_path_fails_loudly_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from tensorpack_amd.core.quadtree import QuadtreeRD
    from tensorpack_amd.kernels.gemm import MTCMatrix, mtc_gemm
    W = np.random.RandomState(0).randn(64, 64).astype(np.float32)
    m = MTCMatrix.from_quadtree(QuadtreeRD(W, None, (32, 16)).select(4.0), W)
    with pytest.raises(RuntimeError, match="GPU"):
        mtc_gemm(np.ones((1, 64), np.float32), m)
    with pytest.raises(RuntimeError, match="GPU"):
        m.to_array()


def test_batch_plan_sizes_and_errors(hip):
    """mtc_gemv_batch_plan is host arithmetic: sizes, the block -> member table, workspace
    slices of the split-K members, and argument errors, all without a GPU."""
    import numpy as np
    d1 = _desc()                                           # 2 panels x 2 chunks: split-K member
    d2 = _desc(K=256, chunk_rows=256, n_chunks=1)          # single chunk
    items = (_abi.MtcGemvBatchItem * 2)()
    for it, d in zip(items, (d1, d2)):
        it.desc = ctypes.pointer(d)
        it.X, it.ldx, it.Y, it.ldy = 0x10000, 256, 0x20000, 64
    plan_n, ws_n = ctypes.c_size_t(), ctypes.c_size_t()
    # units padded to 8 XCDs; one block per small unit (both column halves) for one-row tiles,
    # one per column half for two-row tiles
    for M, per_unit in ((1, 1), (2, 2)):
        assert hip.mtc_gemv_batch_plan(items, 2, M, None, 0, None, 0, ctypes.byref(plan_n), ctypes.byref(ws_n)) == 0
        blocks = 2 * 8 * per_unit
        assert plan_n.value >= blocks * 4 and ws_n.value > 0 and ws_n.value % 256 == 0
        raw = np.zeros(plan_n.value + 64, np.uint8)
        off = (-raw.ctypes.data) % 64
        plan = raw[off:off + plan_n.value]
        ws = 0x100000
        assert hip.mtc_gemv_batch_plan(items, 2, M, ws, ws_n.value, plan.ctypes.data, plan_n.value, None, None) == 0
        block_item = plan[-4 * blocks:].view(np.uint32)
        assert (block_item[:blocks // 2] == 0).all() and (block_item[blocks // 2:] == 1).all()
    assert hip.mtc_gemv_batch_plan(items, 2, 1, None, 0, None, 0, ctypes.byref(plan_n), ctypes.byref(ws_n)) == 0
    raw = np.zeros(plan_n.value + 64, np.uint8)
    off = (-raw.ctypes.data) % 64
    plan = raw[off:off + plan_n.value]
    # errors: empty batch, M = 0, missing X, mixed scale formats, plan or workspace too small
    assert hip.mtc_gemv_batch_plan(items, 0, 1, None, 0, None, 0, ctypes.byref(plan_n), None) == -3
    assert hip.mtc_gemv_batch_plan(items, 2, 0, None, 0, None, 0, ctypes.byref(plan_n), None) == -3
    items[1].X = None
    assert hip.mtc_gemv_batch_plan(items, 2, 1, None, 0, None, 0, ctypes.byref(plan_n), None) == -1
    items[1].X = 0x10000
    d3 = _desc(flags=_abi.MTC_FLAG_FP32_SCALES, leaf_scale=0x3000)
    items[1].desc = ctypes.pointer(d3)
    assert hip.mtc_gemv_batch_plan(items, 2, 1, None, 0, None, 0, ctypes.byref(plan_n), None) == -3
    items[1].desc = ctypes.pointer(d2)
    assert hip.mtc_gemv_batch_plan(items, 2, 1, ws, ws_n.value, plan.ctypes.data, 64, None, None) == -5
    assert hip.mtc_gemv_batch_plan(items, 2, 1, None, 0, plan.ctypes.data, plan_n.value, None, None) == -5
    assert hip.mtc_gemv_f32_batch(None, None, None) == -1
    bogus = np.zeros(256, np.uint8)
    assert hip.mtc_gemv_f32_batch(bogus.ctypes.data, 0x40000, None) == -2


def test_decode_workspace_and_lds_by_m_tile(hip):
    """Decode sizes are host arithmetic. M <= 4 runs one tile of 1, 2 or 4 rows on the vector
    path. 5 <= M <= 8 runs tiles of 8 rows on the matrix core, and so does M > 8 when a chunk is
    longer than 2048 rows. Otherwise M > 8 runs tiles of 16 rows. Matrix-core tiles add a
    staged copy of X, K x tile rows fp32 per tile, after the split-K area, 256-aligned.
    Expected byte counts are worked out by hand for K = 256, 2 panels x 2 chunks of 128 rows."""
    ref = ctypes.byref(_desc())
    # counters: 256 (one aligned line); partials: tiles x 2 panels x 2 chunks x rows x 32 x 4 B
    expect = {1: 256 + 512, 2: 256 + 1024, 4: 256 + 2048,
              5: 256 + 4096 + 256 * 8 * 4, 8: 256 + 4096 + 256 * 8 * 4,
              9: 256 + 8192 + 256 * 16 * 4, 16: 256 + 8192 + 256 * 16 * 4,
              17: 256 + 16384 + 2 * 256 * 16 * 4}
    for M, n in expect.items():
        assert hip.mtc_gemv_workspace_bytes(ref, M) == n, M
    # one chunk: no split-K area, only the staged X of the matrix-core tiles
    one = ctypes.byref(_desc(chunk_rows=256, n_chunks=1))
    assert hip.mtc_gemv_workspace_bytes(one, 4) == 0
    assert hip.mtc_gemv_workspace_bytes(one, 16) == 256 * 16 * 4
    # chunks of 4096 rows keep 8-row tiles at M = 16: two tiles
    big = ctypes.byref(_desc(K=8192, chunk_rows=4096, n_chunks=2))
    assert hip.mtc_gemv_workspace_bytes(big, 16) == 256 + 2 * 2 * 2 * 8 * 32 * 4 + 2 * 8192 * 8 * 4
    lds = hip.mtc_gemv_lds_bytes
    # the on-chip X of a matrix-core block is tile rows x chunk rows fp32, the rest is fixed
    for mt_m in (5, 16):
        assert lds(4096, 2048, 0, mt_m) - lds(4096, 1024, 0, mt_m) == (8 if mt_m == 5 else 16) * 1024 * 4
    assert lds(4096, 2048, 0, 9) == lds(4096, 2048, 0, 16) != lds(4096, 2048, 0, 8)
    assert lds(8192, 4096, 0, 16) == lds(8192, 4096, 0, 8)
    assert lds(4096, 2048, 1, 16) == lds(4096, 2048, 0, 16)     # no gather of X on the matrix core
    assert max(lds(4096, 2048, 0, 16), lds(8192, 4096, 0, 8)) <= 160 * 1024
    assert lds(0, 128, 0, 1) == lds(256, 128, 0, 0) == 0


def test_noalloc_entry_rejects_before_any_gpu_call(hip):
    """mtc_gemv_f32_noalloc checks arguments and the static scratch bound on the host."""
    d = _desc()                                                  # 2 row chunks: needs split-K scratch
    ref = ctypes.byref(d)
    cap = hip.mtc_gemv_noalloc_scratch_bytes()
    assert cap == 8 << 20
    assert hip.mtc_gemv_f32_noalloc(ref, None, 256, 0x10, 64, 1, None) == -1
    assert hip.mtc_gemv_f32_noalloc(ref, 0x10, 256, 0x10, 64, 0, None) == -3
    assert hip.mtc_gemv_f32_noalloc(ref, 0x10, 100, 0x10, 64, 1, None) == -3
    M = 1 << 16                                                  # partials far beyond the scratch
    assert hip.mtc_gemv_workspace_bytes(ref, M) > cap
    assert hip.mtc_gemv_f32_noalloc(ref, 0x10, 256, 0x10, 64, M, None) == -5
    assert b"scratch" in hip.mtc_last_error()
