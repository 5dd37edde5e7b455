"""Device residency of a panel stream and thin launch wrappers over the C-ABI.

PyTorch is used only as the device allocator and for the current HIP stream;
every computation goes through libmtc_hip.so. There is no CPU fallback: with
no GPU or no built library these functions raise.
"""

import ctypes
from typing import Dict, Optional, Tuple

import numpy as np

from . import _abi, _native
from .packer import LAYOUT_MX, PanelStream
from .tilestream import TileStream


def _torch():
    import torch
    return torch


def require_gpu(device=None):
    torch = _torch()
    if not torch.cuda.is_available():
        raise RuntimeError("mtc GPU path needs a ROCm GPU (torch.cuda.is_available() is False)")
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if dev.type != "cuda":
        raise ValueError(f"mtc GPU path runs on a cuda (ROCm) device, got {dev}")
    return dev if dev.index is not None else torch.device("cuda", torch.cuda.current_device())


def _need(ok: bool, what: str) -> None:
    """Argument check that stays on under python -O: the kernels trust these shapes."""
    if not ok:
        raise ValueError(what)


def current_stream_handle(device) -> int:
    torch = _torch()
    return torch.cuda.current_stream(device).cuda_stream


_DEV_ARRAYS = ("payload", "buckets", "unit_hdr", "leaf_word", "leaf_scale", "row_perm", "col_perm", "steps")


class DeviceStream:
    """A PanelStream uploaded to one GPU, plus its ctypes descriptor."""

    def __init__(self, ps: PanelStream, device=None):
        torch = _torch()
        self.device = require_gpu(device)
        self.host = ps
        self.lib = _native.hip_lib()

        def up(a: Optional[np.ndarray], dtype):
            if a is None:
                return None
            return torch.from_numpy(np.ascontiguousarray(a).view(dtype)).to(self.device)

        self.payload = up(ps.payload.view(np.int32), np.int32)
        self.buckets = up(ps.buckets.reshape(-1).view(np.int32), np.int32)
        self.unit_hdr = up(ps.unit_hdr.reshape(-1), np.int32)
        self.leaf_word = up(ps.leaf_word.view(np.int32), np.int32)
        self.leaf_scale = up(ps.leaf_scale, np.float32)
        self.row_perm = up(ps.row_perm, np.int32)
        self.col_perm = up(ps.col_perm, np.int32)
        self.steps = up(None if ps.steps is None else ps.steps.reshape(-1).view(np.int32), np.int32)

        d = _abi.MtcStreamDesc()
        d.abi_version = _abi.ABI_VERSION
        d.flags = (_abi.MTC_FLAG_FP32_SCALES if ps.leaf_scale is not None else 0) | \
            (_abi.MTC_FLAG_MX_LAYOUT if ps.layout == LAYOUT_MX else 0)
        d.K, d.N, d.chunk_rows = ps.K, ps.N, ps.chunk_rows
        d.n_panels, d.n_chunks = ps.n_panels, ps.n_chunks
        d.n_buckets = ps.n_buckets
        d.max_unit_words = int(ps.max_unit_words)
        d.max_unit_words4 = int(ps.max_unit_words4)
        d.fixed_steps = int(ps.fixed_steps)
        d.n_leaves = int(ps.leaf_word.size)
        d.payload_dwords = int(ps.payload.size)
        ptr = lambda t: None if t is None else t.data_ptr()
        d.payload, d.buckets, d.unit_hdr = ptr(self.payload), ptr(self.buckets), ptr(self.unit_hdr)
        d.leaf_word, d.leaf_scale = ptr(self.leaf_word), ptr(self.leaf_scale)
        d.row_perm, d.col_perm = ptr(self.row_perm), ptr(self.col_perm)
        d.steps = ptr(self.steps)
        d.n_steps = 0 if ps.steps is None else int(ps.steps.shape[0])
        self.desc = d
        _abi.check(self.lib, "mtc_check_desc", self.lib.mtc_check_desc(ctypes.byref(d)))
        self._ws: Dict[int, tuple] = {}                # HIP stream handle -> (bytes, tensor)

    def clone(self) -> "DeviceStream":
        """A second device copy of the same stream (distinct buffers, same contents)."""
        other = object.__new__(DeviceStream)
        other.device, other.host, other.lib = self.device, self.host, self.lib
        for name in _DEV_ARRAYS:
            t = getattr(self, name)
            setattr(other, name, None if t is None else t.clone())
        d = _abi.MtcStreamDesc.from_buffer_copy(self.desc)
        ptr = lambda t: None if t is None else t.data_ptr()
        d.payload, d.buckets, d.unit_hdr = ptr(other.payload), ptr(other.buckets), ptr(other.unit_hdr)
        d.leaf_word, d.leaf_scale = ptr(other.leaf_word), ptr(other.leaf_scale)
        d.row_perm, d.col_perm = ptr(other.row_perm), ptr(other.col_perm)
        d.steps = ptr(other.steps)
        other.desc = d
        other._ws = {}
        return other

    def device_bytes(self) -> int:
        n = 0
        for name in _DEV_ARRAYS:
            t = getattr(self, name)
            if t is not None:
                n += t.numel() * t.element_size()
        return n

    @property
    def K(self) -> int:
        return self.host.K

    @property
    def N(self) -> int:
        return self.host.N

    def nbytes(self) -> int:
        return self.host.nbytes()

    def workspace(self, M: int):
        """Zero-initialised GEMV workspace for M rows, one per HIP stream (its counters reset
        themselves at the end of each call, so calls ordered on one stream can share it;
        calls on different streams could overlap, so each stream gets its own)."""
        need = int(self.lib.mtc_gemv_workspace_bytes(ctypes.byref(self.desc), int(M)))
        if need == 0:
            return None, 0
        key = current_stream_handle(self.device)
        have = self._ws.get(key)
        if have is None or have[0] != need:
            torch = _torch()
            self._ws[key] = (need, torch.zeros(need, dtype=torch.uint8, device=self.device))
        return self._ws[key][1], need

    # ---- launches -------------------------------------------------------------------
    def dequant(self, out=None):
        torch = _torch()
        if out is None:
            out = torch.empty((self.K, self.N), dtype=torch.float32, device=self.device)
        _need(out.is_contiguous() and out.dtype == torch.float32 and tuple(out.shape) == (self.K, self.N)
              and out.device == self.device, f"out must be a contiguous ({self.K}, {self.N}) fp32 tensor on {self.device}")
        rc = self.lib.mtc_dequant(ctypes.byref(self.desc), out.data_ptr(), current_stream_handle(self.device))
        _abi.check(self.lib, "mtc_dequant", rc)
        return out

    def gemv_f32(self, X, out=None):
        torch = _torch()
        _need(X.dim() == 2 and X.dtype == torch.float32 and X.stride(1) == 1 and X.shape[1] == self.K
              and X.device == self.device, f"X must be (M, {self.K}) fp32 row-major on {self.device}")
        M = X.shape[0]
        if out is None:
            out = torch.empty((M, self.N), dtype=torch.float32, device=self.device)
        _need(out.dtype == torch.float32 and out.stride(1) == 1 and tuple(out.shape) == (M, self.N)
              and out.device == self.device, f"out must be ({M}, {self.N}) fp32 row-major on {self.device}")
        ws, nbytes = self.workspace(M)
        rc = self.lib.mtc_gemv_f32(ctypes.byref(self.desc), X.data_ptr(), X.stride(0), out.data_ptr(), out.stride(0),
                                   M, None if ws is None else ws.data_ptr(), nbytes,
                                   current_stream_handle(self.device))
        _abi.check(self.lib, "mtc_gemv_f32", rc)
        return out


def gemv_f32_group(streams, X, outs=None):
    """Y_i = X @ W_hat_i for 1..MAX_GROUP single-chunk streams that share X, in one launch
    (mtc_gemv_f32_group). Each Y_i is bit-identical to streams[i].gemv_f32(X)."""
    torch = _torch()
    streams = list(streams)
    n = len(streams)
    if not 1 <= n <= _abi.MAX_GROUP:
        raise ValueError(f"a group holds 1..{_abi.MAX_GROUP} matrices, got {n}")
    dev = streams[0].device
    if any(s.device != dev for s in streams):
        raise ValueError("group members live on different devices")
    _need(X.dim() == 2 and X.dtype == torch.float32 and X.stride(1) == 1 and X.shape[1] == streams[0].K,
          f"X must be (M, {streams[0].K}) fp32 row-major")
    if X.device != dev:
        raise ValueError(f"X is on {X.device}, the streams on {dev}")
    M = X.shape[0]
    if outs is None:
        outs = [torch.empty((M, s.N), dtype=torch.float32, device=dev) for s in streams]
    if len(outs) != n or any(o.device != dev for o in outs):
        raise ValueError("one output per member, on the members' device")
    for o, s in zip(outs, streams):
        _need(o.dtype == torch.float32 and o.stride(1) == 1 and tuple(o.shape) == (M, s.N),
              f"each output must be ({M}, N) fp32 row-major")
    descs = (_abi.DescP * n)(*[ctypes.pointer(s.desc) for s in streams])
    ys = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    lds = (ctypes.c_int64 * n)(*[o.stride(0) for o in outs])
    lib = streams[0].lib
    rc = lib.mtc_gemv_f32_group(descs, n, X.data_ptr(), X.stride(0), ys, lds, M, current_stream_handle(dev))
    _abi.check(lib, "mtc_gemv_f32_group", rc)
    return outs


def _aligned_host(nbytes: int, align: int = 64) -> np.ndarray:
    raw = np.zeros(nbytes + align, dtype=np.uint8)
    off = (-raw.ctypes.data) % align
    return raw[off:off + nbytes]


class GemvBatch:
    """A prepared batched decode launch (mtc_gemv_batch_plan + mtc_gemv_f32_batch): Y_i = X_i @
    W_hat_i for any number of streams, each with its own input and output, in one launch.

    The plan records device addresses of every stream array, X_i, Y_i and the batch's own
    workspace, so this object keeps them alive; `launch()` reruns the same products (new values
    written into the same X tensors are picked up). Every Y_i is bit-identical to
    streams[i].gemv_f32(X_i). Launches of one batch must not overlap in time (they share its
    workspace): issue them on one stream."""

    def __init__(self, streams, Xs, outs=None):
        torch = _torch()
        self.streams = list(streams)
        n = len(self.streams)
        if n < 1 or len(Xs) != n:
            raise ValueError("one input per stream, at least one stream")
        dev = self.streams[0].device
        self.device = dev
        M = Xs[0].shape[0]
        for s, X in zip(self.streams, Xs):
            if s.device != dev or X.device != dev:
                raise ValueError("batch members, inputs and outputs live on one device")
            _need(X.dim() == 2 and X.dtype == torch.float32 and X.stride(1) == 1 and X.shape == (M, s.K),
                  f"each X must be (M={M}, K) fp32 row-major")
        if outs is None:
            outs = [torch.empty((M, s.N), dtype=torch.float32, device=dev) for s in self.streams]
        if len(outs) != n:
            raise ValueError("one output per stream")
        for o, s in zip(outs, self.streams):
            _need(o.device == dev and o.dtype == torch.float32 and o.stride(1) == 1 and tuple(o.shape) == (M, s.N),
                  f"each output must be ({M}, N) fp32 row-major on {dev}")
        self.Xs, self.outs, self.M = list(Xs), list(outs), M
        lib = self.lib = self.streams[0].lib
        items = (_abi.MtcGemvBatchItem * n)()
        for it, s, X, o in zip(items, self.streams, self.Xs, self.outs):
            it.desc = ctypes.pointer(s.desc)
            it.X, it.ldx, it.Y, it.ldy = X.data_ptr(), X.stride(0), o.data_ptr(), o.stride(0)
        plan_n, ws_n = ctypes.c_size_t(), ctypes.c_size_t()
        _abi.check(lib, "mtc_gemv_batch_plan",
                   lib.mtc_gemv_batch_plan(items, n, M, None, 0, None, 0, ctypes.byref(plan_n), ctypes.byref(ws_n)))
        self.workspace = torch.zeros(ws_n.value, dtype=torch.uint8, device=dev) if ws_n.value else None
        self.host_plan = _aligned_host(plan_n.value)
        _abi.check(lib, "mtc_gemv_batch_plan",
                   lib.mtc_gemv_batch_plan(items, n, M, None if self.workspace is None else self.workspace.data_ptr(),
                                           ws_n.value, self.host_plan.ctypes.data, plan_n.value, None, None))
        self.device_plan = torch.from_numpy(self.host_plan.copy()).to(dev)
        torch.cuda.synchronize(dev)

    def launch(self):
        rc = self.lib.mtc_gemv_f32_batch(self.host_plan.ctypes.data, self.device_plan.data_ptr(),
                                         current_stream_handle(self.device))
        _abi.check(self.lib, "mtc_gemv_f32_batch", rc)
        return self.outs


class DeviceTiles:
    """A TileStream (prefill layout) uploaded to one GPU, plus its ctypes descriptor."""

    def __init__(self, ts: TileStream, device=None):
        torch = _torch()
        self.device = require_gpu(device)
        self.host = ts
        self.lib = _native.hip_lib()

        def up(a: Optional[np.ndarray]):
            if a is None:
                return None
            return torch.from_numpy(np.ascontiguousarray(a).reshape(-1).view(np.int32)).to(self.device)

        self.cells, self.step_off, self.payload = up(ts.cells), up(ts.step_off), up(ts.payload)
        self.row_perm, self.col_perm = up(ts.row_perm), up(ts.col_perm)
        d = _abi.MtcTileDesc()
        d.abi_version = _abi.ABI_VERSION
        d.flags = (_abi.MTC_FLAG_FP32_SCALES if ts.fp32_scales else 0) | \
                  (_abi.MTC_FLAG_COLS_GATHERED if ts.cols_gathered else 0)
        d.K, d.N, d.n_ksteps, d.n_col_tiles = ts.K, ts.N, ts.n_ksteps, ts.n_col_tiles
        d.payload_dwords = int(ts.payload.size)
        ptr = lambda t: None if t is None else t.data_ptr()
        d.cells, d.step_off, d.payload = ptr(self.cells), ptr(self.step_off), ptr(self.payload)
        d.row_perm, d.col_perm = ptr(self.row_perm), ptr(self.col_perm)
        self.desc = d
        _abi.check(self.lib, "mtc_check_tile_desc", self.lib.mtc_check_tile_desc(ctypes.byref(d)))

    @property
    def K(self) -> int:
        return self.host.K

    @property
    def N(self) -> int:
        return self.host.N

    def device_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.cells, self.step_off, self.payload, self.row_perm,
                                                           self.col_perm) if t is not None)

    def clone(self) -> "DeviceTiles":
        """A second device copy of the same tile stream (distinct buffers, same contents)."""
        other = object.__new__(DeviceTiles)
        other.device, other.host, other.lib = self.device, self.host, self.lib
        for name in ("cells", "step_off", "payload", "row_perm", "col_perm"):
            t = getattr(self, name)
            setattr(other, name, None if t is None else t.clone())
        d = _abi.MtcTileDesc.from_buffer_copy(self.desc)
        ptr = lambda t: None if t is None else t.data_ptr()
        d.cells, d.step_off, d.payload = ptr(other.cells), ptr(other.step_off), ptr(other.payload)
        d.row_perm, d.col_perm = ptr(other.row_perm), ptr(other.col_perm)
        other.desc = d
        return other

    def workspace(self, M: int, x_dtype: int, need: int = None):
        """The prefill workspace of an M-row call (prefill_workspace: shared by every matrix's calls
        on the current stream)."""
        if need is None:
            need = int(self.lib.mtc_gemm_workspace_bytes(ctypes.byref(self.desc), int(M), int(x_dtype)))
        if need == 0:
            return None, 0
        return prefill_workspace(self.device, need), need

    def gemm_bf16(self, X, out=None, out_dtype=None):
        torch = _torch()
        _need(X.dim() == 2 and X.stride(1) == 1 and X.dtype in (torch.float32, torch.bfloat16) and X.shape[1] == self.K
              and X.device == self.device, f"X must be (M, {self.K}) fp32 or bf16 row-major on {self.device}")
        M = X.shape[0]
        out_dtype = out_dtype or torch.float32
        if out is None:
            out = torch.empty((M, self.N), dtype=out_dtype, device=self.device)
        _need(out.dtype in (torch.float32, torch.bfloat16) and out.stride(1) == 1 and tuple(out.shape) == (M, self.N)
              and out.device == self.device, f"out must be ({M}, {self.N}) fp32 or bf16 row-major on {self.device}")
        xdt = _abi.MTC_DTYPE_BF16 if X.dtype == torch.bfloat16 else _abi.MTC_DTYPE_F32
        ydt = _abi.MTC_DTYPE_BF16 if out.dtype == torch.bfloat16 else _abi.MTC_DTYPE_F32
        ws, nbytes = self.workspace(M, xdt)
        rc = self.lib.mtc_gemm_bf16(ctypes.byref(self.desc), X.data_ptr(), xdt, _row_stride(X), out.data_ptr(), ydt,
                                    _row_stride(out), M, None if ws is None else ws.data_ptr(), nbytes,
                                    current_stream_handle(self.device))
        _abi.check(self.lib, "mtc_gemm_bf16", rc)
        return out

    def gemm_f32(self, X, out=None):
        """Y = X @ W_hat in fp32 on the matrix core (mtc_gemm_f32): the exact W_hat, fp32
        products and sums, for M from a few rows up."""
        torch = _torch()
        _need(X.dim() == 2 and X.stride(1) == 1 and X.dtype == torch.float32 and X.shape[1] == self.K
              and X.device == self.device, f"X must be (M, {self.K}) fp32 row-major on {self.device}")
        M = X.shape[0]
        if out is None:
            out = torch.empty((M, self.N), dtype=torch.float32, device=self.device)
        _need(out.dtype == torch.float32 and out.stride(1) == 1 and tuple(out.shape) == (M, self.N)
              and out.device == self.device, f"out must be ({M}, {self.N}) fp32 row-major on {self.device}")
        need = int(self.lib.mtc_gemm_f32_workspace_bytes(ctypes.byref(self.desc), int(M)))
        ws, nbytes = self.workspace(M, _abi.MTC_DTYPE_F32, need)
        rc = self.lib.mtc_gemm_f32(ctypes.byref(self.desc), X.data_ptr(), _row_stride(X), out.data_ptr(),
                                   _row_stride(out), M, None if ws is None else ws.data_ptr(), nbytes,
                                   current_stream_handle(self.device))
        _abi.check(self.lib, "mtc_gemm_f32", rc)
        return out


def set_prefill_decode_once(enable: bool) -> bool:
    """Switches the decode-once prefill path of gemm_bf16 / gemm_bf16_group on (the default) or
    off for the process (mtc_set_prefill_decode_once); returns the previous setting."""
    return bool(_native.hip_lib().mtc_set_prefill_decode_once(1 if enable else 0))


def _row_stride(T) -> int:
    """Elements between rows of a row-major matrix view; a single row's stride is never used, so
    it is given as the row length (a one-row slice of a wider matrix keeps the wide stride)."""
    return T.stride(0) if T.shape[0] > 1 else T.shape[1]


class GemmBatch:
    """A prepared batched prefill (mtc_gemm_batch_plan + mtc_gemm_bf16_batch): Y_i = X_i @ W_hat_i
    for any number of tile streams, each with its own input and output (one M, X dtype and Y
    dtype), in one staging, one tile and at most one reduction launch. The plan records the
    device addresses of the streams, inputs, outputs and the batch's workspace, so this object
    keeps them alive; `launch()` reruns the same products. Launches of one batch must not
    overlap in time (they share its workspace)."""

    def __init__(self, tiles, Xs, outs=None, out_dtype=None):
        torch = _torch()
        self.tiles = list(tiles)
        n = len(self.tiles)
        if n < 1 or len(Xs) != n:
            raise ValueError("one input per matrix, at least one matrix")
        dev = self.tiles[0].device
        self.device = dev
        M = Xs[0].shape[0]
        xdt_t = Xs[0].dtype
        for t, X in zip(self.tiles, Xs):
            if t.device != dev or X.device != dev:
                raise ValueError("batch members, inputs and outputs live on one device")
            _need(X.dim() == 2 and X.dtype == xdt_t and X.dtype in (torch.float32, torch.bfloat16)
                  and X.stride(1) == 1 and tuple(X.shape) == (M, t.K),
                  f"each X must be (M={M}, K) row-major, all fp32 or all bf16")
        out_dtype = out_dtype or torch.float32
        if outs is None:
            outs = [torch.empty((M, t.N), dtype=out_dtype, device=dev) for t in self.tiles]
        if len(outs) != n or len({o.dtype for o in outs}) != 1:
            raise ValueError("one output per matrix, all of one dtype")
        for o, t in zip(outs, self.tiles):
            _need(o.device == dev and o.dtype in (torch.float32, torch.bfloat16) and o.stride(1) == 1
                  and tuple(o.shape) == (M, t.N), f"each output must be ({M}, N) row-major on {dev}")
        self.Xs, self.outs, self.M = list(Xs), list(outs), M
        xdt = _abi.MTC_DTYPE_BF16 if xdt_t == torch.bfloat16 else _abi.MTC_DTYPE_F32
        ydt = _abi.MTC_DTYPE_BF16 if outs[0].dtype == torch.bfloat16 else _abi.MTC_DTYPE_F32
        lib = self.lib = self.tiles[0].lib
        items = (_abi.MtcGemmBatchItem * n)()
        for it, t, X, o in zip(items, self.tiles, self.Xs, self.outs):
            it.desc = ctypes.pointer(t.desc)
            it.X, it.ldx, it.Y, it.ldy = X.data_ptr(), _row_stride(X), o.data_ptr(), _row_stride(o)
        plan_n, ws_n = ctypes.c_size_t(), ctypes.c_size_t()
        _abi.check(lib, "mtc_gemm_batch_plan", lib.mtc_gemm_batch_plan(items, n, M, xdt, ydt, None, 0, None, 0,
                                                                       ctypes.byref(plan_n), ctypes.byref(ws_n)))
        self.workspace = torch.empty(ws_n.value, dtype=torch.uint8, device=dev) if ws_n.value else None
        self.host_plan = _aligned_host(plan_n.value)
        _abi.check(lib, "mtc_gemm_batch_plan",
                   lib.mtc_gemm_batch_plan(items, n, M, xdt, ydt,
                                           None if self.workspace is None else self.workspace.data_ptr(), ws_n.value,
                                           self.host_plan.ctypes.data, plan_n.value, None, None))
        self.device_plan = torch.from_numpy(self.host_plan.copy()).to(dev)
        torch.cuda.synchronize(dev)

    @property
    def launches(self) -> int:
        """Kernel launches per launch(): X staging if any member stages, the tile launch, and a
        reduction if any member splits K (header fields n_stage and n_reduce)."""
        n_stage, n_reduce = np.frombuffer(self.host_plan, dtype=np.int32, count=2, offset=32)
        return 1 + int(n_stage > 0) + int(n_reduce > 0)

    def launch(self):
        rc = self.lib.mtc_gemm_bf16_batch(self.host_plan.ctypes.data, self.device_plan.data_ptr(),
                                          current_stream_handle(self.device))
        _abi.check(self.lib, "mtc_gemm_bf16_batch", rc)
        return self.outs


_PREFILL_WS: dict = {}


def prefill_workspace(device, need: int):
    """A device buffer of at least `need` bytes for the prefill calls on the current HIP stream of
    `device`, shared by every matrix and group: calls ordered on one stream never overlap, calls on
    two streams may, so each stream has its own. The buffer only grows, to at least twice its last
    size, and a buffer it outgrows is kept, never freed: a HIP graph captured earlier still
    addresses it."""
    torch = _torch()
    key = (str(device), current_stream_handle(device))
    held = _PREFILL_WS.setdefault(key, [])
    if not held or held[-1].numel() < need:
        size = max(int(need), 2 * held[-1].numel() if held else 0)
        held.append(torch.empty(size, dtype=torch.uint8, device=device))
    return held[-1]


def gemm_bf16_group(tiles, X, outs=None, out_dtype=None):
    """Y_i = X @ W_hat_i for 1..MAX_GROUP tile streams that share X (same K), one launch per
    kernel (mtc_gemm_bf16_group). Each Y_i is bit-identical to tiles[i].gemm_bf16(X). The
    workspace is cached per device and HIP stream (calls on one stream are ordered; calls on
    two streams may overlap, so they do not share one)."""
    torch = _torch()
    tiles = list(tiles)
    n = len(tiles)
    if not 1 <= n <= _abi.MAX_GROUP:
        raise ValueError(f"a group holds 1..{_abi.MAX_GROUP} matrices, got {n}")
    dev = tiles[0].device
    if any(t.device != dev for t in tiles):
        raise ValueError("group members live on different devices")
    _need(X.dim() == 2 and X.stride(1) == 1 and X.dtype in (torch.float32, torch.bfloat16) and X.shape[1] == tiles[0].K,
          f"X must be (M, {tiles[0].K}) fp32 or bf16 row-major")
    if X.device != dev:
        raise ValueError(f"X is on {X.device}, the streams on {dev}")
    M = X.shape[0]
    out_dtype = out_dtype or torch.float32
    if outs is None:
        outs = [torch.empty((M, t.N), dtype=out_dtype, device=dev) for t in tiles]
    if len(outs) != n or any(o.device != dev for o in outs):
        raise ValueError("one output per member, on the members' device")
    for o, t in zip(outs, tiles):
        _need(o.dtype in (torch.float32, torch.bfloat16) and o.stride(1) == 1 and tuple(o.shape) == (M, t.N),
              f"each output must be ({M}, N) fp32 or bf16 row-major")
    if len({o.dtype for o in outs}) != 1:
        raise ValueError("group outputs must share one dtype")
    xdt = _abi.MTC_DTYPE_BF16 if X.dtype == torch.bfloat16 else _abi.MTC_DTYPE_F32
    ydt = _abi.MTC_DTYPE_BF16 if outs[0].dtype == torch.bfloat16 else _abi.MTC_DTYPE_F32
    lib = tiles[0].lib
    descs = (_abi.TileDescP * n)(*[ctypes.pointer(t.desc) for t in tiles])
    need = int(lib.mtc_gemm_group_workspace_bytes(descs, n, M, xdt))
    ws = prefill_workspace(dev, need) if need else None
    ys = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
    lds = (ctypes.c_int64 * n)(*[_row_stride(o) for o in outs])
    rc = lib.mtc_gemm_bf16_group(descs, n, X.data_ptr(), xdt, _row_stride(X), ys, ydt, lds, M,
                                 ws.data_ptr() if need else None, need, current_stream_handle(dev))
    _abi.check(lib, "mtc_gemm_bf16_group", rc)
    return outs
