"""HipBackend: the tensor-backend `Backend` contract on one MI355X.

Python mirror of the contract in packages/tensor-backend/src/index.ts:139-317
(same method names, argument meaning and error behaviour), driving
libhipbackend.so through ctypes.  Device work goes to one HIP stream; the
host keeps only metadata.

Design (MI355X-first, not a port of any reference backend):
- Tensors are (storage, element offset, shape, strides).  reshape /
  transpose / slice / split are zero-copy views; ops that need a layout
  the kernel cannot address make a strided copy first.
- Evaluation is partly lazy, which the contract allows (index.ts:7-8):
  `linear` / `quantizedLinear` return a pending result that a following
  `geglu` or `add` absorbs into the GEMM epilogue, and `rope` returns a
  pending rotation that `sdpa` applies while staging Q and K.  Anything else
  that touches a pending tensor launches it first; a pending tensor disposed
  unread is never computed (dead intermediates inside `scope`).
- `sdpa` writes its output physically as [B, L, H, D] and returns a
  [B, H, L, D] view of it, so the encoder's transpose + reshape back to
  [B, L, H*D] (modernbert/src/index.ts:352) is free.
- `layerNorm` and `geglu` of a pending linear are pending too.  When their
  first consumer is a linear layer that reads panel order (16-bit, K % 64 ==
  0, and M >= 4096 or, with 16-bit weights, the small-M slab kernel) they
  are written in panel order (laya_hip.h: 32 x 16 blocks in MFMA
  operand order), which the GEMM loads a whole block per instruction; any
  other reader gets a row-major copy (hb_panel_unpack).  Same values, bit
  for bit: only the addressing differs.
- Every output is rounded once per contract op, exactly as the op-by-op
  sequence would round it (the fused GEGLU and residual epilogues round the
  linear result before applying the next op).
"""
from __future__ import annotations

import json
import math
from typing import Any, Callable, Optional, Sequence

import numpy as np

from . import ffi as F
from .host import (FLOATS, NP_DTYPE, HostQuantized, HostTensor, QuantizedTensor, quant_groups, to_f32,
                   validate_quantized)

# storage dtypes: name -> (code, bytes)
DT = {
    "f32": (F.HB_F32, 4), "f16": (F.HB_F16, 2), "bf16": (F.HB_BF16, 2), "i32": (F.HB_I32, 4),
    "bool": (F.HB_BOOL, 1), "u8": (F.HB_U8, 1), "i8": (F.HB_I8, 1), "u16": (F.HB_U16, 2), "i16": (F.HB_I16, 2),
    "u32": (F.HB_U32, 4),
}
# host dtypes stored widened (Backend.fromHost may widen, index.ts:146-153)
WIDEN = {"f64": "f32", "i64": "i32", "u64": "i32"}
FLOAT_DT = ("f32", "f16", "bf16")


def _contig(shape) -> tuple:
    st = []
    acc = 1
    for d in reversed(shape):
        st.append(acc)
        acc *= d
    return tuple(reversed(st))


def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= d
    return n


def _promote(a: str, b: str) -> str:
    if a == b:
        return a
    fa, fb = a in FLOAT_DT, b in FLOAT_DT
    if fa and fb:
        return "f32"
    if fa:
        return a
    if fb:
        return b
    return "i32"


def _broadcast_shape(*shapes) -> tuple:
    r = max(len(s) for s in shapes)
    out = []
    for i in range(r):
        dims = [s[len(s) - r + i] if len(s) - r + i >= 0 else 1 for s in shapes]
        m = max(dims)
        for d in dims:
            if d != 1 and d != m:
                raise ValueError(f"shapes {[list(s) for s in shapes]} do not broadcast")
        out.append(m if all(d != 0 for d in dims) else 0)
    return tuple(out)


class _Storage:
    __slots__ = ("ptr", "nbytes", "refs", "owner", "cache")

    def __init__(self, owner: "HipBackend", ptr: int, nbytes: int):
        self.owner = owner
        self.ptr = ptr
        self.nbytes = nbytes
        self.refs = 1
        # device summaries derived from this storage's contents, created on
        # first use: key -> [device pointer, fresh]
        self.cache: Optional[dict] = None

    def retain(self):
        self.refs += 1
        return self

    def release(self):
        self.refs -= 1
        if self.refs == 0 and self.ptr:
            if self.cache:
                for ent in self.cache.values():
                    self.owner._free(ent[0])
            self.cache = None
            self.owner._recycle(self.ptr, self.nbytes)
            self.ptr = 0


class HipTensor:
    """Opaque handle: `shape` and `dtype` are public (index.ts:75-78)."""
    __slots__ = ("shape", "dtype", "_st", "_off", "_strides", "_lazy", "_dead", "_meta", "__weakref__")

    def __init__(self, shape, dtype, st: Optional[_Storage], off: int = 0, strides=None, lazy=None):
        self.shape = tuple(map(int, shape))
        self.dtype = dtype
        self._st = st
        self._off = off
        self._strides = tuple(strides) if strides is not None else _contig(self.shape)
        self._lazy = lazy
        self._dead = False
        self._meta: Optional[dict] = None  # created on first use

    @property
    def size(self) -> int:
        return _numel(self.shape)

    def __repr__(self):
        state = "disposed" if self._dead else ("pending" if self._lazy else "ready")
        return f"HipTensor({self.dtype}{list(self.shape)}, {state})"


# ------------------------------------------------------------------ pending work

PANEL_MIN_M = 4096  # the large-M GEMM; below it the small-M slab kernel also takes panel-order operands
SLAB_LDS = 160 * 1024  # the slab kernel's LDS: 64 * K bytes per 32 output columns (x2 with GeGLU)


def _slab_path(M: int, n_out: int, K: int, geglu: bool, cus: int) -> bool:
    """hb_linear takes the small-M slab kernel (16-bit weights, M < 4096):
    the conditions of slab_path in csrc/gemm_kernels.h."""
    return (M < PANEL_MIN_M and K % 64 == 0 and 64 * K * (2 if geglu else 1) <= SLAB_LDS
            and -(-n_out // 32) * -(-M // 128) <= cus)


def _panel_rows(M: int) -> int:
    return (M + 31) // 32 * 32


class _PanelRows:
    """The value of a tensor, an [M, K] 16-bit matrix, held in panel order
    (rows padded to a multiple of 32) in `st`, written for a linear layer that
    reads panel order.  Other readers get a row-major copy (HipBackend._ready): the
    LayerNorm it came from run again row-major (`norm`, same bits), or an
    unpack of the panel."""

    def __init__(self, st, M: int, K: int, norm: Optional["_PendingNorm"] = None):
        self.st, self.M, self.K, self.norm = st, M, K, norm

    def release(self):
        if self.st is not None:
            self.st.release()
            self.st = None
        if self.norm is not None:
            self.norm.release()
            self.norm = None


class _PendingNorm:
    """layerNorm not yet launched (index.ts:216-217): row-major on first
    use, or panel order when a linear layer that reads it consumes it first."""

    def __init__(self, be, x, weight, bias, eps: float, dt: str):
        st, xp, rows, D, ld = be._rows(x)
        self.refs = [st.retain()]
        wdt = None
        wp = bp = 0
        if weight is not None:
            self.refs.append(weight._st.retain())
            wp, wdt = be._ptr(weight), weight.dtype
        if bias is not None:
            self.refs.append(bias._st.retain())
            bp, wdt = be._ptr(bias), bias.dtype
        self.args = (DT[x.dtype][0], xp, ld, DT[wdt or "f32"][0], wp, bp)
        self.rows, self.D, self.eps, self.dt = rows, D, float(eps), dt
        # hb_layernorm_panel's conditions
        pal = 16 if wdt == "f32" else 8
        self.panel_ok = (x.dtype in ("f16", "bf16") and dt == x.dtype and D % 256 == 0 and D <= 2048 and
                         ld % 8 == 0 and xp % 16 == 0 and wdt in (None, "f16", "bf16", "f32") and wp % pal == 0 and
                         bp % pal == 0)

    def release(self):
        for s in self.refs:
            s.release()
        self.refs = []


class _PendingLinear:
    """y = x . w^T (+bias) not yet launched.  Captures device addresses and
    holds a reference on every operand's storage, so the caller may dispose
    the operand tensors before the launch.  `epi` is HB_EPI_GEGLU once a
    geglu has absorbed it; `panel` (a _PanelRows) when x is in panel order."""

    def __init__(self, be, x, w, bias, q=None, panel=None):
        self.be = be
        self.epi = 0
        self.panel = panel
        if panel is not None:
            self.x = (panel.st.ptr, panel.M, panel.K, panel.K)
            self.refs = [panel.st.retain(), w._st.retain()]
        else:
            st, xp, M, K, ldx = be._rows(x)
            self.x = (xp, M, K, ldx)
            self.refs = [st.retain(), w._st.retain()]
        self.wp = be._ptr(w)
        self.bp = 0
        if bias is not None:
            self.refs.append(bias._st.retain())
            self.bp = be._ptr(bias)
        self.q = None
        if q is not None:
            scales, zeros, bits, group, mode, n = q
            self.refs.append(scales._st.retain())
            zp = 0
            if zeros is not None:
                self.refs.append(zeros._st.retain())
                zp = be._ptr(zeros)
            self.q = (be._ptr(scales), zp, bits, group, 1 if mode == "affine" else 0)
        self.N = w.shape[0] if q is None else q[5]
        self.dtype = x.dtype
        M, K = self.x[1], self.x[2]
        # the operand conditions of the MFMA kernels that take panel-order
        # operands (hb_linear / hb_qlinear's, on everything but the output and
        # the residual, which are checked at launch); arow_ok: the large-M one
        ok = x.dtype in ("f16", "bf16") and K % 64 == 0 and self.x[0] % 16 == 0
        if q is None:
            ok = ok and self.wp % 16 == 0
        else:
            sp, zp, bits, group, mode = self.q
            ok = ok and self.wp % 8 == 0 and sp % 2 == 0 and zp % 2 == 0 and group % 8 == 0
        self.operands_ok = ok
        self.arow_ok = ok and M >= PANEL_MIN_M

    def takes_panel(self, epi: int) -> bool:
        """The launch with epilogue `epi` takes a kernel that reads and
        writes panel order: the large-M one, or (16-bit weights) the slab."""
        if self.arow_ok:
            return True
        M, K = self.x[1], self.x[2]
        geglu = bool(epi & F.HB_EPI_GEGLU)
        n_out = self.N // 2 if geglu else self.N
        return self.operands_ok and self.q is None and _slab_path(M, n_out, K, geglu, self.be.cus)

    def fork(self, epi: int) -> "_PendingLinear":
        """The same product with epilogue `epi` (own references)."""
        c = object.__new__(_PendingLinear)
        c.__dict__.update(self.__dict__)
        c.refs = [s.retain() for s in self.refs]
        c.epi = epi
        return c

    @property
    def n_out(self) -> int:
        return self.N // 2 if self.epi & F.HB_EPI_GEGLU else self.N

    def release(self):
        for s in self.refs:
            s.release()
        self.refs = []

    def launch(self, y_ptr: int, ldy: int, flags: int = 0, resid=(0, 0)):
        be = self.be
        xp, M, K, ldx = self.x
        flags |= self.epi
        if self.bp:
            flags |= F.HB_EPI_BIAS
        if resid[0]:
            flags |= F.HB_EPI_RESID
        tmp = None
        if self.panel is not None:
            if (resid[0] and (resid[0] % 16 or resid[1] % 8)) or not self.takes_panel(flags):
                # a residual the MFMA kernels cannot read, or a launch that
                # takes a kernel without panel operands: unpack x first
                tmp = be._malloc(M * K * 2)
                be._call("linear", "hb_panel_unpack", be.ctx, xp, tmp.ptr, K, M, K)
                xp, ldx = tmp.ptr, K
            else:
                flags |= F.HB_X_PANEL
        N = self.N // 2 if flags & F.HB_EPI_GEGLU else self.N
        dt = DT[self.dtype][0]
        try:
            if self.q is None:
                be._call("linear", "hb_linear", be.ctx, dt, xp, ldx, self.wp, self.bp, resid[0], resid[1], y_ptr,
                         ldy, M, N, K, flags)
            else:
                sp, zp, bits, group, mode = self.q
                be._call("quantizedLinear", "hb_qlinear", be.ctx, dt, xp, ldx, self.wp, sp, zp, self.bp, resid[0],
                         resid[1], y_ptr, ldy, M, N, K, bits, group, mode, flags)
        finally:
            if tmp is not None:
                tmp.release()


class _PendingRope:
    """rope not yet launched (index.ts:225-229): applied by sdpa while it
    stages q / k, or by hb_linear_qkv when x is a view of the pending q / k / v
    projection (`lin`, a _SharedLinear; src's storage is None until that
    product is launched row-major)."""

    def __init__(self, be, x, base):
        self.be = be
        self.x = x
        self.base = float(base)
        self.lin = x._lazy.share() if isinstance(x._lazy, _SharedLinear) else None
        self.ref = x._st.retain() if self.lin is None else None
        self.src = (x._st, x._off, x._strides, x.dtype, x.shape)

    def source(self):
        """(storage, offset, strides, dtype, shape) of the unrotated input,
        launching a pending product row-major first."""
        if self.lin is not None and self.src[0] is None:
            st = self.lin.rowmajor()
            self.ref = st.retain()
            self.src = (st,) + self.src[1:]
        return self.src

    def release(self):
        if self.ref is not None:
            self.ref.release()
            self.ref = None
        if self.lin is not None:
            self.lin.release()
            self.lin = None


class _SharedLinear:
    """A pending plain linear whose result has only been viewed so far
    (reshape / transpose / slice keep their strides over the [M, N] output).
    The views share this object; the first reader launches the product
    row-major (`rowmajor`).  sdpa on roped q / k views and the v view of the
    stacked q / k / v projection, laid out as ModernBert.layer takes them
    (modernbert/src/index.ts:348-351), instead launches hb_linear_qkv once
    (`fused`): the product written head-major with the q and k heads rotated,
    the values a separate linear, transpose / split and rope would store."""

    def __init__(self, be, lin: "_PendingLinear", M: int, N: int, dtype: str):
        self.be, self.lin, self.M, self.N, self.dtype = be, lin, M, N, dtype
        self.users = 1
        self.st = None       # the row-major output, once launched
        self.fused_st = {}   # (rope base, L, H) -> storage of the head-major [3, B, H, L, 64] output

    def share(self) -> "_SharedLinear":
        self.users += 1
        return self

    def release(self):
        self.users -= 1
        if self.users == 0:
            self.lin.release()
            if self.st is not None:
                self.st.release()
                self.st = None
            for st in self.fused_st.values():
                st.release()
            self.fused_st = {}

    def rowmajor(self):
        if self.st is None:
            be = self.be
            self.st = be._malloc(self.M * self.N * DT[self.dtype][1])
            be.stats["linear"] += 1
            self.lin.launch(self.st.ptr, self.N)
        return self.st

    def qkv_ok(self) -> bool:
        """hb_linear_qkv's conditions on the product itself."""
        lin = self.lin
        return (lin.epi == 0 and lin.q is None and lin.bp == 0 and lin.arow_ok and self.dtype in ("f16", "bf16")
                and self.N % 192 == 0 and lin.x[2] % 64 == 0 and lin.wp % 16 == 0)

    def fused(self, base: float, L: int, H: int):
        key = (float(base), L, H)
        st = self.fused_st.get(key)
        if st is None:
            be, lin = self.be, self.lin
            xp, M, K, ldx = lin.x
            st = be._malloc(M * self.N * DT[self.dtype][1])
            flags = F.HB_X_PANEL if lin.panel is not None else 0
            be.stats["linear"] += 1
            be.stats["linear_fused_qkv"] += 1
            be._call("linear", "hb_linear_qkv", be.ctx, DT[self.dtype][0], xp, ldx, lin.wp, 0, st.ptr, M, K, L,
                     H, float(base), flags)
            self.fused_st[key] = st
        return st


class _PendingSdpa:
    """sdpa not yet launched (index.ts:230-237).  The result and the views
    taken of it (transpose / reshape keep their strides over the output's
    physical [B, Lq, H, D] storage) share this object; the first reader
    launches it: row-major for most, or in panel order for a linear layer
    that reads panel order reading the contiguous [B*Lq, H*D] view (modernbert's merged
    heads into attn Wo).  Holds a reference on every operand's storage."""

    def __init__(self, be, args, refs, panel_ok: bool):
        self.be, self.args, self.refs, self.panel_ok = be, args, refs, panel_ok
        self.users = 1
        self.st = None  # the row-major output, once launched
        dtc, *_rest = args
        B, H, Lq, D = args[10], args[11], args[12], args[14]
        self.M, self.K, self.es = B * Lq, H * D, 4 if dtc == F.HB_F32 else 2

    def share(self) -> "_PendingSdpa":
        self.users += 1
        return self

    def release(self):
        self.users -= 1
        if self.users == 0:
            for s in self.refs:
                s.release()
            self.refs = []
            if self.st is not None:
                self.st.release()
                self.st = None

    def _count(self):
        be = self.be
        be.stats["sdpa"] += 1
        if self.args[16] or self.args[17]:
            be.stats["sdpa_fused_rope"] += 1

    def rowmajor(self):
        if self.st is None:
            be = self.be
            dtc, qp, qs, kp, ks, vp, vs, mp, ms, info, B, H, Lq, Lk, D, scale, rq, rk = self.args
            self.st = be._malloc(B * Lq * H * D * self.es)
            if B * H * Lq:
                self._count()
                be._call("sdpa", "hb_sdpa", be.ctx, dtc, qp, F.i64s(qs), kp, F.i64s(ks), vp, F.i64s(vs), mp,
                         F.i64s(ms) if ms is not None else None, info, self.st.ptr, F.i64s((Lq * H * D, D, H * D, 1)),
                         B, H, Lq, Lk, D, float(scale), rq, rk)
        return self.st

    def panel(self):
        be = self.be
        dtc, qp, qs, kp, ks, vp, vs, mp, ms, info, B, H, Lq, Lk, D, scale, rq, rk = self.args
        st = be._malloc(_panel_rows(self.M) * self.K * self.es)
        self._count()
        be._call("sdpa", "hb_sdpa_panel", be.ctx, dtc, qp, F.i64s(qs), kp, F.i64s(ks), vp, F.i64s(vs), mp,
                 F.i64s(ms) if ms is not None else None, info, st.ptr, B, H, Lq, Lk, D, float(scale), rq, rk)
        return st


# ------------------------------------------------------------------ recorded graphs

def _flat_outputs(out, op: str) -> list:
    """The tensors of a tensor, list or tuple result."""
    ts = [out] if isinstance(out, HipTensor) else list(out) if isinstance(out, (list, tuple)) else None
    if ts is None or not all(isinstance(t, HipTensor) for t in ts):
        raise TypeError(f"{op}: the function must return a tensor or a list / tuple of tensors")
    return ts


class HipGraph:
    """An op sequence recorded by HipBackend.capture.  run() replays it on
    the backend's stream and returns the output (a tensor, or the list /
    tuple the recorded function returned: the same tensors each time,
    rewritten by the replay; they belong to the caller, who disposes them
    after destroy())."""

    def __init__(self, be: "HipBackend", exec_: int, out, held: list):
        self.be, self.exec, self.out, self.held = be, exec_, out, held
        # the graph writes them
        self._sts = [t._st.retain() for t in _flat_outputs(out, "capture") if t._st is not None]

    def run(self):
        if not self.exec or self.be._destroyed:
            raise RuntimeError("HipGraph: used after destroy()")
        self.be._call("graph", "hb_graph_launch", self.be.ctx, self.exec)
        return self.out

    def destroy(self) -> None:
        if not self.exec:
            return
        be = self.be
        if not be._destroyed:
            be._call("graph", "hb_graph_destroy", be.ctx, self.exec)
            for ptr, nbytes in self.held:  # reused only by work enqueued after the last replay
                be._recycle(ptr, nbytes)
        self.held = []
        self.exec = 0
        for st in self._sts:
            st.release()
        self._sts = []


# ------------------------------------------------------------------ backend

class HipBackend:
    """The `Backend` contract on libhipbackend (one device, one stream)."""

    name = "hip"

    def __init__(self, device: int = 0, lib_path: str | None = None, fuse_qkv: bool = False):
        """`fuse_qkv`: launch an attention block's q / k / v projection as
        hb_linear_qkv (the product written head-major with RoPE applied in the
        GEMM's epilogue) when sdpa consumes it as ModernBert.layer does.  Off
        by default: on the ModernBERT-base shape it is slower than rotating q
        and k while sdpa stages them."""
        self.fuse_qkv = bool(fuse_qkv)
        self.n = F.native(lib_path)
        ctx = F.U(0)
        self.n.call("createHipBackend", "hb_init", device, F.C.byref(ctx))
        self.ctx = ctx.value
        self._scopes: list[list[HipTensor]] = []
        self._destroyed = False
        self._profiling = None  # list of (key, start event, end event) while profiling
        self._prof_only = self._LAUNCHES
        self._event_pool: list[int] = []
        self._blocks: dict[int, list[int]] = {}
        self._capture_held: Optional[list] = None  # blocks disposed while a capture records
        self._capture_summaries: Optional[set] = None  # summaries already enqueued into the recording
        self._compiled: list = []  # release functions of compile() wrappers
        self._cus: Optional[int] = None  # compute units, read once (HipBackend.cus)
        self.stats = {"linear": 0, "linear_fused_geglu": 0, "linear_fused_resid": 0, "linear_fused_qkv": 0, "sdpa": 0,
                      "sdpa_fused_rope": 0, "copies": 0, "panel_unpacks": 0}

    # ---------------------------------------------------------------- plumbing
    # kernel-launching entry points (timed per op key while profiling)
    _LAUNCHES = frozenset(("hb_linear", "hb_linear_qkv", "hb_qlinear", "hb_qgather", "hb_layernorm", "hb_layernorm_panel",
                           "hb_panel_unpack", "hb_panel_pack", "hb_rope", "hb_sdpa", "hb_sdpa_mask_info", "hb_geglu",
                           "hb_unary", "hb_binary", "hb_where", "hb_gather", "hb_reduce", "hb_scan", "hb_meanpool"))

    def _call(self, op: str, name: str, *args):
        prof = self._profiling
        if prof is not None and name in self._prof_only:
            a, b = self._take_event(), self._take_event()
            self.n.call(op, "hb_event_record", self.ctx, a)
            self.n.call(op, name, *args)
            self.n.call(op, "hb_event_record", self.ctx, b)
            key = op
            if name == "hb_linear_qkv":
                key = f"{op}[M={args[7]},N={3 * 64 * args[10]},K={args[8]},qkv]"
            elif name in ("hb_linear", "hb_qlinear"):
                key = f"{op}[M={args[10]},N={args[11]},K={args[12]}{',geglu' if args[-1] & F.HB_EPI_GEGLU else ''}]" \
                    if name == "hb_linear" else f"{op}[M={args[12]},N={args[13]},K={args[14]},q{args[15]}]"
            prof.append((key, a, b))
        else:
            self.n.call(op, name, *args)

    def _take_event(self) -> int:
        if self._event_pool:
            return self._event_pool.pop()
        ev = F.U(0)
        self.n.call("profile", "hb_event_create", self.ctx, F.C.byref(ev))
        return ev.value

    def startProfiling(self, only=None) -> None:
        """Times every kernel launch with HIP events on the stream, like the
        reference's Runtime.startProfiling (backend-webgpu/src/runtime.ts:420-464).
        `only`: a set of entry-point names (e.g. {"hb_linear"}) to time instead
        of every launch."""
        self._prof_only = self._LAUNCHES if only is None else frozenset(only) & self._LAUNCHES
        self._profiling = []

    def stopProfiling(self) -> dict:
        """Waits for the stream; returns {op key: (launches, total GPU ms)}."""
        prof, self._profiling = self._profiling or [], None
        out: dict = {}
        for key, a, b in prof:
            ms = F.C.c_float(0)
            self.n.call("profile", "hb_event_elapsed", a, b, F.C.byref(ms))
            n, t = out.get(key, (0, 0.0))
            out[key] = (n + 1, t + ms.value)
            self._event_pool.extend((a, b))
        return out

    def device_info(self) -> dict:
        buf = F.C.create_string_buffer(1024)
        self._call("deviceInfo", "hb_device_info", self.ctx, buf, 1024)
        return json.loads(buf.value.decode())

    @property
    def cus(self) -> int:
        """The device's compute units (the small-M GEMM's grid condition)."""
        if self._cus is None:
            self._cus = int(self.device_info()["cus"])
        return self._cus

    # Blocks of disposed tensors wait in `_blocks` (size class -> pointers)
    # for the next allocation of the same class, without a call into the
    # library either way.  The library's pool is stream-ordered on the one
    # stream, and so is this: a block handed out again is only written by
    # work queued after everything that read it.  The size classes are the
    # library's (runtime.hip, size_class).
    @staticmethod
    def _size_class(nbytes: int) -> int:
        n = max(1, nbytes)
        if n <= 65536:
            return (n + 255) & ~255
        step = (1 << (n - 1).bit_length()) // 16
        return (n + step - 1) // step * step

    def _malloc(self, nbytes: int) -> _Storage:
        if self._destroyed:
            raise RuntimeError("hip backend: used after destroy()")
        sc = self._size_class(nbytes)
        free = self._blocks.get(sc)
        if free:
            return _Storage(self, free.pop(), nbytes)
        p = F.U(0)
        try:
            self._call("alloc", "hb_alloc", self.ctx, sc, F.C.byref(p))
        except RuntimeError:
            if not any(self._blocks.values()):
                raise
            self._return_blocks()  # hand the waiting blocks back to the library and retry once
            self._call("alloc", "hb_alloc", self.ctx, sc, F.C.byref(p))
        return _Storage(self, p.value, nbytes)

    def _recycle(self, ptr: int, nbytes: int):
        if self._destroyed:
            return
        if self._capture_held is not None:  # a replay of the graph being recorded still writes it
            self._capture_held.append((ptr, nbytes))
            return
        self._blocks.setdefault(self._size_class(nbytes), []).append(ptr)

    def _return_blocks(self):
        for ptrs in self._blocks.values():
            for ptr in ptrs:
                self._free(ptr)
        self._blocks.clear()

    def _free(self, ptr: int):
        if not self._destroyed:
            self._call("dispose", "hb_free", self.ctx, ptr)

    def _track(self, t: HipTensor) -> HipTensor:
        if self._scopes:
            self._scopes[-1].append(t)
        return t

    def _new(self, shape, dtype: str) -> HipTensor:
        shape = tuple(int(d) for d in shape)
        st = self._malloc(_numel(shape) * DT[dtype][1])
        return self._track(HipTensor(shape, dtype, st))

    def _view(self, t: HipTensor, shape, strides, off) -> HipTensor:
        return self._track(HipTensor(shape, t.dtype, t._st.retain(), off, strides))

    def _live(self, *ts, op="op"):
        for t in ts:
            if t is None:
                continue
            if not isinstance(t, HipTensor):
                raise TypeError(f"{op}: expected a hip tensor, got {type(t).__name__}")
            if t._dead:
                raise RuntimeError(f"{op}: tensor used after dispose")

    def _ready(self, t: HipTensor) -> HipTensor:
        """Launches pending work of `t` into its own storage."""
        if t._lazy is None:
            return t
        lz = t._lazy
        t._lazy = None
        if isinstance(lz, _PendingLinear):
            st = self._malloc(_numel(t.shape) * DT[t.dtype][1])
            t._st, t._off, t._strides = st, 0, _contig(t.shape)
            self.stats["linear"] += 1
            lz.launch(st.ptr, lz.n_out)
            lz.release()
        elif isinstance(lz, _PendingNorm):
            st = self._malloc(_numel(t.shape) * DT[t.dtype][1])
            t._st, t._off, t._strides = st, 0, _contig(t.shape)
            dtx, xp, ld, dtw, wp, bp = lz.args
            if lz.rows:
                self._call("layerNorm", "hb_layernorm", self.ctx, dtx, xp, ld, dtw, wp, bp, DT[lz.dt][0], st.ptr,
                           lz.rows, lz.D, lz.eps)
            lz.release()
        elif isinstance(lz, _PendingSdpa):
            t._st = lz.rowmajor().retain()  # t keeps its view (offset, strides) of the [B, Lq, H, D] output
            lz.release()
        elif isinstance(lz, _SharedLinear):
            t._st = lz.rowmajor().retain()  # t keeps its view (offset, strides) of the [M, N] output
            lz.release()
        elif isinstance(lz, _PanelRows):
            st = self._malloc(_numel(t.shape) * DT[t.dtype][1])
            t._st, t._off, t._strides = st, 0, _contig(t.shape)
            if lz.norm is not None:
                nm = lz.norm
                dtx, xp, ld, dtw, wp, bp = nm.args
                self._call("layerNorm", "hb_layernorm", self.ctx, dtx, xp, ld, dtw, wp, bp, DT[nm.dt][0], st.ptr,
                           nm.rows, nm.D, nm.eps)
            else:
                self.stats["panel_unpacks"] += 1
                self._call("read", "hb_panel_unpack", self.ctx, lz.st.ptr, st.ptr, lz.K, lz.M, lz.K)
            lz.release()
        elif isinstance(lz, _PendingRope):
            src_st, off, strides, dtype, shape = lz.source()
            st = self._malloc(_numel(t.shape) * DT[t.dtype][1])
            t._st, t._off, t._strides = st, 0, _contig(t.shape)
            B, H, L, D = self._bhld(shape)
            xs = self._bhld_strides(shape, strides)
            self._call("rope", "hb_rope", self.ctx, DT[dtype][0], src_st.ptr + off * DT[dtype][1], F.i64s(xs),
                       DT[t.dtype][0], st.ptr, B, H, L, D, lz.base)
            lz.release()
        return t

    def _as_panel(self, x: HipTensor) -> Optional[_PanelRows]:
        """x's value in panel order for a linear layer that reads it: already there,
        or written so now if x is a pending layerNorm or a pending GeGLU
        linear that can write it; else None."""
        lz = x._lazy
        if isinstance(lz, _PanelRows):
            return lz
        if isinstance(lz, _PendingNorm) and lz.panel_ok and lz.D % 64 == 0:
            st = self._malloc(_panel_rows(lz.rows) * lz.D * 2)
            dtx, xp, ld, dtw, wp, bp = lz.args
            self._call("layerNorm", "hb_layernorm_panel", self.ctx, dtx, xp, ld, dtw, wp, bp, st.ptr, lz.rows, lz.D,
                       lz.eps)
            x._lazy = _PanelRows(st, lz.rows, lz.D, norm=lz)  # keeps the LayerNorm's operands
            return x._lazy
        if (isinstance(lz, _PendingSdpa) and lz.panel_ok and x.shape[-1] == lz.K and x._off == 0
                and tuple(x._strides) == _contig(x.shape) and _numel(x.shape[:-1]) == lz.M):
            st = lz.panel()
            lz.release()
            x._lazy = _PanelRows(st, lz.M, lz.K)
            return x._lazy
        if (isinstance(lz, _PendingLinear) and lz.epi == F.HB_EPI_GEGLU and lz.takes_panel(lz.epi)
                and lz.n_out % 64 == 0):
            M = lz.x[1]
            st = self._malloc(_panel_rows(M) * lz.n_out * 2)
            self.stats["linear"] += 1
            lz.launch(st.ptr, lz.n_out, F.HB_Y_PANEL)
            lz.release()
            x._lazy = _PanelRows(st, M, lz.n_out)
            return x._lazy
        return None

    def _ptr(self, t: HipTensor) -> int:
        self._ready(t)
        return t._st.ptr + t._off * DT[t.dtype][1]

    def _is_contig(self, t: HipTensor) -> bool:
        exp = _contig(t.shape)
        return all(s == e or d == 1 for s, e, d in zip(t._strides, exp, t.shape))

    def _contiguous(self, t: HipTensor) -> HipTensor:
        """t itself when contiguous, else a contiguous copy (tracked)."""
        self._ready(t)
        if self._is_contig(t):
            return t
        out = self._new(t.shape, t.dtype)
        self._copy_into(t, out._st.ptr, None)
        return out

    def _copy_into(self, t: HipTensor, dst_ptr: int, dst_strides, dst_dtype: Optional[str] = None, op=F.HB_UN_COPY,
                   alpha: float = 0.0):
        self.stats["copies"] += 1
        dd = dst_dtype or t.dtype
        shape = t.shape if t.shape else (1,)
        xs = t._strides if t.shape else (0,)
        ys = F.i64s(dst_strides) if dst_strides is not None else None
        self._call("copy", "hb_unary", self.ctx, op, DT[t.dtype][0], self._ptr(t), F.i64s(xs), DT[dd][0], dst_ptr,
                   ys, F.i64s(shape), len(shape), alpha)

    def _rows(self, t: HipTensor):
        """(storage, ptr, rows, K, ld) for a tensor whose leading dims collapse
        to rows of stride ld with a contiguous last dim; copies otherwise."""
        self._ready(t)
        K = t.shape[-1] if t.shape else 1
        rows = _numel(t.shape[:-1])
        ok = len(t.shape) >= 1 and (t._strides[-1] == 1 or K == 1)
        ld = K
        if ok and len(t.shape) >= 2:
            # leading dims must collapse: stride[i] == stride[i+1] * shape[i+1] (size-1 dims ignored)
            dims = [(d, s) for d, s in zip(t.shape[:-1], t._strides[:-1]) if d != 1]
            if dims:
                ld = dims[-1][1]
                for i in range(len(dims) - 1):
                    if dims[i][1] != dims[i + 1][1] * dims[i + 1][0]:
                        ok = False
                if ld < K:
                    ok = False
        if not ok:
            t = self._contiguous(t)
            ld = K
        return (t._st, self._ptr(t), rows, K, ld)

    @staticmethod
    def _bhld(shape):
        if len(shape) < 2:
            raise ValueError(f"expected [..., L, D], got [{','.join(map(str, shape))}]")
        lead = shape[:-2]
        if len(lead) == 0:
            return 1, 1, shape[-2], shape[-1]
        if len(lead) == 1:
            return 1, lead[0], shape[-2], shape[-1]
        return _numel(lead[:-1]), lead[-1], shape[-2], shape[-1]

    @staticmethod
    def _bhld_strides(shape, strides):
        lead = shape[:-2]
        ls = strides[:-2]
        if len(lead) == 0:
            return (0, 0, strides[-2], strides[-1])
        if len(lead) == 1:
            return (0, ls[0], strides[-2], strides[-1])
        # collapse leading dims into B (must be collapsible)
        dims = [(d, s) for d, s in zip(lead[:-1], ls[:-1]) if d != 1]
        bs = dims[-1][1] if dims else 0
        for i in range(len(dims) - 1):
            if dims[i][1] != dims[i + 1][1] * dims[i + 1][0]:
                return None
        return (bs, ls[-1], strides[-2], strides[-1])

    # ---------------------------------------------------------------- contract: dtype / transfer
    def supports(self, dtype: str) -> bool:
        return dtype in DT

    def fromHost(self, h: HostTensor) -> HipTensor:
        """Copies at call time (index.ts:146-153); f64 / i64 / u64 are widened
        or narrowed to f32 / i32 storage."""
        if self._destroyed:
            raise RuntimeError("hip backend: used after destroy()")
        dtype = h.dtype
        data = np.asarray(h.data)
        if dtype in WIDEN:
            dtype = WIDEN[dtype]
            data = data.astype(NP_DTYPE[dtype])
        if dtype not in DT:
            raise TypeError(f"fromHost: unsupported dtype {h.dtype}")
        if dtype == "bool":
            data = (data != 0).astype(np.uint8)
        data = np.ascontiguousarray(data, dtype=NP_DTYPE[dtype])
        shape = tuple(int(d) for d in h.shape)
        if data.size != _numel(shape):
            raise ValueError(f"fromHost: {data.size} values for shape [{','.join(map(str, shape))}]")
        t = self._new(shape, dtype)
        if data.nbytes:
            self._call("fromHost", "hb_upload", self.ctx, t._st.ptr, data.ctypes.data, data.nbytes)
        return t

    def read(self, t: HipTensor) -> HostTensor:
        self._live(t, op="read")
        c = self._contiguous(t)
        out = np.empty(t.shape, NP_DTYPE[t.dtype])
        if out.nbytes:
            self._call("read", "hb_download", self.ctx, out.ctypes.data, self._ptr(c), out.nbytes)
        else:
            self._call("read", "hb_sync", self.ctx)
        if c is not t:
            self.dispose(c)
        return HostTensor(t.dtype, t.shape, out)

    def dispose(self, t: HipTensor) -> None:
        """Frees now; idempotent (index.ts:156-157)."""
        if t is None or t._dead:
            return
        t._dead = True
        if t._lazy is not None:
            t._lazy.release()
            t._lazy = None
        if t._st is not None:
            t._st.release()
            t._st = None
        for k, v in list((t._meta or {}).items()):
            if isinstance(v, HipTensor):
                self.dispose(v)
        t._meta = None

    def scope(self, fn: Callable[[], Any]):
        """index.ts:158-162: tensors created inside `fn` and not returned
        (directly or one level deep in a list / tuple / dict / object) are
        disposed afterwards."""
        self._scopes.append([])
        try:
            result = fn()
        except BaseException:
            created = self._scopes.pop()
            for t in created:
                self.dispose(t)
            raise
        created = self._scopes.pop()
        keep = set()

        def mark(v):
            if isinstance(v, HipTensor):
                keep.add(id(v))

        mark(result)
        if isinstance(result, (list, tuple)):
            for v in result:
                mark(v)
        elif isinstance(result, dict):
            for v in result.values():
                mark(v)
        elif result is not None and hasattr(result, "__dict__"):
            for v in vars(result).values():
                mark(v)
        for t in created:
            if id(t) in keep:
                if self._scopes:
                    self._scopes[-1].append(t)
            else:
                self.dispose(t)
        return result

    def flush(self, *ts: HipTensor, wait: bool = True) -> None:
        """Forces pending lazy work of `ts` to execute (index.ts:163-164):
        their launches are enqueued now; with `wait` (the default) the call
        also waits for the stream."""
        for t in ts:
            self._live(t, op="flush")
            self._ready(t)
        if wait:
            self._call("flush", "hb_sync", self.ctx)

    def destroy(self) -> None:
        if not self._destroyed:
            for release in self._compiled:
                release()
            self._compiled = []
            self._blocks.clear()  # the library frees every block with the context
            self._call("destroy", "hb_destroy", self.ctx)
            self._destroyed = True

    def capture(self, fn: Callable[[], Any], warmup: bool = True) -> "HipGraph":
        """Records the launches of `fn()` (an op sequence on this backend)
        into a HIP graph; HipGraph.run() replays them and returns the same
        output tensor, rewritten.  No counterpart in the reference's
        Backend: for small batches, where the host's per-op launches bound
        the time.  The graph keeps using the device addresses it recorded:
        the tensors `fn` reads must stay alive (rewrite inputs in place
        between replays with `write`), and blocks disposed while recording
        stay out of the pool until HipGraph.destroy().  Device summaries of
        the inputs (mask tile classes) are recomputed by every replay.
        `warmup` runs `fn` once eagerly first, so one-time set-up that
        allocates or uploads (RoPE tables, summary buffers) happens outside
        the recording.  `fn` returns a tensor or a list / tuple of tensors."""
        if self._capture_held is not None:
            raise RuntimeError("capture: already recording")
        if warmup:
            done = set()
            for t in _flat_outputs(fn(), "capture"):
                if id(t) not in done:
                    done.add(id(t))
                    self.dispose(self._ready(t))
        self.flush()
        held: list = []
        self._capture_held = held
        self._capture_summaries = set()
        self._call("capture", "hb_capture_begin", self.ctx)
        e = F.U(0)
        try:
            out = fn()
            for t in _flat_outputs(out, "capture"):
                self._ready(t)  # the result's pending launches belong to the recording
        except BaseException:
            self._capture_held = None
            self._capture_summaries = None
            try:
                self._call("capture", "hb_capture_end", self.ctx, F.C.byref(e))
                self._call("capture", "hb_graph_destroy", self.ctx, e.value)
            except Exception:
                pass
            for ptr, nbytes in held:
                self._recycle(ptr, nbytes)
            raise
        self._capture_held = None
        self._capture_summaries = None
        try:
            self._call("capture", "hb_capture_end", self.ctx, F.C.byref(e))
        except BaseException:
            for ptr, nbytes in held:
                self._recycle(ptr, nbytes)
            raise
        return HipGraph(self, e.value, out, held)

    def compile(self, fn: Callable) -> Callable:
        """Backend.compile (tensor-backend/src/index.ts:245): wraps `fn`, a
        pure function of tensors returning a tensor or a list / tuple of
        tensors, for replay.  The first call with a given input signature
        (shapes and dtypes) copies its inputs into blocks of their own and
        records `fn` on those (HipBackend.capture); every call copies its
        inputs into its signature's blocks, replays that recording and
        returns fresh copies of the outputs in `fn`'s structure, which the
        caller owns.  A replay re-derives the device summaries of its inputs
        (attention-mask tile classes).  The recordings and their blocks live
        until the wrapper's `release()` or the backend's destroy()."""
        recs: dict = {}

        def run(*args):
            if self._capture_held is not None:
                raise RuntimeError("compile: called while a graph records")
            self._live(*args, op="compile")
            key = tuple((tuple(t.shape), t.dtype) for t in args)
            rec = recs.get(key)
            if rec is None:
                # input blocks of the recording: untracked, owned by the wrapper
                ins = [HipTensor(tuple(t.shape), t.dtype, self._malloc(max(1, _numel(t.shape)) * DT[t.dtype][1]))
                       for t in args]
                for src, dst in zip(args, ins):
                    if src.size:
                        self._copy_into(src, dst._st.ptr, None)
                g = self.capture(lambda: fn(*ins))
                rec = recs[key] = (ins, g)
            else:
                ins, g = rec
                for src, dst in zip(args, ins):
                    if src.size:
                        self._copy_into(src, dst._st.ptr, None)
                    for ent in (dst._st.cache or {}).values():
                        ent[1] = False  # summaries of the old contents
            out = g.run()
            copies = []
            for t in _flat_outputs(out, "compile"):
                c = self._new(t.shape, t.dtype)
                if t.size:
                    self._copy_into(t, c._st.ptr, None)
                copies.append(c)
            if isinstance(out, HipTensor):
                return copies[0]
            return type(out)(copies)

        def release() -> None:
            for ins, g in recs.values():
                outs = _flat_outputs(g.out, "compile")
                g.destroy()
                for t in ins + outs:
                    self.dispose(t)
            recs.clear()

        run.release = release
        self._compiled.append(release)
        return run

    def pool_stats(self) -> dict:
        self._return_blocks()  # blocks waiting for reuse count as cached, not live
        a, b, c = F.U(0), F.U(0), F.U(0)
        self._call("poolStats", "hb_pool_stats", self.ctx, F.C.byref(a), F.C.byref(b), F.C.byref(c))
        return {"live_bytes": a.value, "cached_bytes": b.value, "live_blocks": c.value}

    # ---------------------------------------------------------------- shape
    def _shared_linear(self, x: HipTensor) -> Optional[_SharedLinear]:
        """x's pending plain product as a _SharedLinear that views may share
        (x itself becomes the first view), or None."""
        lz = x._lazy
        if isinstance(lz, _PendingLinear) and lz.epi == 0 and x._off == 0 and len(x.shape) >= 1:
            x._lazy = _SharedLinear(self, lz, _numel(x.shape[:-1]), lz.n_out, x.dtype)
            x._strides = _contig(x.shape)
        return x._lazy if isinstance(x._lazy, _SharedLinear) else None

    def reshape(self, x: HipTensor, shape) -> HipTensor:
        self._live(x, op="reshape")
        shape = [int(d) for d in shape]
        n = x.size
        if shape.count(-1) > 1:
            raise ValueError("reshape: more than one -1")
        if -1 in shape:
            known = _numel([d for d in shape if d != -1])
            shape[shape.index(-1)] = n // known if known else 0
        if _numel(shape) != n:
            raise ValueError(f"reshape: cannot reshape [{','.join(map(str, x.shape))}] to [{','.join(map(str, shape))}]")
        if isinstance(x._lazy, _PendingSdpa) or self._shared_linear(x) is not None:
            # a view of the pending output, not launched yet
            st = self._nocopy_strides(x.shape, x._strides, shape)
            if st is not None:
                return self._track(HipTensor(shape, x.dtype, None, x._off, st, lazy=x._lazy.share()))
        self._ready(x)
        st = self._nocopy_strides(x.shape, x._strides, shape)
        if st is None:
            c = self._contiguous(x)
            return self._view(c, shape, _contig(shape), c._off)
        return self._view(x, shape, st, x._off)

    @staticmethod
    def _nocopy_strides(old_shape, old_strides, new_shape):
        """Strides for viewing (old_shape, old_strides) as new_shape without a
        copy, or None (the classic chunk-matching rule)."""
        if _numel(old_shape) == 0:
            return _contig(new_shape)
        od = [(d, s) for d, s in zip(old_shape, old_strides) if d != 1]
        nd = list(new_shape)
        out = [0] * len(nd)
        oi = 0
        ni = 0
        while ni < len(nd):
            if nd[ni] == 1:
                out[ni] = 1
                ni += 1
                continue
            if oi >= len(od):
                return None
            # gather a chunk of old dims that are contiguous with each other
            size_o = od[oi][0]
            chunk_end = oi
            size_n = nd[ni]
            nstart = ni
            while size_o != size_n:
                if size_o < size_n:
                    chunk_end += 1
                    if chunk_end >= len(od):
                        return None
                    if od[chunk_end - 1][1] != od[chunk_end][1] * od[chunk_end][0]:
                        return None
                    size_o *= od[chunk_end][0]
                else:
                    ni += 1
                    while ni < len(nd) and nd[ni] == 1:
                        out[ni] = 1
                        ni += 1
                    if ni >= len(nd):
                        return None
                    size_n *= nd[ni]
            # assign strides for new dims nstart..ni from the innermost old stride
            stride = od[chunk_end][1]
            for j in range(ni, nstart - 1, -1):
                if nd[j] == 1:
                    out[j] = stride
                    continue
                out[j] = stride
                stride *= nd[j]
            oi = chunk_end + 1
            ni += 1
        if oi != len(od):
            return None
        return tuple(out)

    def transpose(self, x: HipTensor, perm) -> HipTensor:
        self._live(x, op="transpose")
        perm = [int(p) % len(x.shape) if len(x.shape) else 0 for p in perm]
        if sorted(perm) != list(range(len(x.shape))):
            raise ValueError(f"transpose: bad perm {perm} for rank {len(x.shape)}")
        if isinstance(x._lazy, _PendingSdpa) or self._shared_linear(x) is not None:
            # a view of the pending output, not launched yet
            return self._track(HipTensor([x.shape[p] for p in perm], x.dtype, None, x._off,
                                         [x._strides[p] for p in perm], lazy=x._lazy.share()))
        self._ready(x)
        return self._view(x, [x.shape[p] for p in perm], [x._strides[p] for p in perm], x._off)

    def slice(self, x: HipTensor, begin, end) -> HipTensor:
        self._live(x, op="slice")
        lazy_view = self._shared_linear(x) is not None  # a view of a pending product stays pending
        if not lazy_view:
            self._ready(x)
        r = len(x.shape)
        if len(begin) > r or len(end) > r:
            raise ValueError("slice: more bounds than axes")
        off = x._off
        shape = list(x.shape)
        for i in range(r):
            n = x.shape[i]
            b = int(begin[i]) if i < len(begin) else 0
            e = int(end[i]) if i < len(end) else n
            if b < 0:
                b += n
            if e < 0:
                e += n
            b = min(max(b, 0), n)
            e = min(max(e, b), n)
            off += b * x._strides[i]
            shape[i] = e - b
        if lazy_view:
            return self._track(HipTensor(shape, x.dtype, None, off, x._strides, lazy=x._lazy.share()))
        return self._view(x, shape, x._strides, off)

    def split(self, x: HipTensor, parts: int, axis: int) -> list:
        self._live(x, op="split")
        r = len(x.shape)
        a = axis % r
        n = x.shape[a]
        if n % parts:
            raise ValueError(f"split: axis {axis} of size {n} is not divisible into {parts}")
        step = n // parts
        out = []
        for p in range(parts):
            b = [0] * r
            e = list(x.shape)
            b[a] = p * step
            e[a] = (p + 1) * step
            out.append(self.slice(x, b, e))
        return out

    def concat(self, xs: Sequence[HipTensor], axis: int) -> HipTensor:
        self._live(*xs, op="concat")
        r = len(xs[0].shape)
        a = axis % r
        dtype = xs[0].dtype
        for t in xs[1:]:
            dtype = _promote(dtype, t.dtype)
        shape = list(xs[0].shape)
        shape[a] = sum(t.shape[a] for t in xs)
        out = self._new(shape, dtype)
        ost = _contig(shape)
        pos = 0
        es = DT[dtype][1]
        for t in xs:
            if t.size:
                self._copy_into(t, out._st.ptr + pos * ost[a] * es, ost, dtype)
            pos += t.shape[a]
        return out

    def cast(self, x: HipTensor, dtype: str) -> HipTensor:
        self._live(x, op="cast")
        dtype = WIDEN.get(dtype, dtype)
        if dtype not in DT:
            raise TypeError(f"cast: unsupported dtype {dtype}")
        out = self._new(x.shape, dtype)
        if x.size:
            self._copy_into(x, out._st.ptr, None, dtype)
        return out

    # ---------------------------------------------------------------- elementwise
    def _bstrides(self, t: HipTensor, shape) -> tuple:
        r = len(shape)
        pad = r - len(t.shape)
        st = []
        for i in range(r):
            j = i - pad
            if j < 0 or t.shape[j] == 1:
                st.append(0)
            else:
                st.append(t._strides[j])
        return tuple(st)

    def _binary(self, op: int, a: HipTensor, b: HipTensor, name: str, out_dtype: Optional[str] = None):
        self._live(a, b, op=name)
        self._ready(a)
        self._ready(b)
        shape = _broadcast_shape(a.shape, b.shape)
        if out_dtype is None:
            out_dtype = _promote(a.dtype, b.dtype)
        out = self._new(shape, out_dtype)
        if out.size:
            sh = shape if shape else (1,)
            self._call(name, "hb_binary", self.ctx, op, DT[a.dtype][0], self._ptr(a),
                       F.i64s(self._bstrides(a, sh) if shape else (0,)), DT[b.dtype][0], self._ptr(b),
                       F.i64s(self._bstrides(b, sh) if shape else (0,)), DT[out_dtype][0], out._st.ptr, F.i64s(sh),
                       len(sh))
        return out

    def add(self, a: HipTensor, b: HipTensor) -> HipTensor:
        self._live(a, b, op="add")
        fused = self._try_fuse_resid(a, b) or self._try_fuse_resid(b, a)
        if fused is not None:
            return fused
        return self._binary(F.HB_BIN_ADD, a, b, "add")

    def _try_fuse_resid(self, r: HipTensor, lin: HipTensor) -> Optional[HipTensor]:
        lz = lin._lazy
        if not isinstance(lz, _PendingLinear) or lz.epi:
            return None
        if r._lazy is not None and not isinstance(r._lazy, (_PanelRows, _PendingNorm)):
            return None
        if r.shape != lin.shape or r.dtype != lin.dtype:
            return None
        rows = self._rows(r)
        out = self._new(lin.shape, lin.dtype)
        self.stats["linear_fused_resid"] += 1
        lz.launch(out._st.ptr, lz.N, 0, (rows[1], rows[4]))
        return out

    def sub(self, a, b):
        return self._binary(F.HB_BIN_SUB, a, b, "sub")

    def mul(self, a, b):
        return self._binary(F.HB_BIN_MUL, a, b, "mul")

    def div(self, a, b):
        dt = _promote(a.dtype, b.dtype)
        return self._binary(F.HB_BIN_DIV, a, b, "div", dt if dt in FLOAT_DT else "f32")

    def maximum(self, a, b):
        return self._binary(F.HB_BIN_MAX, a, b, "maximum")

    def where(self, cond: HipTensor, a: HipTensor, b: HipTensor) -> HipTensor:
        self._live(cond, a, b, op="where")
        for t in (cond, a, b):
            self._ready(t)
        c = cond if cond.dtype == "bool" else self.cast(cond, "bool")
        shape = _broadcast_shape(c.shape, a.shape, b.shape)
        dt = _promote(a.dtype, b.dtype)
        out = self._new(shape, dt)
        if out.size:
            sh = shape if shape else (1,)
            bs = (lambda t: F.i64s(self._bstrides(t, sh) if shape else (0,)))
            self._call("where", "hb_where", self.ctx, self._ptr(c), bs(c), DT[a.dtype][0], self._ptr(a), bs(a),
                       DT[b.dtype][0], self._ptr(b), bs(b), DT[dt][0], out._st.ptr, F.i64s(sh), len(sh))
        if c is not cond:
            self.dispose(c)
        return out

    def _unary(self, op: int, x: HipTensor, name: str, out_dtype: Optional[str] = None, alpha: float = 0.0):
        self._live(x, op=name)
        self._ready(x)
        if out_dtype is None:
            out_dtype = x.dtype if x.dtype in FLOAT_DT else "f32"
        out = self._new(x.shape, out_dtype)
        if out.size:
            self._copy_into(x, out._st.ptr, None, out_dtype, op, alpha)
        return out

    def scale(self, x, s: float):
        return self._unary(F.HB_UN_SCALE, x, "scale", alpha=float(s))

    def exp(self, x):
        return self._unary(F.HB_UN_EXP, x, "exp")

    def log(self, x):
        return self._unary(F.HB_UN_LOG, x, "log")

    def relu(self, x):
        return self._unary(F.HB_UN_RELU, x, "relu", x.dtype)

    def gelu(self, x):
        return self._unary(F.HB_UN_GELU, x, "gelu")

    # optional general numerics (index.ts:265-316)
    def equal(self, a, b):
        return self._binary(F.HB_BIN_EQ, a, b, "equal", "bool")

    def notEqual(self, a, b):
        return self._binary(F.HB_BIN_NE, a, b, "notEqual", "bool")

    def less(self, a, b):
        return self._binary(F.HB_BIN_LT, a, b, "less", "bool")

    def lessEqual(self, a, b):
        return self._binary(F.HB_BIN_LE, a, b, "lessEqual", "bool")

    def greater(self, a, b):
        return self._binary(F.HB_BIN_GT, a, b, "greater", "bool")

    def greaterEqual(self, a, b):
        return self._binary(F.HB_BIN_GE, a, b, "greaterEqual", "bool")

    def logicalAnd(self, a, b):
        return self._binary(F.HB_BIN_AND, a, b, "logicalAnd", "bool")

    def logicalOr(self, a, b):
        return self._binary(F.HB_BIN_OR, a, b, "logicalOr", "bool")

    def logicalNot(self, x):
        return self._unary(F.HB_UN_NOT, x, "logicalNot", "bool")

    def sqrt(self, x):
        return self._unary(F.HB_UN_SQRT, x, "sqrt")

    def rsqrt(self, x):
        return self._unary(F.HB_UN_RSQRT, x, "rsqrt")

    def pow(self, a, b):
        dt = _promote(a.dtype, b.dtype)
        return self._binary(F.HB_BIN_POW, a, b, "pow", dt if dt in FLOAT_DT else "f32")

    def neg(self, x):
        return self._unary(F.HB_UN_NEG, x, "neg", "i32" if x.dtype == "bool" else x.dtype)

    def abs(self, x):
        return self._unary(F.HB_UN_ABS, x, "abs", "i32" if x.dtype == "bool" else x.dtype)

    def tanh(self, x):
        return self._unary(F.HB_UN_TANH, x, "tanh")

    def sigmoid(self, x):
        return self._unary(F.HB_UN_SIGMOID, x, "sigmoid")

    def erf(self, x):
        return self._unary(F.HB_UN_ERF, x, "erf")

    # ---------------------------------------------------------------- reductions
    def _axis(self, x, axis):
        r = len(x.shape)
        a = axis + r if axis < 0 else axis
        if a < 0 or a >= r:
            raise ValueError(f"axis {axis} out of range for rank {r}")
        return a

    def _reduce(self, op, x, axis, keepDims, name, out_dtype):
        self._live(x, op=name)
        a = self._axis(x, axis)
        c = self._contiguous(x)
        outer = _numel(x.shape[:a])
        n = x.shape[a]
        inner = _numel(x.shape[a + 1:])
        shape = list(x.shape)
        if keepDims:
            shape[a] = 1
        else:
            shape.pop(a)
        out = self._new(shape, out_dtype)
        if outer * inner:
            self._call(name, "hb_reduce", self.ctx, op, DT[x.dtype][0], self._ptr(c), outer, n, inner,
                       DT[out_dtype][0], out._st.ptr)
        if c is not x:
            self.dispose(c)
        return out

    def sum(self, x, axis: int, keepDims: bool = False):
        dt = x.dtype if x.dtype != "bool" else "i32"
        return self._reduce(F.HB_RED_SUM, x, axis, keepDims, "sum", dt)

    def max(self, x, axis: int, keepDims: bool = False):
        return self._reduce(F.HB_RED_MAX, x, axis, keepDims, "max", x.dtype)

    def min(self, x, axis: int, keepDims: bool = False):
        return self._reduce(F.HB_RED_MIN, x, axis, keepDims, "min", x.dtype)

    def mean(self, x, axis: int, keepDims: bool = False):
        return self._reduce(F.HB_RED_MEAN, x, axis, keepDims, "mean", x.dtype if x.dtype in FLOAT_DT else "f32")

    def argmax(self, x, axis: int, keepDims: bool = False):
        return self._reduce(F.HB_RED_ARGMAX, x, axis, keepDims, "argmax", "i32")

    def argmin(self, x, axis: int, keepDims: bool = False):
        return self._reduce(F.HB_RED_ARGMIN, x, axis, keepDims, "argmin", "i32")

    def _scan(self, op, x, axis, name, out_dtype):
        self._live(x, op=name)
        a = self._axis(x, axis)
        c = self._contiguous(x)
        out = self._new(x.shape, out_dtype)
        outer, n, inner = _numel(x.shape[:a]), x.shape[a], _numel(x.shape[a + 1:])
        if out.size:
            self._call(name, "hb_scan", self.ctx, op, DT[x.dtype][0], self._ptr(c), outer, n, inner,
                       DT[out_dtype][0], out._st.ptr)
        if c is not x:
            self.dispose(c)
        return out

    def softmax(self, x, axis: int):
        return self._scan(F.HB_SCAN_SOFTMAX, x, axis, "softmax", x.dtype if x.dtype in FLOAT_DT else "f32")

    def sort(self, x, axis: int):
        return self._scan(F.HB_SCAN_SORT, x, axis, "sort", x.dtype)

    def cumsum(self, x, axis: int):
        return self._scan(F.HB_SCAN_CUMSUM, x, axis, "cumsum", "i32" if x.dtype == "bool" else x.dtype)

    # ---------------------------------------------------------------- linear algebra & NN
    def matmul(self, a: HipTensor, b: HipTensor) -> HipTensor:
        """[..., m, k] @ [..., k, n] with broadcast leading dims, as one
        linear per batch entry over b^T (f32 accumulation)."""
        self._live(a, b, op="matmul")
        if len(a.shape) < 2 or len(b.shape) < 2 or a.shape[-1] != b.shape[-2]:
            raise ValueError(f"matmul: [{a.shape}] @ [{b.shape}]")
        dt = _promote(a.dtype, b.dtype)
        lead = _broadcast_shape(a.shape[:-2], b.shape[:-2])
        m, k, n = a.shape[-2], a.shape[-1], b.shape[-1]
        out = self._new(tuple(lead) + (m, n), dt)
        A = self._contiguous(a if a.dtype == dt else self.cast(a, dt))
        Bt = self.transpose(b if b.dtype == dt else self.cast(b, dt), list(range(len(b.shape) - 2)) +
                            [len(b.shape) - 1, len(b.shape) - 2])
        Bt = self._contiguous(Bt)
        As = self._bstrides(A, tuple(lead) + (m, k))
        Bs = self._bstrides(Bt, tuple(lead) + (n, k))
        es = DT[dt][1]
        for idx in np.ndindex(*lead) if lead else [()]:
            ao = A._off + sum(i * s for i, s in zip(idx, As[:-2]))
            bo = Bt._off + sum(i * s for i, s in zip(idx, Bs[:-2]))
            oo = sum(i * s for i, s in zip(idx, _contig(tuple(lead) + (m, n))[:-2]))
            if A._strides[-1] != 1:
                raise ValueError("matmul: internal layout")
            self._ready(A)
            self._call("matmul", "hb_linear", self.ctx, DT[dt][0], A._st.ptr + ao * es, A._strides[-2] if m > 1 else k,
                       Bt._st.ptr + bo * es, 0, 0, 0, out._st.ptr + oo * es, n, m, n, k, 0)
        return out

    def linear(self, x: HipTensor, w: HipTensor, b: Optional[HipTensor] = None) -> HipTensor:
        """y = x . w^T (+ b), w [out, in], f32 accumulation (index.ts:211-215).
        Returns a pending tensor; see the module docstring."""
        self._live(x, w, b, op="linear")
        if len(w.shape) != 2 or not x.shape or x.shape[-1] != w.shape[1]:
            raise ValueError(f"linear: x [{','.join(map(str, x.shape))}] vs w [{','.join(map(str, w.shape))}]")
        dt = x.dtype if x.dtype in FLOAT_DT else "f32"
        if x.dtype != dt:
            x = self.cast(x, dt)
        if w.dtype != dt:
            w = self.cast(w, dt)
        w = self._contiguous(w)
        if b is not None:
            if b.shape != (w.shape[0],):
                raise ValueError(f"linear: bias [{','.join(map(str, b.shape))}] vs out {w.shape[0]}")
            b = self._contiguous(b if b.dtype == dt else self.cast(b, dt))
        pend = _PendingLinear(self, x, w, b, panel=self._panel_for(x, w=w))
        return self._track(HipTensor(x.shape[:-1] + (w.shape[0],), dt, None, lazy=pend))

    def _panel_for(self, x: HipTensor, w: Optional[HipTensor] = None, q=None) -> Optional[_PanelRows]:
        """The panel-order form of x when this linear layer takes a kernel
        that reads it: the large-M one, or for 16-bit weights the small-M slab
        kernel as the launch without an epilogue takes it (weights side
        checked here, x side by _as_panel; a launch that ends up taking
        another kernel unpacks x)."""
        if x.dtype not in ("f16", "bf16") or not x.shape:
            return None
        M = _numel(x.shape[:-1])
        if M < PANEL_MIN_M and (q is not None or w is None
                                or not _slab_path(M, w.shape[0], x.shape[-1], False, self.cus)):
            return None
        if x._lazy is None or isinstance(x._lazy, _PendingRope):
            return None
        if q is None:
            if self._ptr(w) % 16:
                return None
        else:
            qw, scales, zeros, group = q
            if (self._ptr(qw) % 8 or self._ptr(scales) % 2 or (zeros is not None and self._ptr(zeros) % 2)
                    or group % 8):
                return None
        return self._as_panel(x)

    def layerNorm(self, x: HipTensor, weight: Optional[HipTensor], bias: Optional[HipTensor], eps: float):
        self._live(x, weight, bias, op="layerNorm")
        dt = x.dtype if x.dtype in FLOAT_DT else "f32"
        st, xp, rows, D, ld = self._rows(x)
        wdt = None
        wp = bp = 0
        if weight is not None:
            weight = self._contiguous(weight)
            wp, wdt = self._ptr(weight), weight.dtype
        if bias is not None:
            bias = self._contiguous(bias)
            if wdt is not None and bias.dtype != wdt:
                bias = self.cast(bias, wdt)
            bp, wdt = self._ptr(bias), bias.dtype
        pend = _PendingNorm(self, x, weight, bias, eps, dt)
        return self._track(HipTensor(x.shape, dt, None, lazy=pend))

    def embedding(self, table: HipTensor, ids: HipTensor) -> HipTensor:
        self._live(table, ids, op="embedding")
        V, D = table.shape
        t = self._contiguous(table)
        i = self._contiguous(ids if ids.dtype == "i32" else self.cast(ids, "i32"))
        out = self._new(ids.shape + (D,), table.dtype)
        if out.size:
            self._call("embedding", "hb_gather", self.ctx, DT[table.dtype][0], self._ptr(t), V, D, self._ptr(i),
                       ids.size, 0, DT[table.dtype][0], out._st.ptr)
        return out

    def gatherRows(self, x: HipTensor, idx: HipTensor) -> HipTensor:
        self._live(x, idx, op="gatherRows")
        B, L, D = x.shape
        M = idx.shape[1]
        t = self._contiguous(x)
        i = self._contiguous(idx if idx.dtype == "i32" else self.cast(idx, "i32"))
        out = self._new((B, M, D), x.dtype)
        if out.size:
            self._call("gatherRows", "hb_gather", self.ctx, DT[x.dtype][0], self._ptr(t), L, D, self._ptr(i), B * M,
                       M, DT[x.dtype][0], out._st.ptr)
        return out

    def rope(self, x: HipTensor, base: float) -> HipTensor:
        """Split-half RoPE on [B, H, L, Dh] (index.ts:225-229); pending so
        that sdpa can apply it while staging Q / K."""
        self._live(x, op="rope")
        if x.shape[-1] % 2:
            raise ValueError("rope: head dim must be even")
        if not isinstance(x._lazy, _SharedLinear):  # a view of a pending product stays pending
            self._ready(x)
        dt = x.dtype if x.dtype in FLOAT_DT else "f32"
        if self._bhld_strides(x.shape, x._strides) is None:
            x = self._contiguous(x)
        pend = _PendingRope(self, x, base)
        return self._track(HipTensor(x.shape, dt, None, lazy=pend))

    def _attn_operand(self, t: HipTensor):
        """(ptr, strides[4], rope_base, storage) of a [B, H, L, D] sdpa operand."""
        lz = t._lazy
        if isinstance(lz, _PendingRope) and lz.src[3] == t.dtype:
            st, off, strides, dtype, shape = lz.source()
            return st.ptr + off * DT[dtype][1], self._bhld_strides(shape, strides), lz.base, st
        self._ready(t)
        s = self._bhld_strides(t.shape, t._strides)
        if s is None:
            t = self._contiguous(t)
            s = self._bhld_strides(t.shape, t._strides)
        return self._ptr(t), s, 0.0, t._st

    def _qkv_fused(self, q: HipTensor, k: HipTensor, v: HipTensor):
        """sdpa operands from one hb_linear_qkv launch, when q and k are
        roped views and v a view of the same pending [B*L, 3*H*64] projection,
        taken as modernbert/src/index.ts:348-351 takes them (reshape to
        [B, L, 3, H, 64], transpose to [3, B, H, L, 64], split); else None."""
        lq, lk, S = q._lazy, k._lazy, v._lazy
        if not (self.fuse_qkv and isinstance(lq, _PendingRope) and isinstance(lk, _PendingRope) and isinstance(S, _SharedLinear)):
            return None
        if lq.lin is not S or lk.lin is not S or lq.base != lk.base or lq.base <= 0 or not S.qkv_ok():
            return None
        B, H, L, D = q.shape
        if D != 64 or tuple(k.shape) != tuple(q.shape) or tuple(v.shape) != tuple(q.shape) or B * L != S.M \
                or S.N != 3 * H * 64 or not (q.dtype == k.dtype == v.dtype == S.dtype):
            return None
        rows = (L * S.N, 64, S.N, 1)  # [B, H, L, 64] over the [B*L, 3*H*64] product
        for (_, off, strides, dtype, shape), want in ((lq.src, 0), (lk.src, H * 64)):
            if off != want or tuple(strides) != rows or tuple(shape) != tuple(q.shape) or dtype != S.dtype:
                return None
        if v._off != 2 * H * 64 or tuple(v._strides) != rows:
            return None
        st = S.fused(lq.base, L, H)
        part = B * H * L * 64 * DT[S.dtype][1]
        hs = (H * L * 64, L * 64, 64, 1)
        return [(st.ptr + i * part, hs, 0.0, st) for i in range(3)]

    def sdpa(self, q: HipTensor, k: HipTensor, v: HipTensor, mask: Optional[HipTensor], scale: float) -> HipTensor:
        self._live(q, k, v, mask, op="sdpa")
        if len(q.shape) != 4:
            raise ValueError("sdpa: q must be [B, H, L, D]")
        B, H, Lq, D = q.shape
        Lk = k.shape[2]
        if k.shape[0] != B or k.shape[1] != H or v.shape[2] != Lk or k.shape[3] != D or v.shape[3] != D:
            raise ValueError(f"sdpa: q [{q.shape}] k [{k.shape}] v [{v.shape}]")
        dt = _promote(_promote(q.dtype, k.dtype), v.dtype)
        if dt not in FLOAT_DT:
            dt = "f32"
        ops = self._qkv_fused(q, k, v)
        if ops is None:
            ops = []
            for t in (q, k, v):
                if t.dtype != dt:
                    t = self.cast(t, dt)
                ops.append(self._attn_operand(t))
        (qp, qs, rq, qst), (kp, ks, rk, kst), (vp, vs, _, vst) = ops
        refs = [qst.retain(), kst.retain(), vst.retain()]
        mp, ms = 0, None
        mc = None
        if mask is not None:
            self._ready(mask)
            mc = mask if mask.dtype == "bool" else self.cast(mask, "bool")
            if len(mc.shape) > 4:
                for r in refs:
                    r.release()
                raise ValueError("sdpa: mask rank > 4")
            full = (B, H, Lq, Lk)
            _broadcast_shape(mc.shape, full)
            ms = self._bstrides(mc, full)
            mp = self._ptr(mc)
            refs.append(mc._st.retain())
        info = self._mask_info(mc, ms, B, Lq, Lk) if mc is not None else 0
        # hb_sdpa_panel's conditions (its MFMA path), for a consumer that reads panel order
        panel_ok = (dt in ("f16", "bf16") and D == 64 and Lk > 0 and (H * D) % 64 == 0
                    and all(p % 16 == 0 for p in (qp, kp, vp)) and all(st_[3] == 1 for st_ in (qs, ks, vs))
                    and all(st_[i] % 8 == 0 for st_ in (qs, ks, vs) for i in range(3))
                    and (ms is None or ms[1] == 0) and (Lk + 63) // 64 <= 1024
                    and 0 <= ks[2] < 1 << 24 and 0 <= vs[2] < 1 << 24)
        args = (DT[dt][0], qp, qs, kp, ks, vp, vs, mp, ms, info, B, H, Lq, Lk, D, float(scale), rq, rk)
        pend = _PendingSdpa(self, args, refs, panel_ok)
        if mc is not None and mc is not mask:
            self.dispose(mc)  # its storage is held by the pending launch
        # output physically [B, Lq, H, D], returned as a [B, H, Lq, D] view
        return self._track(HipTensor((B, H, Lq, D), dt, None, 0, (Lq * H * D, D, H * D, 1), lazy=pend))

    def _mask_info(self, mc: HipTensor, ms, B: int, Lq: int, Lk: int) -> int:
        """Device summary of a bool mask (per-tile: no / all / some keys
        visible), cached on the mask's storage so the 14 sliding-window
        layers of an encode share one pass over the mask.  It is rebuilt when
        stale (the mask was rewritten in place by `write`) and, while a graph
        records, enqueued once into the recording, so every replay
        summarises the mask as it is at that replay."""
        if ms[1] != 0 or not (B and Lq and Lk):
            return 0
        key = ("sdpa_tiles", mc._off, tuple(ms), B, Lq, Lk)
        if mc._st.cache is None:
            mc._st.cache = {}
        cache = mc._st.cache
        ent = cache.get(key)
        if ent is None:
            n = F.C.c_size_t(0)
            self._call("sdpa", "hb_sdpa_mask_info_bytes", B, Lq, Lk, F.C.byref(n))
            p = F.U(0)
            self._call("sdpa", "hb_alloc", self.ctx, max(1, n.value), F.C.byref(p))
            ent = cache[key] = [p.value, False]
        rec = self._capture_summaries
        if rec is not None:
            # Recorded, not run: only a replay writes this summary, so the
            # entry's freshness is left as it was (an entry first built
            # inside a recording stays stale and an eager call after the
            # recording, or after an aborted one, rebuilds it).
            if (id(mc._st), key) not in rec:
                self._call("sdpa", "hb_sdpa_mask_info", self.ctx, self._ptr(mc), F.i64s(ms), B, Lq, Lk, ent[0])
                rec.add((id(mc._st), key))
        elif not ent[1]:
            self._call("sdpa", "hb_sdpa_mask_info", self.ctx, self._ptr(mc), F.i64s(ms), B, Lq, Lk, ent[0])
            ent[1] = True
        return ent[0]

    def write(self, t: HipTensor, h: HostTensor) -> None:
        """Overwrites a contiguous tensor's values in place with host data of
        the same dtype and shape (copied at call time).  No counterpart in the
        reference's Backend, whose tensors are immutable: it rewrites the
        inputs of a recorded graph between replays (HipBackend.capture).
        Device summaries derived from the old contents (attention-mask tile
        classes) are marked stale and rebuilt on their next use."""
        self._live(t, op="write")
        if self._capture_held is not None:
            raise RuntimeError("write: a graph is recording (rewrite inputs between replays)")
        if t._lazy is not None or not self._is_contig(t):
            raise ValueError("write: the tensor must be a materialised, contiguous tensor")
        dtype = WIDEN.get(h.dtype, h.dtype)
        if dtype != t.dtype or tuple(int(d) for d in h.shape) != t.shape:
            raise ValueError(f"write: {h.dtype}[{','.join(map(str, h.shape))}] into "
                             f"{t.dtype}[{','.join(map(str, t.shape))}]")
        data = np.asarray(h.data)
        if dtype == "bool":
            data = (data != 0).astype(np.uint8)
        data = np.ascontiguousarray(data, dtype=NP_DTYPE[dtype])
        if data.nbytes:
            self._call("write", "hb_upload", self.ctx, self._ptr(t), data.ctypes.data, data.nbytes)
        for ent in (t._st.cache or {}).values():
            ent[1] = False

    # ---------------------------------------------------------------- optional fused ops
    def geglu(self, x: HipTensor) -> HipTensor:
        """gelu(value) * gate (index.ts:240-241); absorbed into a pending
        linear's epilogue when x is one."""
        self._live(x, op="geglu")
        F2 = x.shape[-1]
        if F2 % 2:
            raise ValueError("geglu: last axis must be even")
        lz = x._lazy
        if isinstance(lz, _PendingLinear) and lz.epi == 0:
            self.stats["linear_fused_geglu"] += 1
            return self._track(HipTensor(x.shape[:-1] + (F2 // 2,), x.dtype, None, lazy=lz.fork(F.HB_EPI_GEGLU)))
        dt = x.dtype if x.dtype in FLOAT_DT else "f32"
        st, xp, rows, _, ld = self._rows(x)
        out = self._new(x.shape[:-1] + (F2 // 2,), dt)
        if rows:
            self._call("geglu", "hb_geglu", self.ctx, DT[x.dtype][0], xp, ld, DT[dt][0], out._st.ptr, rows, F2 // 2)
        return out

    def meanPool(self, x: HipTensor, mask: HipTensor) -> HipTensor:
        self._live(x, mask, op="meanPool")
        B, L, D = x.shape
        c = self._contiguous(x)
        m = self._contiguous(mask if mask.dtype == "bool" else self.cast(mask, "bool"))
        out = self._new((B, D), "f32")
        if out.size:
            self._call("meanPool", "hb_meanpool", self.ctx, DT[x.dtype][0], self._ptr(c), self._ptr(m), B, L, D,
                       out._st.ptr)
        return out

    # ---------------------------------------------------------------- quantized weights
    def fromHostQuantized(self, h: HostQuantized, dtype: str) -> Optional[QuantizedTensor]:
        """Keeps W packed on the device (laya format v1, f16 scales / zeros).
        Declines (None) when the scales or zeros are not exactly f16 values
        or the dtype is not a float (index.ts:250-256)."""
        validate_quantized(h)
        if dtype not in FLOAT_DT:
            return None
        s32 = to_f32(h.scales)
        s16 = s32.astype(np.float16)
        if not np.array_equal(s16.astype(np.float32), s32, equal_nan=True):
            return None
        z16 = None
        if h.mode == "affine":
            z32 = to_f32(h.biases)
            z16 = z32.astype(np.float16)
            if not np.array_equal(z16.astype(np.float32), z32, equal_nan=True):
                return None
        N, K = h.shape
        G = quant_groups(K, h.groupSize)
        w = self.fromHost(HostTensor("u8", (N, K * h.bits // 8), np.asarray(h.data, np.uint8).reshape(N, -1)))
        sc = self.fromHost(HostTensor("f16", (N, G), s16.reshape(N, G)))
        zb = self.fromHost(HostTensor("f16", (N, G), z16.reshape(N, G))) if z16 is not None else None
        if sc._meta is None:
            sc._meta = {}
        sc._meta["deq_dtype"] = dtype
        return QuantizedTensor((N, K), h.bits, h.groupSize, h.mode, dtype, True, w, sc, zb)

    def quantizedLinear(self, x: HipTensor, w: HipTensor, scales: HipTensor, biases: Optional[HipTensor], opts,
                        bias: Optional[HipTensor] = None) -> HipTensor:
        """y = x . dequant(w)^T (+ bias) in x's dtype, f32 accumulation
        (index.ts:257-261).  Pending, like linear."""
        self._live(x, w, scales, biases, bias, op="quantizedLinear")
        N = w.shape[0]
        K = w.shape[1] * 8 // opts.bits
        if x.shape[-1] != K:
            raise ValueError(f"quantizedLinear: x [{x.shape}] vs w [{N}, {K}]")
        dt = x.dtype if x.dtype in FLOAT_DT else "f32"
        if x.dtype != dt:
            x = self.cast(x, dt)
        if bias is not None:
            bias = self._contiguous(bias if bias.dtype == dt else self.cast(bias, dt))
        pan = self._panel_for(x, q=(w, scales, biases, opts.groupSize))
        pend = _PendingLinear(self, x, w, bias, (scales, biases, opts.bits, opts.groupSize, opts.mode, N), panel=pan)
        return self._track(HipTensor(x.shape[:-1] + (N,), dt, None, lazy=pend))

    def quantizedEmbedding(self, w: HipTensor, scales: HipTensor, biases: Optional[HipTensor], opts,
                           ids: HipTensor) -> HipTensor:
        self._live(w, scales, biases, ids, op="quantizedEmbedding")
        V = w.shape[0]
        K = w.shape[1] * 8 // opts.bits
        dt = (scales._meta or {}).get("deq_dtype", scales.dtype)
        i = self._contiguous(ids if ids.dtype == "i32" else self.cast(ids, "i32"))
        out = self._new(ids.shape + (K,), dt)
        if out.size:
            self._call("quantizedEmbedding", "hb_qgather", self.ctx, self._ptr(w), self._ptr(scales),
                       self._ptr(biases) if biases is not None else 0, V, K, opts.bits, opts.groupSize,
                       1 if opts.mode == "affine" else 0, self._ptr(i), ids.size, DT[dt][0], out._st.ptr)
        return out

    # ---------------------------------------------------------------- timing (bench support)
    def event(self) -> int:
        ev = F.U(0)
        self._call("event", "hb_event_create", self.ctx, F.C.byref(ev))
        return ev.value

    def record(self, ev: int) -> None:
        self._call("event", "hb_event_record", self.ctx, ev)

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = F.C.c_float(0)
        self._call("event", "hb_event_elapsed", a, b, F.C.byref(ms))
        return ms.value


def createHipBackend(device: int = 0, lib_path: str | None = None, fuse_qkv: bool = False) -> HipBackend:
    """Factory named like the reference's createMlxBackend / createWebGpuBackend."""
    return HipBackend(device, lib_path, fuse_qkv)
