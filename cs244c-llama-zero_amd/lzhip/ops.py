"""Tensor-level wrappers over the C ABI.

Every function takes and returns torch tensors that live on a ROCm GPU,
validates shapes/dtypes/strides on the host, allocates outputs from torch's
caching allocator and enqueues the HIP kernel on torch's current stream.  A CPU
tensor or an unsupported dtype raises: there is no fallback computation.
"""
from __future__ import annotations

import ctypes
import math
from typing import Dict, Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import BF16, F16, F32

_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}
# 16-bit float formats (the MFMA GEMM and attention operands)
HALF_DTYPES = (torch.bfloat16, torch.float16)


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"llama-zero HIP kernels support float32, bfloat16 and float16 tensors, got {t.dtype}") from None


def require_gpu(*tensors: Optional[torch.Tensor]) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                f"llama-zero HIP kernels run on a ROCm GPU; got a tensor on {t.device}. "
                "Move the model and inputs to 'cuda'."
            )


def stream_ptr(device: Optional[torch.device] = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _row_stride(t: torch.Tensor) -> int:
    """Leading dimension of a 2-D row-major view (last stride must be 1)."""
    if t.dim() != 2:
        raise ValueError(f"expected a 2-D view, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 and t.size(1) > 1:
        raise ValueError("expected unit stride in the last dimension")
    return max(t.stride(0), t.size(1)) if t.size(0) > 1 else t.size(1)


# ---------------------------------------------------------------------------
# optimizer path
# ---------------------------------------------------------------------------

def adamw_(
    p: torch.Tensor,
    m: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    *,
    lr: float,
    beta1: float,
    beta2: float,
    eps: float,
    weight_decay: float,
    step: int,
    grad_scale: Optional[torch.Tensor] = None,
    p_out: Optional[torch.Tensor] = None,
    hyper: Optional[torch.Tensor] = None,
) -> None:
    """In-place fused AdamW on flat fp32 p/m/v with gradient g (fp32 or bf16).
    With `hyper` (float32 [3] on the device, written by adamw_step_) lr and
    step are ignored: the step-dependent factors come from device memory."""
    require_gpu(p, m, v, g, grad_scale, p_out, hyper)
    n = p.numel()
    for t, name in ((m, "exp_avg"), (v, "exp_avg_sq"), (g, "grad")):
        if t.numel() != n:
            raise ValueError(f"{name} has {t.numel()} elements, expected {n}")
    for t in (p, m, v):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("AdamW master/moment buffers must be contiguous float32")
    if not g.is_contiguous():
        raise ValueError("gradient must be contiguous")
    if grad_scale is not None and (grad_scale.dtype != torch.float32 or grad_scale.numel() < 1):
        raise ValueError("grad_scale must be a float32 device scalar")
    if p_out is not None and (p_out.numel() != n or not p_out.is_contiguous()):
        raise ValueError("p_out must be contiguous with the same number of elements")
    if hyper is not None:
        if hyper.dtype != torch.float32 or hyper.numel() < 3:
            raise ValueError("hyper must hold 3 float32 values")
        _lib.call(
            "lz_adamw_dev",
            p.data_ptr(), m.data_ptr(), v.data_ptr(), g.data_ptr(), dtype_code(g),
            _ptr(p_out), dtype_code(p_out) if p_out is not None else F32, n,
            float(beta1), float(beta2), float(eps), float(weight_decay), hyper.data_ptr(),
            _ptr(grad_scale), stream_ptr(p.device),
        )
        return
    _lib.call(
        "lz_adamw",
        p.data_ptr(), m.data_ptr(), v.data_ptr(), g.data_ptr(), dtype_code(g),
        _ptr(p_out), dtype_code(p_out) if p_out is not None else F32, n,
        float(lr), float(beta1), float(beta2), float(eps), float(weight_decay), int(step),
        _ptr(grad_scale), stream_ptr(p.device),
    )


def adamw_norm_workspace_words(n: int) -> int:
    """float64 words of workspace adamw_norm_ needs for n elements."""
    return int(_lib.load().lz_adamw_norm_workspace(int(n)))


def adamw_norm_(
    p: torch.Tensor,
    m: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    acc: torch.Tensor,
    workspace: torch.Tensor,
    *,
    lr: float,
    beta1: float,
    beta2: float,
    eps: float,
    weight_decay: float,
    step: int,
    grad_scale: Optional[torch.Tensor] = None,
    p_out: Optional[torch.Tensor] = None,
) -> None:
    """adamw_ that also adds sum(g^2) (g as stored) to acc (float64 device
    scalar) from the same read of g, in a fixed summation order; `workspace`
    is a float64 device buffer of at least adamw_norm_workspace_words(n)."""
    require_gpu(p, m, v, g, acc, workspace, grad_scale, p_out)
    n = p.numel()
    for t, name in ((m, "exp_avg"), (v, "exp_avg_sq"), (g, "grad")):
        if t.numel() != n:
            raise ValueError(f"{name} has {t.numel()} elements, expected {n}")
    for t in (p, m, v):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("AdamW master/moment buffers must be contiguous float32")
    if not g.is_contiguous():
        raise ValueError("gradient must be contiguous")
    if acc.dtype != torch.float64 or workspace.dtype != torch.float64 or not workspace.is_contiguous():
        raise ValueError("accumulator and workspace must be float64")
    if grad_scale is not None and (grad_scale.dtype != torch.float32 or grad_scale.numel() < 1):
        raise ValueError("grad_scale must be a float32 device scalar")
    if p_out is not None and (p_out.numel() != n or not p_out.is_contiguous()):
        raise ValueError("p_out must be contiguous with the same number of elements")
    _lib.call(
        "lz_adamw_norm",
        p.data_ptr(), m.data_ptr(), v.data_ptr(), g.data_ptr(), dtype_code(g),
        _ptr(p_out), dtype_code(p_out) if p_out is not None else F32, n,
        float(lr), float(beta1), float(beta2), float(eps), float(weight_decay), int(step),
        _ptr(grad_scale), acc.data_ptr(), workspace.data_ptr(), workspace.numel(), stream_ptr(p.device),
    )


def adamw_step_(step: torch.Tensor, lr: float, beta1: float, beta2: float, weight_decay: float,
                hyper: torch.Tensor) -> None:
    """step (int64 device scalar) += 1 and hyper (float32 [3]) = the AdamW
    factors of the new step, on the device: for optimizer steps replayed from
    a HIP graph."""
    require_gpu(step, hyper)
    if step.dtype != torch.int64 or step.numel() != 1 or hyper.dtype != torch.float32 or hyper.numel() < 3:
        raise ValueError("step must be one int64, hyper three float32 values")
    _lib.call("lz_adamw_step", step.data_ptr(), float(lr), float(beta1), float(beta2), float(weight_decay),
              hyper.data_ptr(), stream_ptr(step.device))


def sumsq_(x: torch.Tensor, acc: torch.Tensor) -> None:
    """acc (float64 device scalar) += sum(x^2)."""
    require_gpu(x, acc)
    if acc.dtype != torch.float64:
        raise ValueError("accumulator must be float64")
    if not x.is_contiguous():
        raise ValueError("x must be contiguous")
    _lib.call("lz_sumsq", x.data_ptr(), dtype_code(x), x.numel(), acc.data_ptr(), stream_ptr(x.device))


def sumsq_multi_(xs: Sequence[torch.Tensor], acc: torch.Tensor) -> None:
    """acc (float64 device scalar) += sum of x^2 over every tensor in xs
    (contiguous, one dtype), one launch per 24 tensors."""
    require_gpu(acc, *xs)
    if acc.dtype != torch.float64:
        raise ValueError("accumulator must be float64")
    if not xs:
        return
    dt = xs[0].dtype
    rows = []
    for x in xs:
        if x.dtype != dt or not x.is_contiguous():
            raise ValueError("sumsq_multi_ needs contiguous tensors of one dtype")
        rows += [x.data_ptr(), x.numel()]
    table = (ctypes.c_int64 * len(rows))(*rows)
    _lib.call("lz_sumsq_multi", ctypes.addressof(table), len(xs), dtype_code(xs[0]), acc.data_ptr(),
              stream_ptr(acc.device))


def adamw_multi_(ps, ms, vs, gs, p_outs, lr: float, beta1: float, beta2: float, eps: float, weight_decay: float,
                 step: int, grad_scale: Optional[torch.Tensor] = None, hyper: Optional[torch.Tensor] = None) -> None:
    """adamw_ on every (p, m, v, g, p_out) in one launch per 24 tensors: fp32
    p/m/v, gradients of one dtype, p_out all None or all of one dtype.  The
    same bits as adamw_ tensor by tensor."""
    n = len(ps)
    if not (len(ms) == len(vs) == len(gs) == len(p_outs) == n):
        raise ValueError("adamw_multi_: list lengths differ")
    if n == 0:
        return
    require_gpu(*ps, *ms, *vs, *gs, grad_scale, hyper)
    gdt = gs[0].dtype
    odt = None if p_outs[0] is None else p_outs[0].dtype
    rows = []
    for p, m, v, g, po in zip(ps, ms, vs, gs, p_outs):
        if p.dtype != torch.float32 or m.dtype != torch.float32 or v.dtype != torch.float32:
            raise ValueError("p, m and v must be float32")
        if g.dtype != gdt or (None if po is None else po.dtype) != odt:
            raise ValueError("adamw_multi_: mixed gradient or output dtypes")
        k = p.numel()
        if m.numel() != k or v.numel() != k or g.numel() != k or (po is not None and po.numel() != k):
            raise ValueError("adamw_multi_: size mismatch")
        for t in (p, m, v, g, po):
            if t is not None and not t.is_contiguous():
                raise ValueError("adamw_multi_ needs contiguous tensors")
        if po is not None:
            require_gpu(po)
        rows += [p.data_ptr(), m.data_ptr(), v.data_ptr(), g.data_ptr(), _ptr(po) or 0, k]
    if hyper is not None and (hyper.dtype != torch.float32 or hyper.numel() < 3):
        raise ValueError("hyper must hold 3 float32 values")
    table = (ctypes.c_int64 * len(rows))(*rows)
    _lib.call("lz_adamw_multi", ctypes.addressof(table), n, dtype_code(gs[0]),
              F32 if odt is None else _DTYPES[odt], float(lr), float(beta1), float(beta2), float(eps),
              float(weight_decay), int(step), _ptr(hyper), _ptr(grad_scale), stream_ptr(ps[0].device))


def clip_finalize(acc: torch.Tensor, max_norm: float, norm_out: torch.Tensor, scale_out: torch.Tensor,
                  inv_grad_scale: float = 1.0) -> None:
    """norm_out = sqrt(acc) * inv_grad_scale (the true norm of gradients that
    carry a loss scale); scale_out = inv_grad_scale * the clip factor."""
    require_gpu(acc, norm_out, scale_out)
    _lib.call(
        "lz_clip_finalize", acc.data_ptr(), float(max_norm), float(inv_grad_scale), norm_out.data_ptr(),
        scale_out.data_ptr(), stream_ptr(acc.device),
    )


def fill_(x: torch.Tensor, value: float) -> torch.Tensor:
    require_gpu(x)
    if not x.is_contiguous():
        raise ValueError("fill_ needs a contiguous tensor")
    code = 3 if x.dtype == torch.float64 else dtype_code(x)
    _lib.call("lz_fill", x.data_ptr(), code, x.numel(), float(value), stream_ptr(x.device))
    return x


def zeros(shape, dtype: torch.dtype, device) -> torch.Tensor:
    """A zero-filled device tensor written by this library's fill kernel;
    integer dtypes are filled through a float view of the same width (zero
    has the same bits)."""
    t = torch.empty(shape, dtype=dtype, device=device)
    if t.numel():
        v = t
        if not t.is_floating_point():
            views = {8: torch.float64, 4: torch.float32, 2: torch.bfloat16}
            if t.element_size() not in views:
                raise TypeError(f"zeros: no fill for {dtype}")
            v = t.view(views[t.element_size()])
        fill_(v, 0.0)
    return t


def cast(src: torch.Tensor, dtype: torch.dtype, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    require_gpu(src, out)
    if not src.is_contiguous():
        raise ValueError("cast needs a contiguous source")
    if out is None:
        out = torch.empty(src.shape, dtype=dtype, device=src.device)
    if out.numel() != src.numel() or not out.is_contiguous():
        raise ValueError("cast output must be contiguous with the same number of elements")
    _lib.call("lz_cast", src.data_ptr(), dtype_code(src), out.data_ptr(), dtype_code(out), src.numel(),
              stream_ptr(src.device))
    return out


def axpy_f32_(dst: torch.Tensor, src: torch.Tensor, alpha: float = 1.0) -> None:
    require_gpu(dst, src)
    if dst.dtype != torch.float32 or not dst.is_contiguous() or not src.is_contiguous():
        raise ValueError("axpy_f32_ needs a contiguous float32 destination and contiguous source")
    if dst.numel() != src.numel():
        raise ValueError(f"size mismatch {dst.numel()} vs {src.numel()}")
    _lib.call("lz_axpy_f32", dst.data_ptr(), src.data_ptr(), dtype_code(src), dst.numel(), float(alpha),
              stream_ptr(dst.device))


def add_(dst: torch.Tensor, src: torch.Tensor) -> None:
    require_gpu(dst, src)
    if dst.dtype != src.dtype or dst.numel() != src.numel() or not dst.is_contiguous() or not src.is_contiguous():
        raise ValueError("add_ needs contiguous tensors of one dtype and size")
    _lib.call("lz_add_inplace", dst.data_ptr(), src.data_ptr(), dtype_code(dst), dst.numel(), stream_ptr(dst.device))


def scale_(x: torch.Tensor, alpha: float) -> None:
    require_gpu(x)
    if not x.is_contiguous():
        raise ValueError("scale_ needs a contiguous tensor")
    _lib.call("lz_scale_inplace", x.data_ptr(), dtype_code(x), x.numel(), float(alpha), stream_ptr(x.device))


def scale_dev_(x: torch.Tensor, scale: torch.Tensor) -> None:
    """x *= scale[0] with `scale` a one-element fp32 device tensor."""
    require_gpu(x, scale)
    if not x.is_contiguous():
        raise ValueError("scale_dev_ needs a contiguous tensor")
    if scale.dtype != torch.float32 or scale.numel() != 1:
        raise ValueError("scale must be one fp32 element")
    _lib.call("lz_scale_dev", x.data_ptr(), dtype_code(x), x.numel(), scale.data_ptr(), stream_ptr(x.device))


class SegmentTable:
    """Device table of {ptr, numel, flat_offset} records for the multi-tensor
    gather/scatter kernels.  Built on the host, uploaded once per call site."""

    def __init__(self, records: Sequence[Tuple[int, int, int]], device: torch.device) -> None:
        if not records:
            raise ValueError("empty segment table")
        host = torch.tensor([v for rec in records for v in rec], dtype=torch.int64)
        self.nseg = len(records)
        self.device = device
        self.tensor = host.to(device, non_blocking=False)

    @classmethod
    def from_tensors(cls, tensors: Sequence[Optional[torch.Tensor]], offsets: Sequence[int],
                     numels: Sequence[int], device: torch.device) -> "SegmentTable":
        recs = []
        for t, off, n in zip(tensors, offsets, numels):
            if t is not None:
                require_gpu(t)
                if not t.is_contiguous():
                    raise ValueError("segment tensors must be contiguous")
                if t.numel() != n:
                    raise ValueError(f"segment has {t.numel()} elements, expected {n}")
            recs.append((0 if t is None else t.data_ptr(), int(n), int(off)))
        return cls(recs, device)


class HostTable:
    """{ptr, numel, flat_offset} records kept in host memory; the kernels get
    them by value, so building one per call costs no device traffic."""

    def __init__(self, records: Sequence[Tuple[int, int, int]]) -> None:
        if not records:
            raise ValueError("empty segment table")
        flat = [int(v) for rec in records for v in rec]
        self.nseg = len(records)
        self.array = (ctypes.c_int64 * len(flat))(*flat)

    @classmethod
    def from_tensors(cls, tensors: Sequence[Optional[torch.Tensor]], offsets: Sequence[int],
                     numels: Sequence[int]) -> "HostTable":
        recs = []
        for t, off, n in zip(tensors, offsets, numels):
            if t is not None:
                require_gpu(t)
                if not t.is_contiguous():
                    raise ValueError("segment tensors must be contiguous")
                if t.numel() != n:
                    raise ValueError(f"segment has {t.numel()} elements, expected {n}")
            recs.append((0 if t is None else t.data_ptr(), int(n), int(off)))
        return cls(recs)


def mt_gather_host(table: HostTable, src_dtype: torch.dtype, dst: torch.Tensor, begin: int, end: int,
                   accumulate: bool = False) -> None:
    """dst[i - begin] (=|+=) flat element i of the concatenated segments."""
    require_gpu(dst)
    if dst.numel() < end - begin or not dst.is_contiguous():
        raise ValueError("gather destination too small or not contiguous")
    _lib.call("lz_mt_gather_host", ctypes.addressof(table.array), table.nseg, _DTYPES[src_dtype], dst.data_ptr(),
              dtype_code(dst), int(begin), int(end), int(bool(accumulate)), stream_ptr(dst.device))


def mt_scatter_host(src: torch.Tensor, table: HostTable, dst_dtype: torch.dtype, begin: int, end: int) -> None:
    """flat element i of the concatenated segments = src[i - begin]."""
    require_gpu(src)
    if src.numel() < end - begin or not src.is_contiguous():
        raise ValueError("scatter source too small or not contiguous")
    _lib.call("lz_mt_scatter_host", src.data_ptr(), dtype_code(src), ctypes.addressof(table.array), table.nseg,
              _DTYPES[dst_dtype], int(begin), int(end), stream_ptr(src.device))


def mt_gather(table: SegmentTable, src_dtype: torch.dtype, dst: torch.Tensor, begin: int, end: int,
              accumulate: bool = False) -> None:
    require_gpu(dst)
    if dst.numel() < end - begin or not dst.is_contiguous():
        raise ValueError("gather destination too small or not contiguous")
    _lib.call("lz_mt_gather", table.tensor.data_ptr(), table.nseg, _DTYPES[src_dtype], dst.data_ptr(),
              dtype_code(dst), int(begin), int(end), int(bool(accumulate)), stream_ptr(dst.device))


def mt_scatter(src: torch.Tensor, table: SegmentTable, dst_dtype: torch.dtype, begin: int, end: int) -> None:
    require_gpu(src)
    if src.numel() < end - begin or not src.is_contiguous():
        raise ValueError("scatter source too small or not contiguous")
    _lib.call("lz_mt_scatter", src.data_ptr(), dtype_code(src), table.tensor.data_ptr(), table.nseg,
              _DTYPES[dst_dtype], int(begin), int(end), stream_ptr(src.device))


# ---------------------------------------------------------------------------
# model ops
# ---------------------------------------------------------------------------

def rmsnorm_fwd(x2: torch.Tensor, w: torch.Tensor, eps: float) -> Tuple[torch.Tensor, torch.Tensor]:
    require_gpu(x2, w)
    rows, cols = x2.shape
    if w.numel() != cols or w.dtype != x2.dtype or not w.is_contiguous():
        raise ValueError("RMSNorm weight must be contiguous, of the activation dtype and size dim")
    y = torch.empty((rows, cols), dtype=x2.dtype, device=x2.device)
    rstd = torch.empty((rows,), dtype=torch.float32, device=x2.device)
    _lib.call("lz_rmsnorm_fwd", x2.data_ptr(), w.data_ptr(), y.data_ptr(), rstd.data_ptr(), dtype_code(x2), rows, cols,
              _row_stride(x2), cols, float(eps), stream_ptr(x2.device))
    return y, rstd


_norm_workspaces: Dict[Tuple[int, int], torch.Tensor] = {}


def _rmsnorm_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The RMSNorm backward's dw partials for the current stream, kept
    between calls (one allocation per stream instead of one per call); calls
    on one stream never overlap."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream_ptr(device))
    ws = _norm_workspaces.get(key)
    if ws is None or ws.numel() * 4 < nbytes:
        ws = torch.empty(((max(nbytes, 16) + 15) // 16 * 4,), dtype=torch.float32, device=device)
        _norm_workspaces[key] = ws
    return ws


def rmsnorm_bwd(x2: torch.Tensor, w: torch.Tensor, rstd: torch.Tensor, dy2: torch.Tensor,
                dres: Optional[torch.Tensor] = None, need_dw: bool = True, dw_sink=None
                ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """dx and dw; with dw_sink (a GradSink holding w) dw is written or added
    into w's gradient buffer there and None is returned for it."""
    require_gpu(x2, w, rstd, dy2, dres)
    rows, cols = x2.shape
    dx = torch.empty((rows, cols), dtype=x2.dtype, device=x2.device)
    dw_acc = 0
    if dw_sink is not None and need_dw:
        dw_buf, acc = dw_sink.take(w)
        dw, dw_acc = None, int(acc)
    else:
        dw = torch.empty((cols,), dtype=w.dtype, device=w.device) if need_dw else None
        dw_buf = dw
    ws = _rmsnorm_workspace(x2.device, int(_lib.load().lz_rmsnorm_bwd_workspace(rows, cols)))
    if dres is not None:
        if dres.shape != dx.shape or dres.dtype != dx.dtype:
            raise ValueError("residual gradient must match dx")
        if _row_stride(dres) != cols or dres.stride(-1) != 1:
            dres = dres.contiguous()  # the kernel reads dres with dx's row stride
    _lib.call("lz_rmsnorm_bwd", x2.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy2.data_ptr(), _ptr(dres), dx.data_ptr(),
              _ptr(dw_buf), dw_acc, ws.data_ptr(), ws.numel() * 4, dtype_code(x2), rows, cols, _row_stride(x2),
              _row_stride(dy2), cols, stream_ptr(x2.device))
    return dx, dw


def rope_table(seq: int, hd: int, inv_freq: torch.Tensor, dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [seq, hd] in `dtype` from the hd/2 inverse frequencies; the
    position and angle are formed in inv_freq's dtype."""
    require_gpu(inv_freq)
    if inv_freq.numel() != hd // 2 or not inv_freq.is_contiguous():
        raise ValueError("inv_freq must hold hd/2 contiguous values")
    cos = torch.empty((seq, hd), dtype=dtype, device=inv_freq.device)
    sin = torch.empty((seq, hd), dtype=dtype, device=inv_freq.device)
    _lib.call("lz_rope_table", cos.data_ptr(), sin.data_ptr(), _DTYPES[dtype], seq, hd, inv_freq.data_ptr(),
              dtype_code(inv_freq), stream_ptr(cos.device))
    return cos, sin


def rope_(x2: torch.Tensor, seq: int, nheads: int, hd: int, cos: torch.Tensor, sin: torch.Tensor,
          backward: bool = False, pos_offset: int = 0) -> None:
    """In place on the first nheads*hd columns of every row of x2 (rows b*S+s)."""
    require_gpu(x2, cos, sin)
    if cos.dtype != x2.dtype or sin.dtype != x2.dtype:
        raise ValueError("RoPE tables must have the activation dtype")
    if cos.size(0) < seq + pos_offset or cos.size(1) != hd:
        raise ValueError("RoPE table too short")
    rows = x2.size(0)
    _lib.call("lz_rope", x2.data_ptr(), dtype_code(x2), _row_stride(x2), rows, seq, nheads, hd, cos.data_ptr(),
              sin.data_ptr(), int(pos_offset), int(bool(backward)), stream_ptr(x2.device))


def swiglu_fwd(g2: torch.Tensor, u2: torch.Tensor) -> torch.Tensor:
    require_gpu(g2, u2)
    rows, cols = g2.shape
    h = torch.empty((rows, cols), dtype=g2.dtype, device=g2.device)
    _lib.call("lz_swiglu_fwd", g2.data_ptr(), _row_stride(g2), u2.data_ptr(), _row_stride(u2), h.data_ptr(), cols,
              rows, cols, dtype_code(g2), stream_ptr(g2.device))
    return h


def swiglu_bwd(g2: torch.Tensor, u2: torch.Tensor, dh2: torch.Tensor, dg2: torch.Tensor, du2: torch.Tensor) -> None:
    require_gpu(g2, u2, dh2, dg2, du2)
    rows, cols = g2.shape
    _lib.call("lz_swiglu_bwd", g2.data_ptr(), _row_stride(g2), u2.data_ptr(), _row_stride(u2), dh2.data_ptr(),
              _row_stride(dh2), dg2.data_ptr(), _row_stride(dg2), du2.data_ptr(), _row_stride(du2), rows, cols,
              dtype_code(g2), stream_ptr(g2.device))


def embedding_fwd(ids: torch.Tensor, table: torch.Tensor, bad_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    require_gpu(ids, table)
    if ids.dtype != torch.int64:
        raise TypeError("token ids must be int64")
    ids_c = ids.contiguous()
    vocab, dim = table.shape
    out = torch.empty((*ids.shape, dim), dtype=table.dtype, device=table.device)
    _lib.call("lz_embedding_fwd", ids_c.data_ptr(), ids_c.numel(), table.data_ptr(), vocab, dim, out.data_ptr(), dim,
              dtype_code(table), _ptr(bad_flag), stream_ptr(table.device))
    return out


def embedding_bwd(ids: torch.Tensor, dout2: torch.Tensor, vocab: int, dtype: torch.dtype,
                  grad: Optional[torch.Tensor] = None, accumulate: Optional[bool] = None) -> torch.Tensor:
    """The table gradient; written into `grad` when given, added to it when
    accumulate (default: whenever grad is given)."""
    require_gpu(ids, dout2, grad)
    ids_c = ids.contiguous()
    dim = dout2.size(1)
    out = torch.empty((vocab, dim), dtype=dtype, device=dout2.device) if grad is None else grad
    if grad is not None and (grad.numel() != vocab * dim or not grad.is_contiguous() or grad.dtype != dtype):
        raise ValueError("embedding gradient buffer must be a contiguous [vocab, dim] tensor of the table dtype")
    acc = (grad is not None) if accumulate is None else bool(accumulate)
    ws = torch.empty((vocab * dim,), dtype=torch.float32, device=dout2.device)
    _lib.call("lz_embedding_bwd", ids_c.data_ptr(), ids_c.numel(), dout2.data_ptr(), _row_stride(dout2), vocab, dim,
              out.data_ptr(), int(acc), ws.data_ptr(), _DTYPES[dtype], stream_ptr(dout2.device))
    return out


def transpose2d(src: torch.Tensor, out: Optional[torch.Tensor] = None, ld_out: Optional[int] = None) -> torch.Tensor:
    """dst[c, r] = src[r, c] for a 2-D row-major view."""
    require_gpu(src)
    rows, cols = src.shape
    if out is None:
        ld = ld_out or rows
        out = torch.empty((cols, ld), dtype=src.dtype, device=src.device)
    ld = out.stride(0)
    _lib.call("lz_transpose", src.data_ptr(), out.data_ptr(), dtype_code(src), 1, 1, rows, cols, _row_stride(src), 0, 0,
              ld, 0, 0, stream_ptr(src.device))
    return out


def transpose_heads(x2: torch.Tensor, B: int, S: int, nheads: int, hd: int, col0: int = 0) -> torch.Tensor:
    """[B*S, ld] rows holding heads at columns col0 + h*hd  ->  [B, nheads, hd, S]."""
    require_gpu(x2)
    ld = _row_stride(x2)
    out = torch.empty((B, nheads, hd, S), dtype=x2.dtype, device=x2.device)
    base = x2.data_ptr() + col0 * x2.element_size()
    _lib.call("lz_transpose", base, out.data_ptr(), dtype_code(x2), B, nheads, S, hd, ld, S * ld, hd, S,
              nheads * hd * S, hd * S, stream_ptr(x2.device))
    return out


def copy2d(src: torch.Tensor, dst: torch.Tensor) -> torch.Tensor:
    """dst[:rows, :cols] = src for two 2-D row-major views of one dtype."""
    require_gpu(src, dst)
    if src.dtype != dst.dtype:
        raise ValueError("copy2d needs one dtype")
    rows, cols = src.shape
    _lib.call("lz_copy2d", src.data_ptr(), _row_stride(src), dst.data_ptr(), _row_stride(dst), rows, cols,
              dtype_code(src), stream_ptr(src.device))
    return dst


def _round8(n: int) -> int:
    return (n + 7) // 8 * 8


def nt_operand(t2: torch.Tensor) -> torch.Tensor:
    """Returns t2, or a zero-padded copy, as a [rows, K8] view whose leading
    dimension and reduction length are multiples of 8 with a 16-byte aligned
    base (what the MFMA GEMM requires).  Padding columns are zero, so they do
    not change the product."""
    rows, k = t2.shape
    ld = _row_stride(t2)
    if k % 8 == 0 and ld % 8 == 0 and t2.data_ptr() % 16 == 0:
        return t2
    k8 = _round8(k)
    buf = torch.empty((rows, k8), dtype=t2.dtype, device=t2.device)
    if k8 != k:
        fill_(buf, 0.0)
    copy2d(t2, buf[:, :k])
    return buf


def transpose_padded(src2: torch.Tensor) -> torch.Tensor:
    """[R, C] -> [C, R8] with zero columns R..R8 (an NT operand whose reduction
    dimension is R)."""
    rows, cols = src2.shape
    r8 = _round8(rows)
    out = torch.empty((cols, r8), dtype=src2.dtype, device=src2.device)
    if r8 != rows:
        fill_(out, 0.0)
    transpose2d(src2, out=out)
    return out


class LaunchProbe:
    """Opt-in timing of GEMM launches with HIP events recorded on the launch
    stream: (flops, start, end, kernel key) per launch, the key being
    (a_kmajor, b_kmajor, lz_gemm_plan code), or (True, True, "swiglu") /
    (True, True, "rope") for the fused gate|up + SwiGLU and QKV + RoPE
    products.  Used by the benchmark to measure the MFMA
    kernels inside a timed training step."""

    def __init__(self, only=None) -> None:
        """only: a kernel key; when set, events are recorded around that
        key's launches alone (every other launch runs without them)."""
        self.records = []
        self.only = only

    def wants(self, key) -> bool:
        return self.only is None or key == self.only

    def add(self, flops: float, start, end, key=None) -> None:
        self.records.append((flops, start, end, key))

    def summary(self, key=None) -> Tuple[int, float, float]:
        """(launches, total flops, total milliseconds) over every launch, or
        over the launches of one kernel key — call after a sync."""
        rec = [r for r in self.records if key is None or r[3] == key]
        ms = sum(s.elapsed_time(e) for _, s, e, _ in rec)
        return len(rec), sum(f for f, _, _, _ in rec), ms

    def by_key(self) -> Dict[tuple, Tuple[int, float, float]]:
        """{kernel key: (launches, flops, milliseconds)} — call after a sync."""
        return {k: self.summary(k) for k in {r[3] for r in self.records}}


def gemm_unsplit(M: int, N: int, K: int, a_kmajor: bool, b_kmajor: bool) -> bool:
    """Whether lz_gemm runs this product without splitting K."""
    return int(_lib.load().lz_gemm_plan(M, N, K, int(a_kmajor), int(b_kmajor))) % 64 == 1


def gemm_kernel_name(key) -> str:
    """Kernel name (as profilers print it, namespaces dropped) of a
    LaunchProbe key of a bf16 product."""
    ak, bk, code = key
    if code == "swiglu":
        return "gemm_swiglu_kernel"
    if code == "rope":
        return "gemm_rope_kernel<128>"
    if code == "rope64":
        return "gemm_rope_kernel<64>"
    if code == "swiglu_bwd":
        return "gemm_swiglu_bwd_kernel"
    if code == "f32":
        return f"gemm_f32_kernel<{'true' if ak else 'false'}, {'true' if bk else 'false'}>"
    cfg, splits = code // 64, code % 64
    tf = lambda b: "true" if b else "false"
    if cfg == 5:
        name = f"gemm_dma_kernel<FmtBF16, 2, 4, {tf(ak)}, {tf(bk)}, 64, 2>"
    elif cfg == 6:
        name = f"gemm_dma_n192_kernel<FmtBF16, {tf(bk)}>"
    else:
        bm, wn = (128, 2) if cfg == 2 else (256, 4 if cfg == 0 else 2)
        name = f"gemm_kernel<FmtBF16, {bm}, {bm}, 2, {wn}, {tf(ak)}, {tf(bk)}>"
    return name + (f" split-K x{splits} (+ splitk_reduce_kernel)" if splits > 1 else "")


_gemm_probe: Optional[LaunchProbe] = None


def set_gemm_probe(probe: Optional[LaunchProbe]) -> None:
    global _gemm_probe
    _gemm_probe = probe


def gemm_nt(a2: torch.Tensor, b2: torch.Tensor, out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
            residual: Optional[torch.Tensor] = None, alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """out[M,N] = alpha * a2[M,K] . b2[N,K]^T (+ beta*out) (+ residual)."""
    return gemm(a2, b2, True, True, out=out, out_dtype=out_dtype, residual=residual, alpha=alpha, beta=beta)


def _gemm_operand(t: torch.Tensor, kmajor: bool) -> Tuple[torch.Tensor, bool]:
    """Returns (operand, kmajor) satisfying the kernel's layout rules.  A
    K-major operand is zero-padded along K when needed (nt_operand); an
    M/N-major operand [K, R] whose R, row stride or base is not 8-element
    aligned is transposed into a K-major padded copy instead."""
    if kmajor:
        return nt_operand(t), True
    k, r = t.shape
    if r % 8 == 0 and _row_stride(t) % 8 == 0 and t.data_ptr() % 16 == 0 and t.stride(-1) == 1:
        return t, False
    return transpose_padded(t), True


def gemm(a: torch.Tensor, b: torch.Tensor, a_kmajor: bool = True, b_kmajor: bool = True,
         out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None,
         residual: Optional[torch.Tensor] = None, alpha: float = 1.0, beta: float = 0.0) -> torch.Tensor:
    """out[M,N] = alpha * sum_k A(m,k) B(n,k) (+ beta*out) (+ residual), two
    bf16, two fp16 or two fp32 operands, fp32 accumulation, the output in
    the operands' dtype or fp32.  `a` is [M,K] when a_kmajor else [K,M];
    `b` is [N,K] when b_kmajor else [K,N].  So x.W^T is gemm(x, W),
    dy.W is gemm(dy, W, b_kmajor=False) and dy^T.x is
    gemm(dy, x, a_kmajor=False, b_kmajor=False)."""
    require_gpu(a, b, out, residual)
    if a.dtype == torch.float32 and b.dtype == torch.float32:
        return _gemm_f32(a, b, a_kmajor, b_kmajor, out, out_dtype, residual, alpha, beta)
    if a.dtype != b.dtype or a.dtype not in HALF_DTYPES:
        raise TypeError(
            f"the MFMA GEMM takes two bfloat16, two float16 or two float32 operands (got {a.dtype}, {b.dtype})"
        )
    M, K = a.shape if a_kmajor else (a.shape[1], a.shape[0])
    N, K2 = b.shape if b_kmajor else (b.shape[1], b.shape[0])
    if K != K2:
        raise ValueError(f"GEMM reduction mismatch {K} vs {K2}")
    a, a_kmajor = _gemm_operand(a, a_kmajor)
    b, b_kmajor = _gemm_operand(b, b_kmajor)
    if K % 8 and (a_kmajor or b_kmajor):
        # a K-major operand is zero-padded to K8: bring the other one to the same K
        if not a_kmajor:
            a, a_kmajor = transpose_padded(a), True
        if not b_kmajor:
            b, b_kmajor = transpose_padded(b), True
    Kp = _round8(K) if (a_kmajor or b_kmajor) else K
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype or a.dtype, device=a.device)
    if residual is not None and (residual.dtype != a.dtype or tuple(residual.shape) != (M, N)):
        raise ValueError(f"residual must be a {a.dtype} [M, N] view")
    lib = _lib.load()
    ws_bytes = int(lib.lz_gemm_workspace(M, N, Kp, int(a_kmajor), int(b_kmajor)))
    ws = torch.empty(((ws_bytes + 15) // 16) * 4, dtype=torch.float32, device=a.device) if ws_bytes else None
    probe = _gemm_probe
    if probe is not None:
        key = (bool(a_kmajor), bool(b_kmajor), int(lib.lz_gemm_plan(M, N, Kp, int(a_kmajor), int(b_kmajor))))
        if not probe.wants(key):
            probe = None
    if probe is not None:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
    _lib.call("lz_gemm", a.data_ptr(), _row_stride(a), int(a_kmajor), b.data_ptr(), _row_stride(b), int(b_kmajor),
              dtype_code(a), out.data_ptr(), _row_stride(out), dtype_code(out), _ptr(residual),
              _row_stride(residual) if residual is not None else 0, M, N, Kp, float(alpha), float(beta), _ptr(ws),
              ws_bytes if ws is not None else 0, stream_ptr(a.device))
    if probe is not None:
        end.record()
        probe.add(2.0 * M * N * K, start, end, key)
    return out


def _unit_stride_2d(t: torch.Tensor, name: str) -> int:
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.size(1) > 1 and t.stride(1) != 1:
        raise ValueError(f"{name} needs unit stride in its last dimension")
    return _row_stride(t)


def _gemm_f32(a, b, a_kmajor, b_kmajor, out, out_dtype, residual, alpha, beta) -> torch.Tensor:
    """gemm() for float32 operands: the fp32 MFMA kernel (any shape and
    leading dimension, fp32 accumulation, fp32 or bf16 output, fp32 residual)."""
    M, K = a.shape if a_kmajor else (a.shape[1], a.shape[0])
    N, K2 = b.shape if b_kmajor else (b.shape[1], b.shape[0])
    if K != K2:
        raise ValueError(f"GEMM reduction mismatch {K} vs {K2}")
    lda, ldb = _unit_stride_2d(a, "A"), _unit_stride_2d(b, "B")
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype or torch.float32, device=a.device)
    if tuple(out.shape) != (M, N) or out.dtype not in _DTYPES:
        raise ValueError(f"out must be a float32 or bfloat16 [{M}, {N}] view")
    ldc = _unit_stride_2d(out, "out")
    ldr = 0
    if residual is not None:
        if residual.dtype != torch.float32 or tuple(residual.shape) != (M, N):
            raise ValueError("residual of a float32 GEMM must be a float32 [M, N] view")
        ldr = _unit_stride_2d(residual, "residual")
    lib = _lib.load()
    ws_bytes = int(lib.lz_gemm_f32_workspace(M, N, K))
    ws = torch.empty(((ws_bytes + 15) // 16) * 4, dtype=torch.float32, device=a.device) if ws_bytes else None
    probe = _gemm_probe
    if probe is not None and not probe.wants((bool(a_kmajor), bool(b_kmajor), "f32")):
        probe = None
    if probe is not None:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
    _lib.call("lz_gemm_f32", a.data_ptr(), lda, int(bool(a_kmajor)), b.data_ptr(), ldb, int(bool(b_kmajor)),
              out.data_ptr(), ldc, dtype_code(out), _ptr(residual), ldr, M, N, K, float(alpha), float(beta),
              _ptr(ws), ws_bytes if ws is not None else 0, stream_ptr(a.device))
    if probe is not None:
        end.record()
        probe.add(2.0 * M * N * K, start, end, (bool(a_kmajor), bool(b_kmajor), "f32"))
    return out


def swiglu_fusable(x2: torch.Tensor, w: torch.Tensor) -> bool:
    """Whether gemm_swiglu takes x2 [M, K] and w [2F, K]: M % 256, F % 128 and
    K % 64 == 0, bf16, unit column stride and 16-byte aligned rows."""
    if x2.dim() != 2 or w.dim() != 2 or x2.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        return False
    M, K = x2.shape
    n2, k2 = w.shape
    if k2 != K or n2 % 256 or M % 256 or K % 64 or M == 0:
        return False
    return all(t.stride(1) == 1 and _row_stride(t) % 8 == 0 and t.data_ptr() % 16 == 0 for t in (x2, w))


def gemm_swiglu(x2: torch.Tensor, w: torch.Tensor, gu: Optional[torch.Tensor] = None) -> torch.Tensor:
    """h = silu(x2 . w[:F]^T) * (x2 . w[F:]^T) ([M, F] bf16) for w = [gate; up]
    ([2F, K]) in one kernel; the product x2 . w^T also goes to gu ([M, 2F])
    when given.  Bit-identical to gemm(x2, w) followed by swiglu_fwd."""
    require_gpu(x2, w, gu)
    if not swiglu_fusable(x2, w):
        raise ValueError(f"gemm_swiglu: unsupported shapes/layout x {tuple(x2.shape)}, w {tuple(w.shape)}")
    M, K = x2.shape
    F = w.shape[0] // 2
    if gu is not None and (tuple(gu.shape) != (M, 2 * F) or gu.dtype != torch.bfloat16 or gu.stride(1) != 1
                           or _row_stride(gu) % 8 or gu.data_ptr() % 16):
        raise ValueError("gu must be an aligned bf16 [M, 2F] view")
    h = torch.empty((M, F), dtype=torch.bfloat16, device=x2.device)
    probe = _gemm_probe
    if probe is not None and not probe.wants((True, True, "swiglu")):
        probe = None
    if probe is not None:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
    _lib.call("lz_gemm_swiglu", x2.data_ptr(), _row_stride(x2), w.data_ptr(), _row_stride(w), _ptr(gu),
              _row_stride(gu) if gu is not None else 0, h.data_ptr(), F, M, F, K, stream_ptr(x2.device))
    if probe is not None:
        end.record()
        probe.add(2.0 * M * 2 * F * K, start, end, (True, True, "swiglu"))
    return h


def swiglu_bwd_fusable(dy2: torch.Tensor, wd: torch.Tensor, gu: torch.Tensor) -> bool:
    """Whether gemm_swiglu_bwd takes dy2 [M, K], the down weight wd [K, F] and
    gu [M, 2F]: M % 256, F % 256 and K % 64 == 0, bf16, unit column stride
    and 16-byte aligned rows."""
    if dy2.dim() != 2 or wd.dim() != 2 or gu.dim() != 2:
        return False
    if any(t.dtype != torch.bfloat16 for t in (dy2, wd, gu)):
        return False
    M, K = dy2.shape
    k2, F = wd.shape
    if k2 != K or tuple(gu.shape) != (M, 2 * F) or M % 256 or F % 256 or K % 64 or M == 0:
        return False
    return all(t.stride(1) == 1 and _row_stride(t) % 8 == 0 and t.data_ptr() % 16 == 0 for t in (dy2, wd, gu))


def gemm_swiglu_bwd(dy2: torch.Tensor, wd: torch.Tensor, gu: torch.Tensor,
                    dgu: Optional[torch.Tensor] = None) -> torch.Tensor:
    """[dgate | dup] ([M, 2F] bf16) of SwiGLU's backward on dm = dy2 . wd
    (the down projection's input gradient) with gu = [gate | up], in one
    kernel that never stores dm.  Bit-identical to gemm(dy2, wd,
    b_kmajor=False) followed by swiglu_bwd."""
    require_gpu(dy2, wd, gu, dgu)
    if not swiglu_bwd_fusable(dy2, wd, gu):
        raise ValueError(f"gemm_swiglu_bwd: unsupported shapes/layout dy {tuple(dy2.shape)}, w {tuple(wd.shape)}, "
                         f"gu {tuple(gu.shape)}")
    M, K = dy2.shape
    F = wd.shape[1]
    if dgu is None:
        dgu = torch.empty((M, 2 * F), dtype=torch.bfloat16, device=dy2.device)
    elif (tuple(dgu.shape) != (M, 2 * F) or dgu.dtype != torch.bfloat16 or dgu.stride(1) != 1
          or _row_stride(dgu) % 8 or dgu.data_ptr() % 16):
        raise ValueError("dgu must be an aligned bf16 [M, 2F] view")
    probe = _gemm_probe
    if probe is not None and not probe.wants((True, False, "swiglu_bwd")):
        probe = None
    if probe is not None:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
    _lib.call("lz_gemm_swiglu_bwd", dy2.data_ptr(), _row_stride(dy2), wd.data_ptr(), _row_stride(wd), gu.data_ptr(),
              _row_stride(gu), dgu.data_ptr(), _row_stride(dgu), M, F, K, stream_ptr(dy2.device))
    if probe is not None:
        end.record()
        probe.add(2.0 * M * F * K, start, end, (True, False, "swiglu_bwd"))
    return dgu


def rope_fusable(x2: torch.Tensor, w: torch.Tensor, nrope: int, hd: int, cos: torch.Tensor) -> bool:
    """Whether gemm_rope takes x2 [M, K] and w [N, K] with RoPE on the first
    nrope columns: head dim 128 or 64, M, N and nrope multiples of 256,
    K % 64 == 0, bf16, contiguous [>= S, hd] tables and 16-byte aligned
    rows."""
    if hd not in (128, 64) or x2.dim() != 2 or w.dim() != 2 or x2.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        return False
    M, K = x2.shape
    N, k2 = w.shape
    if k2 != K or M % 256 or N % 256 or K % 64 or nrope % 256 or nrope > N or M == 0:
        return False
    if cos.dtype != torch.bfloat16 or cos.dim() != 2 or cos.size(1) != hd or not cos.is_contiguous():
        return False
    return all(t.stride(1) == 1 and _row_stride(t) % 8 == 0 and t.data_ptr() % 16 == 0 for t in (x2, w))


def gemm_rope(x2: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, seq: int,
              nrope: int, hd: int = 128) -> torch.Tensor:
    """x2 . w^T ([M, N] bf16) with RoPE (rows b*S+s at position s) applied to
    columns [0, nrope) as heads of hd (128 or 64), in one kernel.
    Bit-identical to gemm(x2, w) followed by rope_ on those columns."""
    require_gpu(x2, w, cos, sin)
    if not rope_fusable(x2, w, nrope, hd, cos) or sin.shape != cos.shape or not sin.is_contiguous():
        raise ValueError(f"gemm_rope: unsupported shapes/layout x {tuple(x2.shape)}, w {tuple(w.shape)}")
    if cos.size(0) < seq:
        raise ValueError("RoPE table too short")
    M, K = x2.shape
    N = w.shape[0]
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x2.device)
    key = (True, True, "rope" if hd == 128 else "rope64")
    probe = _gemm_probe
    if probe is not None and not probe.wants(key):
        probe = None
    if probe is not None:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
    _lib.call("lz_gemm_rope_hd", x2.data_ptr(), _row_stride(x2), w.data_ptr(), _row_stride(w), out.data_ptr(), N,
              cos.data_ptr(), sin.data_ptr(), seq, nrope, hd, M, N, K, stream_ptr(x2.device))
    if probe is not None:
        end.record()
        probe.add(2.0 * M * N * K, start, end, key)
    return out


def ce_fwd(logits2: torch.Tensor, labels: torch.Tensor, seq: int, ignore_index: int = -100,
           lse: Optional[torch.Tensor] = None, row_loss: Optional[torch.Tensor] = None
           ) -> Tuple[torch.Tensor, torch.Tensor]:
    require_gpu(logits2, labels, lse, row_loss)
    rows, vocab = logits2.shape
    if lse is None:
        lse = torch.empty((rows,), dtype=torch.float32, device=logits2.device)
    if row_loss is None:
        row_loss = torch.empty((rows,), dtype=torch.float32, device=logits2.device)
    for t in (lse, row_loss):
        if t.dtype != torch.float32 or t.numel() != rows or not t.is_contiguous():
            raise ValueError("lse / row_loss must be contiguous fp32 with one element per row")
    _lib.call("lz_ce_fwd", logits2.data_ptr(), _row_stride(logits2), rows, vocab, dtype_code(logits2),
              labels.data_ptr(), seq, ignore_index, lse.data_ptr(), row_loss.data_ptr(), stream_ptr(logits2.device))
    return lse, row_loss


def ce_reduce(row_loss: torch.Tensor, labels: torch.Tensor, rows: int, seq: int, vocab: int, clamp: bool,
              ignore_index: int = -100) -> Tuple[torch.Tensor, torch.Tensor]:
    loss = torch.empty((), dtype=torch.float32, device=row_loss.device)
    count = torch.empty((), dtype=torch.float32, device=row_loss.device)
    _lib.call("lz_ce_reduce", row_loss.data_ptr(), labels.data_ptr(), rows, seq, vocab, ignore_index, loss.data_ptr(),
              count.data_ptr(), int(bool(clamp)), stream_ptr(row_loss.device))
    return loss, count


def ce_bwd(logits2: torch.Tensor, labels: torch.Tensor, seq: int, lse: torch.Tensor, grad_loss: torch.Tensor,
           count: torch.Tensor, out: Optional[torch.Tensor] = None, ignore_index: int = -100) -> torch.Tensor:
    require_gpu(logits2, labels, lse, grad_loss, count, out)
    rows, vocab = logits2.shape
    if out is None:
        out = torch.empty((rows, vocab), dtype=logits2.dtype, device=logits2.device)
    g = grad_loss.to(torch.float32) if grad_loss.dtype != torch.float32 else grad_loss
    g = g.contiguous()
    _lib.call("lz_ce_bwd", logits2.data_ptr(), _row_stride(logits2), rows, vocab, dtype_code(logits2), labels.data_ptr(),
              seq, ignore_index, lse.data_ptr(), g.data_ptr(), count.data_ptr(), out.data_ptr(), _row_stride(out),
              dtype_code(out), stream_ptr(logits2.device))
    return out


def attn_path(dtype: torch.dtype, S: int, hd: int, ldq: int, ldk: int, ldv: int, ldo: int) -> int:
    """2: MFMA on LDS tiles (no transposed operands), 1: MFMA with transposed
    operand buffers (V^T forward; Q^T, K^T, dO^T backward), 0: generic."""
    if dtype not in _DTYPES:
        return 0
    return int(_lib.load().lz_attn_path(_DTYPES[dtype], S, hd, ldq, ldk, ldv, ldo))


def attn_fwd(q2: torch.Tensor, k2: torch.Tensor, v2: torch.Tensor, B: int, S: int, H: int, KV: int, hd: int,
             scale: float, vt: Optional[torch.Tensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """q2/k2/v2: [B*S, ld] row views (head h at columns h*hd).  Returns
    o [B*S, H*hd] and lse [B, H, S]."""
    require_gpu(q2, k2, v2, vt)
    o = torch.empty((B * S, H * hd), dtype=q2.dtype, device=q2.device)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q2.device)
    _lib.call("lz_attn_fwd", q2.data_ptr(), _row_stride(q2), k2.data_ptr(), _row_stride(k2), v2.data_ptr(),
              _row_stride(v2), _ptr(vt), o.data_ptr(), H * hd, lse.data_ptr(), B, S, H, KV, hd, float(scale),
              dtype_code(q2), stream_ptr(q2.device))
    return o, lse


def _attn_mask_args(mask: torch.Tensor, B: int, H: int, S: int):
    """(kind, strides array) of an attention mask broadcastable to [B, H, S, S]
    (bool: True keeps the score; fp32/bf16: added to it)."""
    require_gpu(mask)
    kinds = {torch.bool: 1, torch.float32: 2, torch.bfloat16: 3, torch.float16: 4}
    if mask.dtype not in kinds:
        raise TypeError(f"attention mask must be bool, float32, bfloat16 or float16 (got {mask.dtype})")
    try:
        strides = mask.expand(B, H, S, S).stride()
    except RuntimeError as e:
        raise ValueError(f"attention mask of shape {tuple(mask.shape)} does not broadcast to {(B, H, S, S)}") from e
    return kinds[mask.dtype], (ctypes.c_int64 * 4)(*strides)


def attn_fwd_general(q2, k2, v2, B: int, S: int, H: int, KV: int, hd: int, scale: float,
                     mask: Optional[torch.Tensor] = None, dropout_p: float = 0.0, seed: int = 0):
    """attn_fwd on the one-wave-per-row kernels, with an explicit mask in
    place of the causal one (mask=None: causal) and/or attention dropout
    (dropout_p with seed, see dropout_seed); returns o, lse."""
    require_gpu(q2, k2, v2)
    kind, st = _attn_mask_args(mask, B, H, S) if mask is not None else (0, None)
    o = torch.empty((B * S, H * hd), dtype=q2.dtype, device=q2.device)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q2.device)
    _lib.call("lz_attn_fwd_general", q2.data_ptr(), _row_stride(q2), k2.data_ptr(), _row_stride(k2), v2.data_ptr(),
              _row_stride(v2), _ptr(mask), kind, ctypes.addressof(st) if st is not None else None, float(dropout_p),
              int(seed), o.data_ptr(), H * hd, lse.data_ptr(), B, S, H, KV, hd, float(scale), dtype_code(q2),
              stream_ptr(q2.device))
    return o, lse


def attn_bwd_general(q2, k2, v2, o2, do2, lse, B, S, H, KV, hd, scale, dq2, dk2, dv2,
                     mask: Optional[torch.Tensor] = None, dropout_p: float = 0.0, seed: int = 0) -> None:
    """Backward of attn_fwd_general with the forward's mask, dropout_p and
    seed."""
    require_gpu(q2, k2, v2, o2, do2, lse, dq2, dk2, dv2)
    kind, st = _attn_mask_args(mask, B, H, S) if mask is not None else (0, None)
    delta = torch.empty((B, H, S), dtype=torch.float32, device=q2.device)
    _lib.call("lz_attn_delta", o2.data_ptr(), _row_stride(o2), do2.data_ptr(), _row_stride(do2), delta.data_ptr(),
              B, S, H, hd, dtype_code(o2), stream_ptr(q2.device))
    _lib.call("lz_attn_bwd_general", q2.data_ptr(), _row_stride(q2), k2.data_ptr(), _row_stride(k2), v2.data_ptr(),
              _row_stride(v2), do2.data_ptr(), _row_stride(do2), lse.data_ptr(), delta.data_ptr(), _ptr(mask), kind,
              ctypes.addressof(st) if st is not None else None, float(dropout_p), int(seed), dq2.data_ptr(),
              _row_stride(dq2), dk2.data_ptr(), _row_stride(dk2), dv2.data_ptr(), _row_stride(dv2), B, S, H, KV, hd,
              float(scale), dtype_code(q2), stream_ptr(q2.device))


_MASK64 = (1 << 64) - 1


def _mix64(z: int) -> int:
    """SplitMix64's output function (Steele, Lea & Flood, OOPSLA 2014)."""
    z &= _MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK64
    return z ^ (z >> 31)


def dropout_seed(device: torch.device) -> int:
    """The stream key of one dropout call, drawn from the device's torch
    generator as torch's own GPU dropout draws its Philox (seed, offset):
    the key mixes the generator's seed and offset, and the offset advances
    by 4.  torch.manual_seed, torch.cuda.set_rng_state and the activation
    checkpoint's RNG replay therefore replay the masks."""
    if device.type != "cuda":
        raise RuntimeError(f"lzhip dropout needs a GPU tensor (got device {device})")
    idx = device.index if device.index is not None else torch.cuda.current_device()
    gen = torch.cuda.default_generators[idx]
    off = int(gen.get_offset())
    gen.set_offset(off + 4)
    return dropout_key(int(gen.initial_seed()), off)


def dropout_key(seed: int, offset: int) -> int:
    return _mix64((seed & _MASK64) ^ _mix64(offset + 0x9E3779B97F4A7C15))


def dropout_(x: torch.Tensor, p: float, seed: int, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = x * keep / (1 - p) (out=None: in place), keep from (seed, flat
    element index); the same call with the same seed is its backward."""
    require_gpu(x, out)
    if not x.is_contiguous():
        raise ValueError("dropout_: x must be contiguous")
    y = x if out is None else out
    if y.shape != x.shape or y.dtype != x.dtype or not y.is_contiguous():
        raise ValueError("dropout_: out must be a contiguous tensor of x's shape and dtype")
    if not 0.0 <= p <= 1.0:
        raise ValueError(f"dropout probability has to be between 0 and 1, but got {p}")
    _lib.call("lz_dropout", x.data_ptr(), y.data_ptr(), x.numel(), float(p), int(seed), dtype_code(x),
              stream_ptr(x.device))
    return y


def dropout_mask(n: int, p: float, seed: int, device: torch.device) -> torch.Tensor:
    """The keep mask (uint8, 1 = kept) that dropout_ and attention dropout
    use for elements 0..n-1 of seed's stream."""
    keep = torch.empty(n, dtype=torch.uint8, device=device)
    require_gpu(keep)
    _lib.call("lz_dropout_mask", keep.data_ptr(), n, float(p), int(seed), stream_ptr(keep.device))
    return keep


def attn_bwd(q2, k2, v2, o2, do2, lse, B, S, H, KV, hd, scale, dq2, dk2, dv2, qt=None, kt=None, dot=None,
             rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> None:
    """dq2/dk2/dv2 = gradients of causal GQA attention.  With rope = (cos,
    sin) (rope_'s tables), dq2 and dk2 are the gradients of q and k before
    RoPE: the RoPE backward is applied in the same call."""
    require_gpu(q2, k2, v2, o2, do2, lse, dq2, dk2, dv2)
    rc = rs = None
    if rope is not None:
        rc, rs = rope
        require_gpu(rc, rs)
        if rc.dtype != q2.dtype or rs.dtype != q2.dtype or rc.size(0) < S or tuple(rc.shape[1:]) != (hd,) \
                or rs.shape != rc.shape or not (rc.is_contiguous() and rs.is_contiguous()):
            raise ValueError("RoPE tables must be contiguous [>= S, hd] in the activation dtype")
    delta = torch.empty((B, H, S), dtype=torch.float32, device=q2.device)
    strides = [_row_stride(t) for t in (q2, k2, v2, do2, o2, dq2, dk2, dv2)]
    if (attn_path(q2.dtype, S, hd, *strides[:4]) == 2 and strides[4] % 8 == 0
            and all(st % 4 == 0 for st in strides[5:])
            and all(t.data_ptr() % 16 == 0 for t in (q2, k2, v2, o2, do2))):
        # LDS-tile kernels: the dQ pass computes delta from the O and dO rows
        # and runs first (no separate delta launch)
        _lib.call("lz_attn_bwd_with_o", q2.data_ptr(), strides[0], k2.data_ptr(), strides[1], v2.data_ptr(),
                  strides[2], o2.data_ptr(), strides[4], do2.data_ptr(), strides[3], lse.data_ptr(),
                  delta.data_ptr(), dq2.data_ptr(), strides[5], dk2.data_ptr(), strides[6], dv2.data_ptr(),
                  strides[7], B, S, H, KV, hd, float(scale), _ptr(rc), _ptr(rs), dtype_code(q2),
                  stream_ptr(q2.device))
        return
    _lib.call("lz_attn_delta", o2.data_ptr(), _row_stride(o2), do2.data_ptr(), _row_stride(do2), delta.data_ptr(),
              B, S, H, hd, dtype_code(o2), stream_ptr(q2.device))
    _lib.call("lz_attn_bwd", q2.data_ptr(), _row_stride(q2), k2.data_ptr(), _row_stride(k2), v2.data_ptr(),
              _row_stride(v2), do2.data_ptr(), _row_stride(do2), lse.data_ptr(), delta.data_ptr(), _ptr(qt), _ptr(kt),
              _ptr(dot), dq2.data_ptr(), _row_stride(dq2), dk2.data_ptr(), _row_stride(dk2), dv2.data_ptr(),
              _row_stride(dv2), B, S, H, KV, hd, float(scale), _ptr(rc), _ptr(rs), dtype_code(q2),
              stream_ptr(q2.device))
