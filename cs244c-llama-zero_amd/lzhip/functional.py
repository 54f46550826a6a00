"""Autograd functions of the LLaMA training step, each backed by the HIP kernels.

The model modules call these; every forward and backward pass below runs the
gfx950 kernels of libllamazero_hip.so (through lzhip.ops).  Activations are 2-D
row views [tokens, features]; projections that the reference computes as
separate nn.Linear calls on the same input (q/k/v, gate/up) run as one GEMM
over the concatenated weight rows.
"""
from __future__ import annotations

import math
import threading
from contextlib import contextmanager
from typing import Iterator, List, Optional, Sequence, Tuple

import torch
from torch.autograd import Function

from . import ops

_local = threading.local()


@contextmanager
def output_unused() -> Iterator[None]:
    """Marks a module call whose output value nobody reads: the ZeRO-3
    recompute in backward (reference zero/stage3_optimizer.py:213-237) runs the
    module again only to take autograd.grad of its output with the incoming
    gradient, which needs the output's graph, not its value.  The op that
    produces a module's output may then leave the value uncomputed (its
    backward must not need it); the gradients are the same."""
    prev = getattr(_local, "output_unused", False)
    _local.output_unused = True
    try:
        yield
    finally:
        _local.output_unused = prev


def output_is_unused() -> bool:
    """Whether the current module call runs under output_unused()."""
    return getattr(_local, "output_unused", False)


def _rows(t: torch.Tensor) -> torch.Tensor:
    """[..., C] -> [rows, C] view (copies only if the layout cannot be viewed)."""
    if not t.is_contiguous():
        t = t.contiguous()
    return t.view(-1, t.shape[-1])


@torch.no_grad()
def pack_parameters_(module: torch.nn.Module) -> int:
    """Re-points every parameter of `module` (tied ones once) at a view of one
    flat device buffer per dtype, in registration order, so that q/k/v and
    gate/up sit adjacent and fused_weight returns views instead of copying
    them on every forward and backward.  Values, Parameter objects and
    state_dict are unchanged.  Returns the number of parameters packed."""
    params, seen = [], set()
    for prm in module.parameters():
        if id(prm) not in seen:
            seen.add(id(prm))
            params.append(prm)
    by_dtype = {}
    for prm in params:
        ops.require_gpu(prm)
        by_dtype.setdefault(prm.dtype, []).append(prm)
    for dtype, group in by_dtype.items():
        flat = torch.empty(sum(prm.numel() for prm in group), dtype=dtype, device=group[0].device)
        off = 0
        for prm in group:
            n = prm.numel()
            view = flat[off : off + n].view(prm.shape)
            ops.copy2d(prm.data.contiguous().view(-1, prm.shape[-1] if prm.dim() else 1),
                       view.view(-1, prm.shape[-1] if prm.dim() else 1))
            prm.data = view
            off += n
    return len(params)


class GradSink:
    """Parameter gradients written by the backward kernels themselves, for
    gradient accumulation over micro-batches (reference train.py:236-257:
    zero_grad, then (loss / GA).backward() per micro-batch).

    Every parameter's .grad is a view of one flat buffer per dtype.  The
    first backward of a step writes each weight gradient over its .grad (the
    GEMM with beta 0, the RMSNorm and embedding kernels without their
    accumulate flag); later ones add into it (beta 1, accumulate), and the
    autograd Functions return no gradient for the parameter.  So autograd
    neither adds the micro-batches' gradients nor sums the tied weight's two
    contributions with its own kernels.  Call begin_step() where the
    reference calls optimizer.zero_grad(); finish() sets the gradients of
    parameters no backward reached to None.  Engines that read gradients through
    autograd hooks (ZeRO stage 2) must not be combined with a sink."""

    def __init__(self, module: torch.nn.Module) -> None:
        self.params: List[torch.nn.Parameter] = []
        seen = set()
        for prm in module.parameters():
            if prm.requires_grad and id(prm) not in seen:
                seen.add(id(prm))
                self.params.append(prm)
        by_dtype = {}
        for prm in self.params:
            ops.require_gpu(prm)
            by_dtype.setdefault(prm.dtype, []).append(prm)
        self.flat = {}
        self._views = {}
        for dtype, group in by_dtype.items():
            flat = ops.zeros((sum(prm.numel() for prm in group),), dtype, group[0].device)
            self.flat[dtype] = flat
            off = 0
            for prm in group:
                self._views[id(prm)] = flat[off : off + prm.numel()].view(prm.shape)
                off += prm.numel()
        self._fresh = {id(prm): True for prm in self.params}
        for prm in self.params:
            prm._lz_grad_sink = self
        self.begin_step()

    def begin_step(self) -> None:
        for prm in self.params:
            prm.grad = self._views[id(prm)]
            self._fresh[id(prm)] = True

    def take(self, prm: torch.Tensor) -> Tuple[torch.Tensor, bool]:
        """(gradient buffer, accumulate?) for the next write of prm's gradient."""
        fresh = self._fresh[id(prm)]
        self._fresh[id(prm)] = False
        if prm.grad is not self._views[id(prm)]:
            prm.grad = self._views[id(prm)]
        return self._views[id(prm)], not fresh

    def finish(self) -> None:
        """Leaves .grad None on parameters that no backward of the step
        reached, as zero_grad(set_to_none=True) followed by backward does
        (reference train.py:231), so optimizers skip them: no weight decay and
        no moment decay for a parameter the step did not use."""
        for prm in self.params:
            if self._fresh[id(prm)]:
                prm.grad = None

    def detach(self) -> None:
        for prm in self.params:
            if getattr(prm, "_lz_grad_sink", None) is self:
                del prm._lz_grad_sink


def _sink(weight: torch.Tensor) -> Optional[GradSink]:
    return getattr(weight, "_lz_grad_sink", None)


def _sink_views(weights: Sequence[torch.Tensor]) -> Optional[Tuple[torch.Tensor, bool]]:
    """The fused gradient buffer of weights that share one sink, as a view
    over their adjacent .grad buffers, and whether it accumulates; None when
    any weight has no sink or the buffers are not adjacent."""
    sinks = [_sink(w) for w in weights]
    if sinks[0] is None or any(sk is not sinks[0] for sk in sinks):
        return None
    sink = sinks[0]
    views = [sink._views[id(w)] for w in weights]
    fused = fused_weight(views)
    if len(views) > 1 and fused.data_ptr() != views[0].data_ptr():
        return None
    if fused.untyped_storage().data_ptr() != views[0].untyped_storage().data_ptr():
        return None
    accs = [sink.take(w)[1] for w in weights]
    if len(set(accs)) != 1:
        raise RuntimeError("fused weights reached the gradient sink out of step")
    return fused, accs[0]


def fused_weight(weights: Sequence[torch.Tensor]) -> torch.Tensor:
    """Concatenation of weight matrices along their output rows.  When the
    storages are already adjacent (parameters that are views of one flat
    buffer in registration order) this is a view; otherwise a copy."""
    w0 = weights[0]
    if len(weights) == 1:
        return w0
    k = w0.shape[1]
    n_total = sum(w.shape[0] for w in weights)
    base = w0.untyped_storage().data_ptr()
    adjacent = all(
        w.is_contiguous() and w.dtype == w0.dtype and w.shape[1] == k and w.untyped_storage().data_ptr() == base
        for w in weights
    )
    if adjacent:
        expect = w0.data_ptr()
        for w in weights:
            if w.data_ptr() != expect:
                adjacent = False
                break
            expect += w.numel() * w.element_size()
    if adjacent:
        return w0.as_strided((n_total, k), (k, 1), w0.storage_offset())
    out = torch.empty((n_total, k), dtype=w0.dtype, device=w0.device)
    r = 0
    for w in weights:
        ops.copy2d(w.view(w.shape[0], k), out[r : r + w.shape[0]])
        r += w.shape[0]
    return out


_side_streams = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for a product that runs
    beside another one."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    st = _side_streams.get(idx)
    if st is None:
        st = torch.cuda.Stream(device=idx)
        _side_streams[idx] = st
    return st


def _linear_fwd(x2: torch.Tensor, w: torch.Tensor, residual2: Optional[torch.Tensor] = None) -> torch.Tensor:
    return ops.gemm(x2, w, residual=residual2)


def _linear_bwd(dy2: torch.Tensor, x2: torch.Tensor, w: torch.Tensor, need_dx: bool, need_dw: bool,
                sink_weights: Optional[Sequence[torch.Tensor]] = None
                ) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
    """dx = dy . W (W read N-major), dW = dy^T . x (both read M/N-major): the
    GEMM consumes the stored layouts directly, nothing is transposed.  With
    `sink_weights` (the weights whose rows make up w) in a GradSink, dW goes
    straight into their gradient buffers and None is returned for it."""
    dx = dw = None
    if need_dx:
        dx = ops.gemm(dy2, w, b_kmajor=False)  # [M, K]
    if need_dw:
        target = _sink_views(sink_weights) if sink_weights is not None else None
        if target is not None:
            buf, acc = target
            ops.gemm(dy2, x2, a_kmajor=False, b_kmajor=False, out=buf.view(w.shape), beta=1.0 if acc else 0.0)
        else:
            dw = ops.gemm(dy2, x2, a_kmajor=False, b_kmajor=False, out_dtype=w.dtype)  # [N, K]
            if sink_weights is not None and _sink(sink_weights[0]) is not None:
                # sink buffers that are not adjacent: hand each weight its rows
                r = 0
                for wt in sink_weights:
                    buf, acc = _sink(wt).take(wt)
                    part = dw[r : r + wt.shape[0]]
                    if acc:
                        ops.add_(buf, part)
                    else:
                        ops.copy2d(part, buf.view(part.shape))
                    r += wt.shape[0]
                dw = None
    return dx, dw


class LinearFn(Function):
    """y = x . W^T (+ residual) — nn.Linear without bias (model/llama.py:81-84,
    133, 139-141, 178) with the block's residual add folded into the GEMM
    epilogue (model/llama.py:158-159)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, residual: Optional[torch.Tensor]):
        x2 = _rows(x)
        r2 = _rows(residual) if residual is not None else None
        y = _linear_fwd(x2, weight, r2)
        ctx.save_for_backward(x2, weight)
        ctx.has_residual = residual is not None
        ctx.in_shape = x.shape
        return y.view(*x.shape[:-1], weight.shape[0])

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        x2, weight = ctx.saved_tensors
        dy2 = _rows(dy)
        dx, dw = _linear_bwd(dy2, x2, weight, ctx.needs_input_grad[0], ctx.needs_input_grad[1], [weight])
        if dx is not None:
            dx = dx.view(ctx.in_shape)
        dres = dy if (ctx.has_residual and ctx.needs_input_grad[2]) else None
        return dx, dw, dres


def linear(x: torch.Tensor, weight: torch.Tensor, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    return LinearFn.apply(x, weight, residual)


class RMSNormFn(Function):
    """RMSNorm (model/llama.py:14-22) forward/backward kernels."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, eps: float):
        x2 = _rows(x)
        y, rstd = ops.rmsnorm_fwd(x2, weight, eps)
        ctx.save_for_backward(x2, weight, rstd)
        ctx.in_shape = x.shape
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        x2, weight, rstd = ctx.saved_tensors
        dx, dw = ops.rmsnorm_bwd(x2, weight, rstd, _rows(dy), need_dw=ctx.needs_input_grad[1],
                                 dw_sink=_sink(weight) if ctx.needs_input_grad[1] else None)
        return dx.view(ctx.in_shape), dw, None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return RMSNormFn.apply(x, weight, eps)


class RMSNormResidualFn(Function):
    """(rmsnorm(x), x): the pre-norm block reads x twice — through the norm
    and as the residual.  Returning x from here makes this function the only
    consumer of x, so its backward adds the residual gradient inside the
    RMSNorm backward kernel instead of autograd summing two gradients."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, weight: torch.Tensor, eps: float):
        x2 = _rows(x)
        y, rstd = ops.rmsnorm_fwd(x2, weight, eps)
        ctx.save_for_backward(x2, weight, rstd)
        ctx.in_shape = x.shape
        return y.view(x.shape), x.view_as(x)

    @staticmethod
    def backward(ctx, dy: torch.Tensor, dres: Optional[torch.Tensor]):
        x2, weight, rstd = ctx.saved_tensors
        if dy is None:
            return dres, None, None
        r2 = _rows(dres) if dres is not None else None
        dx, dw = ops.rmsnorm_bwd(x2, weight, rstd, _rows(dy), dres=r2, need_dw=ctx.needs_input_grad[1],
                                 dw_sink=_sink(weight) if ctx.needs_input_grad[1] else None)
        return dx.view(ctx.in_shape), dw, None


def rms_norm_with_residual(x: torch.Tensor, weight: torch.Tensor, eps: float):
    return RMSNormResidualFn.apply(x, weight, eps)


class RopeFn(Function):
    """apply_rotary_pos_emb on a [..., S, hd] tensor (model/llama.py:25-39)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
        seq, hd = x.shape[-2], x.shape[-1]
        out = x.contiguous().clone() if x.is_contiguous() else x.contiguous()
        ops.rope_(out.view(-1, hd), seq, 1, hd, cos, sin)
        ctx.save_for_backward(cos, sin)
        ctx.seq, ctx.hd = seq, hd
        return out

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        cos, sin = ctx.saved_tensors
        g = dy.contiguous().clone() if dy.is_contiguous() else dy.contiguous()
        ops.rope_(g.view(-1, ctx.hd), ctx.seq, 1, ctx.hd, cos, sin, backward=True)
        return g, None, None


class AttnProjFn(Function):
    """Fused QKV projection + RoPE + causal GQA flash attention
    (model/llama.py:95-117).  Input h [B, S, d] (the normed residual stream),
    weights Wq [H*hd, d], Wk/Wv [KV*hd, d]; returns the attention output
    [B, S, H*hd] that o_proj consumes.  mask: SDPA's attn_mask in place of
    the causal mask; dropout_p > 0: attention dropout with the stream key
    `seed` (both on the one-wave-per-row kernels)."""

    @staticmethod
    def forward(ctx, h, wq, wk, wv, cos, sin, n_heads: int, n_kv: int, scale: float, mask=None,
                dropout_p: float = 0.0, seed: int = 0):
        B, S, d = h.shape
        hd = wq.shape[0] // n_heads
        h2 = _rows(h)
        w = fused_weight([wq, wk, wv])
        nrope = (n_heads + n_kv) * hd
        if ops.rope_fusable(h2, w, nrope, hd, cos):
            qkv = ops.gemm_rope(h2, w, cos, sin, S, nrope, hd)  # RoPE in the GEMM's epilogue
        else:
            qkv = _linear_fwd(h2, w)                         # [B*S, (H+2KV)*hd]
            ops.rope_(qkv, S, n_heads + n_kv, hd, cos, sin)  # q and k heads, in place
        H, KV = n_heads, n_kv
        q2 = qkv[:, : H * hd]
        k2 = qkv[:, H * hd : (H + KV) * hd]
        v2 = qkv[:, (H + KV) * hd :]
        ld = qkv.shape[1]
        general = mask is not None or dropout_p > 0.0
        if general:
            o, lse = ops.attn_fwd_general(q2, k2, v2, B, S, H, KV, hd, scale, mask, dropout_p, seed)
        else:
            vt = None
            if ops.attn_path(qkv.dtype, S, hd, ld, ld, ld, H * hd) == 1:
                vt = ops.transpose_heads(qkv, B, S, KV, hd, col0=(H + KV) * hd)
            o, lse = ops.attn_fwd(q2, k2, v2, B, S, H, KV, hd, scale, vt)
        ctx.save_for_backward(h2, wq, wk, wv, qkv, o, lse, cos, sin)
        ctx.mask = mask
        ctx.general = (general, dropout_p, seed)
        ctx.meta = (B, S, H, KV, hd, scale)
        return o.view(B, S, H * hd)

    @staticmethod
    def backward(ctx, do):
        h2, wq, wk, wv, qkv, o, lse, cos, sin = ctx.saved_tensors
        B, S, H, KV, hd, scale = ctx.meta
        do2 = _rows(do)
        ld = qkv.shape[1]
        dqkv = torch.empty_like(qkv)
        q2, k2, v2 = qkv[:, : H * hd], qkv[:, H * hd : (H + KV) * hd], qkv[:, (H + KV) * hd :]
        dq2, dk2, dv2 = dqkv[:, : H * hd], dqkv[:, H * hd : (H + KV) * hd], dqkv[:, (H + KV) * hd :]
        general, dropout_p, seed = ctx.general
        if general:
            ops.attn_bwd_general(q2, k2, v2, o, do2, lse, B, S, H, KV, hd, scale, dq2, dk2, dv2, ctx.mask,
                                 dropout_p, seed)
        else:
            qt = kt = dot = None
            if ops.attn_path(qkv.dtype, S, hd, ld, ld, ld, do2.stride(0)) == 1:
                qt = ops.transpose_heads(qkv, B, S, H, hd, col0=0)
                kt = ops.transpose_heads(qkv, B, S, KV, hd, col0=H * hd)
                dot = ops.transpose_heads(do2, B, S, H, hd, col0=0)
            ops.attn_bwd(q2, k2, v2, o, do2, lse, B, S, H, KV, hd, scale, dq2, dk2, dv2, qt=qt, kt=kt, dot=dot)
        # RoPE's backward as its own pass over dq|dk: attn_bwd(rope=...) can
        # fold it into the dQ/dK stores, but in the MFMA output layout each
        # lane's table reads are 8-byte pieces of 32 different rows, which
        # cost more than this coalesced pass
        ops.rope_(dqkv, S, H + KV, hd, cos, sin, backward=True)
        need_w = any(ctx.needs_input_grad[1:4])
        w = fused_weight([wq, wk, wv])
        dh2, dw = _linear_bwd(dqkv, h2, w, ctx.needs_input_grad[0], need_w, [wq, wk, wv])
        dwq = dwk = dwv = None
        if dw is not None:
            nq, nk = wq.shape[0], wk.shape[0]
            dwq, dwk, dwv = dw[:nq], dw[nq : nq + nk], dw[nq + nk :]
        dh = dh2.view(B, S, -1) if dh2 is not None else None
        return dh, dwq, dwk, dwv, None, None, None, None, None, None, None, None


class MLPFn(Function):
    """SwiGLU MLP (model/llama.py:136-146): down(silu(gate x) * up x), gate and
    up as one GEMM, with an optional residual added in the down projection's
    epilogue.  dropout_p > 0: the gated activations pass through dropout
    (model/llama.py:146) with the stream key `seed` before the down
    projection."""

    @staticmethod
    def forward(ctx, x, wg, wu, wd, residual, grad_wanted=True, dropout_p: float = 0.0, seed: int = 0,
                compute_output: bool = True):
        x2 = _rows(x)
        F_ = wg.shape[0]
        w = fused_weight([wg, wu])
        if ops.swiglu_fusable(x2, w):
            # one kernel: the gate|up product and silu(gate) * up from its
            # epilogue; gate|up is stored only when the backward needs it
            gu = torch.empty((x2.shape[0], 2 * F_), dtype=x2.dtype, device=x2.device) if grad_wanted else None
            m = ops.gemm_swiglu(x2, w, gu=gu)
        else:
            gu = _linear_fwd(x2, w)                 # [T, 2F]
            m = ops.swiglu_fwd(gu[:, :F_], gu[:, F_:])
        if dropout_p > 0.0:
            ops.dropout_(m, dropout_p, seed)  # the saved m is the dropped-out input of down_proj
        ctx.dropout = (dropout_p, seed)
        r2 = _rows(residual) if residual is not None else None
        if compute_output:
            y = _linear_fwd(m, wd, r2)
        else:
            # the caller reads only the graph (output_unused): the down
            # projection's product is not formed; the backward needs m, not y
            y = torch.empty((m.shape[0], wd.shape[0]), dtype=m.dtype, device=m.device)
        if grad_wanted:
            ctx.save_for_backward(x2, wg, wu, wd, gu, m)
        ctx.has_residual = residual is not None
        ctx.in_shape = x.shape
        return y.view(*x.shape[:-1], wd.shape[0])

    @staticmethod
    def backward(ctx, dy):
        x2, wg, wu, wd, gu, m = ctx.saved_tensors
        F_ = wg.shape[0]
        dy2 = _rows(dy)
        dropout_p, seed = ctx.dropout
        if dropout_p == 0.0 and ops.swiglu_bwd_fusable(dy2, wd, gu):
            # dm = dy . W_down goes straight into SwiGLU's backward in the
            # GEMM's epilogue (same bits as the two kernels, dm never stored).
            # An unsplit W_down gradient runs beside it on a second stream:
            # that kernel's epilogue phases are HBM-bound with the matrix
            # cores idle, the weight gradient's main loop is the opposite
            # (1B shapes: 752 -> 709 us for the pair).  A split one (125M:
            # 8 ways and a reduce) already fills the chip and measured no
            # gain; other layers' input and weight gradients run slower
            # side by side, so they do not.
            # (one stream while a graph is being captured)
            if (ctx.needs_input_grad[3] and not torch.cuda.is_current_stream_capturing()
                    and ops.gemm_unsplit(wd.shape[0], wd.shape[1], dy2.shape[0], False, False)):
                main = torch.cuda.current_stream(dy2.device)
                side = _side_stream(dy2.device)
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    _, dwd = _linear_bwd(dy2, m, wd, False, True, [wd])
                dgu = ops.gemm_swiglu_bwd(dy2, wd, gu)
                main.wait_stream(side)
                if dwd is not None:
                    dwd.record_stream(main)  # made on the side stream, read on this one
            else:
                dgu = ops.gemm_swiglu_bwd(dy2, wd, gu)
                _, dwd = _linear_bwd(dy2, m, wd, False, ctx.needs_input_grad[3], [wd])
        else:
            dm, dwd = _linear_bwd(dy2, m, wd, True, ctx.needs_input_grad[3], [wd])
            if dropout_p > 0.0:
                ops.dropout_(dm, dropout_p, seed)  # the forward's keep mask and scale
            dgu = torch.empty_like(gu)
            ops.swiglu_bwd(gu[:, :F_], gu[:, F_:], dm, dgu[:, :F_], dgu[:, F_:])
        w = fused_weight([wg, wu])
        need_w = ctx.needs_input_grad[1] or ctx.needs_input_grad[2]
        dx2, dw = _linear_bwd(dgu, x2, w, ctx.needs_input_grad[0], need_w, [wg, wu])
        dwg = dwu = None
        if dw is not None:
            dwg, dwu = dw[:F_], dw[F_:]
        dx = dx2.view(ctx.in_shape) if dx2 is not None else None
        dres = dy if (ctx.has_residual and ctx.needs_input_grad[4]) else None
        return dx, dwg, dwu, dwd, dres, None, None, None, None


class DropoutFn(Function):
    """nn.Dropout in training mode (model/llama.py:175,213 on the token
    embeddings): x * keep / (1 - p) with the keep mask of the stream key
    `seed`; the backward regenerates the mask instead of storing it."""

    @staticmethod
    def forward(ctx, x, p: float, seed: int):
        xc = x.contiguous()
        y = ops.dropout_(xc, p, seed, out=torch.empty_like(xc))
        ctx.p, ctx.seed = p, seed
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        g = dy.contiguous()
        return ops.dropout_(g, ctx.p, ctx.seed, out=torch.empty_like(g)), None, None


def dropout(x: torch.Tensor, p: float, training: bool = True) -> torch.Tensor:
    """F.dropout on the HIP kernel (identity when not training or p == 0)."""
    if not training or p == 0.0:
        return x
    if not 0.0 <= p <= 1.0:
        raise ValueError(f"dropout probability has to be between 0 and 1, but got {p}")
    return DropoutFn.apply(x, float(p), ops.dropout_seed(x.device))


class SwiGLUPointwiseFn(Function):
    """silu(g) * u alone (for callers that keep the projections separate)."""

    @staticmethod
    def forward(ctx, g, u):
        h = ops.swiglu_fwd(_rows(g), _rows(u))
        ctx.save_for_backward(g, u)
        return h.view(g.shape)

    @staticmethod
    def backward(ctx, dh):
        g, u = ctx.saved_tensors
        g2, u2 = _rows(g), _rows(u)
        dg = torch.empty_like(g2)
        du = torch.empty_like(u2)
        ops.swiglu_bwd(g2, u2, _rows(dh), dg, du)
        return dg.view(g.shape), du.view(u.shape)


class EmbeddingFn(Function):
    """Token embedding lookup (model/llama.py:174,212)."""

    @staticmethod
    def forward(ctx, ids, weight):
        out = ops.embedding_fwd(ids, weight)
        ctx.save_for_backward(ids)
        ctx.vocab, ctx.dtype = weight.shape[0], weight.dtype
        ctx.sink_weight = weight if _sink(weight) is not None else None
        return out

    @staticmethod
    def backward(ctx, dout):
        (ids,) = ctx.saved_tensors
        if not ctx.needs_input_grad[1]:
            return None, None
        if ctx.sink_weight is not None:
            buf, acc = _sink(ctx.sink_weight).take(ctx.sink_weight)
            ops.embedding_bwd(ids, _rows(dout), ctx.vocab, ctx.dtype, grad=buf, accumulate=acc)
            return None, None
        grad = ops.embedding_bwd(ids, _rows(dout), ctx.vocab, ctx.dtype)
        return None, grad


class CrossEntropyFn(Function):
    """Mean shifted cross entropy of [B, S, V] logits against labels [B, S]
    (model/llama.py:273-302).  clamp=True divides by max(count, 1) (the chunked
    variant); clamp=False divides by count (F.cross_entropy's mean).  With
    inplace=True the backward writes the logits gradient over the saved logits
    (only when no one else reads them)."""

    @staticmethod
    def forward(ctx, logits, labels, clamp: bool, inplace: bool):
        B, S, V = logits.shape
        l2 = _rows(logits)
        lab = labels.contiguous()
        lse, row_loss = ops.ce_fwd(l2, lab, S)
        loss, count = ops.ce_reduce(row_loss, lab, B * S, S, V, clamp)
        ctx.save_for_backward(l2, lab, lse, count)
        ctx.shape = (B, S, V)
        ctx.inplace = inplace
        return loss

    @staticmethod
    def backward(ctx, gloss):
        l2, lab, lse, count = ctx.saved_tensors
        B, S, V = ctx.shape
        out = l2 if ctx.inplace else None
        d = ops.ce_bwd(l2, lab, S, lse, gloss.reshape(1), count, out=out)
        return d.view(B, S, V), None, None, None


def cross_entropy(logits: torch.Tensor, labels: torch.Tensor, clamp: bool, inplace: bool = False) -> torch.Tensor:
    return CrossEntropyFn.apply(logits, labels, clamp, inplace)


class LMHeadCEFn(Function):
    """Fused LM head + shifted cross entropy: the tied lm_head product
    (model/llama.py:178) and the loss of model/llama.py:273-302 without ever
    holding the [B*S, V] logits.  Logits are formed for whole sequences, as
    many as fit in `chunk_bytes`, in one reused buffer.  When gradients are
    wanted, each chunk's logit gradient (softmax - onehot) / count for a unit
    loss gradient is written over the chunk right after its loss and
    contracted at once into dx (bf16) and an fp32 dW accumulator, so the
    logits are read from HBM once more instead of being stored.  Backward
    scales both by the incoming loss gradient (a device scalar)."""

    @staticmethod
    def forward(ctx, x, weight, labels, clamp: bool, chunk_bytes: int, grad_wanted: bool):
        B, S, d = x.shape
        V = weight.shape[0]
        T = B * S
        dev = x.device
        x2 = _rows(x)
        lab = labels.contiguous()
        lab_flat = lab.view(-1)
        # gradients only when the caller records them (a no-grad forward, such
        # as ZeRO-3's first pass, skips the backward products)
        need_x = grad_wanted and ctx.needs_input_grad[0]
        need_w = grad_wanted and ctx.needs_input_grad[1]
        seqs = max(1, chunk_bytes // (max(S, 1) * V * x.element_size()))
        rows_per = min(T, seqs * max(S, 1))
        buf = torch.empty((rows_per, V), dtype=x.dtype, device=dev)
        lse = torch.empty((T,), dtype=torch.float32, device=dev)
        row_loss = torch.empty((T,), dtype=torch.float32, device=dev)
        # the number of scored positions (the gradient's divisor) before any chunk
        _, count = ops.ce_reduce(ops.zeros((T,), torch.float32, dev), lab, T, S, V, clamp)
        dx = dw32 = unit = None
        if need_x or need_w:
            unit = ops.fill_(torch.empty((1,), dtype=torch.float32, device=dev), 1.0)
            if need_x:
                dx = torch.empty((T, d), dtype=x.dtype, device=dev)
            if need_w:
                # written by the first chunk's product (beta 0), accumulated by later ones
                dw32 = (torch.empty((V, d), dtype=torch.float32, device=dev) if T > 0
                        else ops.zeros((V, d), torch.float32, dev))
        for r0 in range(0, T, rows_per):
            r1 = min(T, r0 + rows_per)
            lg = buf[: r1 - r0]
            ops.gemm(x2[r0:r1], weight, out=lg)
            ops.ce_fwd(lg, lab_flat[r0:r1], S, lse=lse[r0:r1], row_loss=row_loss[r0:r1])
            if unit is not None:
                ops.ce_bwd(lg, lab_flat[r0:r1], S, lse[r0:r1], unit, count, out=lg)
                if need_x:
                    ops.gemm(lg, weight, b_kmajor=False, out=dx[r0:r1])
                if need_w:
                    ops.gemm(lg, x2[r0:r1], a_kmajor=False, b_kmajor=False, out=dw32, beta=1.0 if r0 > 0 else 0.0)
        loss, _ = ops.ce_reduce(row_loss, lab, T, S, V, clamp)
        ctx.save_for_backward(dx, dw32)
        ctx.x_shape, ctx.w_dtype = x.shape, weight.dtype
        ctx.weight_ref = weight if _sink(weight) is not None else None
        return loss

    @staticmethod
    def backward(ctx, gloss):
        dx, dw32 = ctx.saved_tensors
        g = gloss.reshape(1).to(torch.float32).contiguous()
        gx = gw = None
        if dx is not None and ctx.needs_input_grad[0]:
            ops.scale_dev_(dx, g)
            gx = dx.view(ctx.x_shape)
        if dw32 is not None and ctx.needs_input_grad[1]:
            ops.scale_dev_(dw32, g)
            sink = _sink(ctx.weight_ref) if ctx.weight_ref is not None else None
            if sink is not None:
                buf, acc = sink.take(ctx.weight_ref)
                if acc:
                    ops.add_(buf.view(-1), ops.cast(dw32, ctx.w_dtype).view(-1))
                else:
                    ops.cast(dw32, ctx.w_dtype, out=buf)
            else:
                gw = ops.cast(dw32, ctx.w_dtype)
        return gx, gw, None, None, None, None


def lm_head_cross_entropy(x: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, clamp: bool,
                          chunk_bytes: int = 1 << 30) -> torch.Tensor:
    return LMHeadCEFn.apply(x, weight, labels, clamp, chunk_bytes, torch.is_grad_enabled())
