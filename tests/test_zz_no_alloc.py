"""lz_rmsnorm_bwd_noalloc: the RMSNorm backward on the library's own device
scratch (no workspace argument, no allocation) against lz_rmsnorm_bwd with a
caller workspace, through the C ABI.  The two share their kernels and their
partition of rows, so dx and dw must agree bit for bit: on two calls in a
row (the second smaller, reusing the scratch the first left behind), in bf16
and fp32, with a residual gradient and with dw accumulation.  Shapes beyond
the scratch are refused with an error before any launch.
"""
from __future__ import annotations

import pytest
import torch

from lzhip import _lib, ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _inputs(rows, cols, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g).to(dtype).to(DEV)
    w = (1.0 + 0.02 * torch.randn(cols, generator=g)).to(dtype).to(DEV)
    dy = torch.randn(rows, cols, generator=g).to(dtype).to(DEV)
    dres = torch.randn(rows, cols, generator=g).to(dtype).to(DEV)
    _, rstd = ops.rmsnorm_fwd(x, w, 1e-5)
    return x, w, dy, dres, rstd


def _with_workspace(x, w, rstd, dy, dres, dw0):
    rows, cols = x.shape
    dx = torch.empty_like(x)
    dw = dw0.clone()
    ws = ops._rmsnorm_workspace(DEV, int(_lib.load().lz_rmsnorm_bwd_workspace(rows, cols)))
    _lib.call("lz_rmsnorm_bwd", x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr(), dres.data_ptr(),
              dx.data_ptr(), dw.data_ptr(), 1, ws.data_ptr(), ws.numel() * 4, ops.dtype_code(x), rows, cols, cols,
              cols, cols, ops.stream_ptr(DEV))
    return dx, dw


def _no_alloc(x, w, rstd, dy, dres, dw0):
    rows, cols = x.shape
    dx = torch.empty_like(x)
    dw = dw0.clone()
    _lib.call("lz_rmsnorm_bwd_noalloc", x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr(), dres.data_ptr(),
              dx.data_ptr(), dw.data_ptr(), 1, ops.dtype_code(x), rows, cols, cols, cols, cols, ops.stream_ptr(DEV))
    return dx, dw


@pytest.mark.parametrize("dtype,shapes", [
    (torch.bfloat16, [(16 * 1024, 2048), (333, 768)]),
    (torch.bfloat16, [(1000, 4096), (512, 256)]),
    (torch.float32, [(512, 256), (50, 100)]),
    (torch.float16, [(4096, 2048), (333, 768)]),
])
def test_no_alloc_matches_workspace_entry(dtype, shapes):
    for i, (rows, cols) in enumerate(shapes):
        x, w, dy, dres, rstd = _inputs(rows, cols, dtype, seed=rows + cols + i)
        dw0 = torch.full((cols,), 0.25, dtype=dtype, device=DEV)
        ref_dx, ref_dw = _with_workspace(x, w, rstd, dy, dres, dw0)
        got_dx, got_dw = _no_alloc(x, w, rstd, dy, dres, dw0)
        torch.cuda.synchronize()
        assert torch.equal(got_dx, ref_dx), (rows, cols)
        assert torch.equal(got_dw, ref_dw), (rows, cols)
        # and against the math: dw - 0.25 is the column sum of dy * x * rstd
        want = (dy.double() * x.double() * rstd.double()[:, None]).sum(0)
        err = float(((got_dw.double() - 0.25) - want).norm() / want.norm())
        assert err < (1e-5 if dtype == torch.float32 else 1e-2), (rows, cols, err)


def test_no_alloc_refuses_shapes_beyond_its_scratch():
    # fp32 rows of 8192 columns take per-wave partial rows: far more than 8 MiB
    rows, cols = 4096, 8192
    x = torch.zeros(rows, cols, device=DEV)
    w = torch.ones(cols, device=DEV)
    rstd = torch.ones(rows, device=DEV)
    dx = torch.empty_like(x)
    dw = torch.empty(cols, device=DEV)
    lib = _lib.load()
    rc = lib.lz_rmsnorm_bwd_noalloc(x.data_ptr(), w.data_ptr(), rstd.data_ptr(), x.data_ptr(), None, dx.data_ptr(),
                                    dw.data_ptr(), 0, ops.dtype_code(x), rows, cols, cols, cols, cols,
                                    ops.stream_ptr(DEV))
    assert rc != 0
    assert "scratch" in _lib.last_error()
