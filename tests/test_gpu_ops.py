"""Kernel-level parity: every HIP entry point against the CPU oracle (or, for
floating-point GEMM products, a float32/float64 CPU matmul of the same op).

Tolerances:
  - integer/index/byte work (gather/scatter, transpose, embedding forward):
    bit-exact;
  - fp32 kernels (AdamW, sum of squares): 1e-5 relative;
  - RoPE in bf16 reproduces the reference's per-op rounding: bit-exact given
    the same cos/sin tables;
  - bf16 kernels: within a few bf16 ulps of the float64 oracle (stated per test).
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from lzhip import _lib, ops
from oracle import ops as R

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _seed(s):
    torch.manual_seed(s)
    return torch.Generator().manual_seed(s)


def _rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _grad_err(dq: torch.Tensor, ref: torch.Tensor, dv_ref: torch.Tensor) -> float:
    """Error of a query or key gradient relative to the larger of its own
    norm and dV's: with one key per query (S = 1) the exact dQ and dK are
    zero and the kernels' values are the rounding noise of delta - dO.V,
    which only a scale from elsewhere can judge."""
    d = (dq.double().cpu() - ref.double().cpu()).norm()
    return float(d / max(ref.double().norm(), dv_ref.double().norm(), torch.tensor(1e-30, dtype=torch.float64)))


def test_library_is_the_in_tree_build():
    lib = _lib.load()
    assert lib.lz_version() == 1
    assert torch.cuda.is_available()
    assert lib.lz_device_cus() > 0


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------
@pytest.mark.parametrize(
    "M,N,K",
    [(64, 64, 64), (256, 256, 128), (300, 200, 72), (1000, 520, 136), (2048, 2048, 2048), (4096, 1536, 768)],
)
def test_gemm_nt_bf16_and_fp32_out(M, N, K):
    g = _seed(M + N + K)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    b = torch.randn(N, K, generator=g).to(torch.bfloat16)
    ref = a.double() @ b.double().t()
    c32 = ops.gemm_nt(a.to(DEV), b.to(DEV), out_dtype=torch.float32).cpu()
    # fp32 accumulation of exact bf16 products: error ~ sqrt(K) * eps32 * |terms|
    tol = 1e-5 * math.sqrt(K) * float(a.float().abs().max() * b.float().abs().max()) * 4
    assert float((c32.double() - ref).abs().max()) <= tol
    c16 = ops.gemm_nt(a.to(DEV), b.to(DEV)).cpu()
    assert c16.dtype == torch.bfloat16
    # one bf16 rounding of the fp32 result
    assert torch.allclose(c16.double(), c32.double(), rtol=2 ** -8, atol=1e-6)


def test_gemm_residual_alpha_beta():
    g = _seed(7)
    M, N, K = 384, 256, 192
    a = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    b = torch.randn(N, K, generator=g).to(torch.bfloat16).to(DEV)
    r = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    c0 = torch.randn(M, N, generator=g).to(DEV)
    ab = a.double().cpu() @ b.double().cpu().t()
    out = ops.gemm_nt(a, b, residual=r).cpu().double()
    # bf16 output: the product is rounded to bf16, then the sum with the
    # residual is rounded again (the reference's nn.Linear output + x in bf16)
    want = ab + r.double().cpu()
    assert bool(((out - want).abs() <= 2 ** -8 * (ab.abs() + want.abs()) + 1e-6).all())
    prod16 = ops.gemm_nt(a, b).cpu()  # the same product alone, rounded once
    two_step = (prod16.float() + r.float().cpu()).to(torch.bfloat16).double()
    assert torch.equal(out, two_step)
    acc = c0.clone()
    ops.gemm_nt(a, b, out=acc, alpha=0.5, beta=1.0)
    assert torch.allclose(acc.cpu().double(), 0.5 * ab + c0.double().cpu(), rtol=1e-5, atol=1e-3)


def test_gemm_strided_views_and_padding_helpers():
    g = _seed(11)
    M, N, K = 200, 96, 40  # K not a multiple of 64
    big = torch.randn(M, K + 24, generator=g).to(torch.bfloat16).to(DEV)
    a = big[:, 8 : 8 + K]  # row stride K+24, offset 8 elements (16 B)
    b = torch.randn(N, K, generator=g).to(torch.bfloat16).to(DEV)
    c = ops.gemm_nt(a, b, out_dtype=torch.float32).cpu().double()
    ref = a.cpu().double() @ b.cpu().double().t()
    assert torch.allclose(c, ref, rtol=1e-5, atol=1e-3)
    # odd reduction length through the padding helpers
    x = torch.randn(37, 13, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randn(29, 13, generator=g).to(torch.bfloat16).to(DEV)
    y = ops.gemm_nt(ops.nt_operand(x), ops.nt_operand(w), out_dtype=torch.float32).cpu().double()
    assert torch.allclose(y, x.cpu().double() @ w.cpu().double().t(), rtol=1e-5, atol=1e-3)
    xt = ops.transpose_padded(x)
    assert xt.shape == (13, 40)
    assert torch.equal(xt[:, :37].cpu(), x.cpu().t())
    assert torch.count_nonzero(xt[:, 37:]) == 0


def _layout_operand(t, kmajor):
    """t is the logical [rows, K] operand; returns the stored tensor."""
    return t.to(DEV) if kmajor else t.t().contiguous().to(DEV)


@pytest.mark.parametrize("a_kmajor,b_kmajor", [(True, True), (True, False), (False, True), (False, False)])
@pytest.mark.parametrize(
    "M,N,K",
    [(64, 64, 64), (520, 264, 200), (1000, 1000, 520), (1000, 1000, 512), (2048, 1024, 1536),
     # one full round of 256x256 tiles (the 256x192 tiling would take two)
     (4096, 4096, 128),
     # few output tiles, long K: split along K (K not a multiple of 64 in the last case)
     (512, 384, 8192), (1024, 768, 8200)],
)
def test_gemm_layouts(M, N, K, a_kmajor, b_kmajor):
    g = _seed(M * 3 + N + K + 2 * a_kmajor + b_kmajor)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    b = torch.randn(N, K, generator=g).to(torch.bfloat16)
    ref = a.double() @ b.double().t()
    A, B = _layout_operand(a, a_kmajor), _layout_operand(b, b_kmajor)
    c32 = ops.gemm(A, B, a_kmajor, b_kmajor, out_dtype=torch.float32).cpu()
    tol = 1e-5 * math.sqrt(K) * float(a.float().abs().max() * b.float().abs().max()) * 4
    assert float((c32.double() - ref).abs().max()) <= tol
    c16 = ops.gemm(A, B, a_kmajor, b_kmajor).cpu()
    assert torch.allclose(c16.double(), c32.double(), rtol=2 ** -8, atol=1e-6)
    # accumulation into an existing fp32 C and a bf16 residual, split or not
    c0 = torch.randn(M, N, generator=g)
    r = torch.randn(M, N, generator=g).to(torch.bfloat16)
    acc = c0.to(DEV)
    ops.gemm(A, B, a_kmajor, b_kmajor, out=acc, alpha=0.5, beta=1.0, residual=r.to(DEV))
    want = 0.5 * ref + c0.double() + r.double()
    assert float((acc.cpu().double() - want).abs().max()) <= 0.5 * tol + 1e-5 * float(want.abs().max())


@pytest.mark.parametrize("b_kmajor", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "M,N,K",
    [(16384, 768, 768),  # 64 x 4 interior tiles: one full round on 256 CUs
     (4096, 3072, 768),  # 16 x 16 interior tiles
     (4000, 2904, 1024)],  # edge tiles in M (last 160 rows) and N (last 24 columns)
)
def test_gemm_n192_tiles(M, N, K, dtype, b_kmajor):
    """The 256x192 direct-to-LDS tiles (plan code 6) on every epilogue path:
    fp32 output, bf16 / fp16 output rounded once, with a residual (rounded
    twice, as the reference's Linear output + x), and alpha / beta
    accumulation into fp32 and 16-bit outputs."""
    lib = _lib.load()
    assert int(lib.lz_gemm_plan(M, N, K, 1, int(b_kmajor))) == 6 * 64 + 1
    g = _seed(M + 7 * N + K + b_kmajor)
    a = torch.randn(M, K, generator=g).to(dtype)
    b = torch.randn(N, K, generator=g).to(dtype)
    ref = a.double() @ b.double().t()
    A, B = a.to(DEV), _layout_operand(b, b_kmajor)
    tol = 1e-5 * math.sqrt(K) * float(a.float().abs().max() * b.float().abs().max()) * 4
    c32 = ops.gemm(A, B, True, b_kmajor, out_dtype=torch.float32).cpu()
    assert float((c32.double() - ref).abs().max()) <= tol
    eps = 2 ** -8 if dtype == torch.bfloat16 else 2 ** -11
    c16 = ops.gemm(A, B, True, b_kmajor).cpu()
    assert c16.dtype == dtype
    assert torch.equal(c16, c32.to(dtype))  # the fp32 sum rounded once
    r = torch.randn(M, N, generator=g).to(dtype)
    cr = ops.gemm(A, B, True, b_kmajor, residual=r.to(DEV)).cpu()
    assert torch.equal(cr, (c16.float() + r.float()).to(dtype))
    c0 = torch.randn(M, N, generator=g)
    acc = c0.to(DEV)
    ops.gemm(A, B, True, b_kmajor, out=acc, alpha=0.5, beta=1.0)
    assert float((acc.cpu().double() - (0.5 * ref + c0.double())).abs().max()) <= 0.5 * tol + 1e-5 * float(c0.abs().max())
    h0 = torch.randn(M, N, generator=g).to(dtype)
    acc16 = h0.to(DEV)
    ops.gemm(A, B, True, b_kmajor, out=acc16, alpha=0.5, beta=1.0)
    want = 0.5 * ref + h0.double()
    assert bool(((acc16.cpu().double() - want).abs() <= eps * want.abs() + 0.5 * tol + 1e-6).all())


def test_gemm_long_k_over_a_wide_mn_major_operand_splits():
    """A K range whose M-major rows span more than 2^30 elements (8192 x
    262144) is split so that each split's buffer offsets fit; the product
    matches a float32 one."""
    lib = _lib.load()
    M, N, K = 8192, 512, 262144
    code = int(lib.lz_gemm_plan(M, N, K, 0, 0))
    assert code // 64 == 5 and code % 64 >= 3
    g = torch.Generator(device=DEV).manual_seed(3)
    a = torch.randn(K, M, device=DEV, generator=g).to(torch.bfloat16)
    b = torch.randn(K, N, device=DEV, generator=g).to(torch.bfloat16)
    c = ops.gemm(a, b, False, False, out_dtype=torch.float32)
    ref = torch.matmul(a.float().t(), b.float())
    del a, b
    assert float((c - ref).abs().max()) <= 1e-5 * math.sqrt(K) * 4.0 * 25.0


def test_gemm_split_k_workspace_and_determinism():
    lib = ops._lib.load()
    M, N, K = 512, 384, 8192
    assert lib.lz_gemm_workspace(M, N, K, 0, 0) > 0  # the plan splits this shape
    assert lib.lz_gemm_workspace(16384, 4096, 2048, 1, 1) == 0
    g = _seed(5)
    a = torch.randn(K, M, generator=g).to(torch.bfloat16).to(DEV)
    b = torch.randn(K, N, generator=g).to(torch.bfloat16).to(DEV)
    c1 = ops.gemm(a, b, False, False, out_dtype=torch.float32)
    c2 = ops.gemm(a, b, False, False, out_dtype=torch.float32)
    assert torch.equal(c1, c2)
    # without a workspace the same product runs unsplit (same values up to summation order)
    c3 = torch.empty_like(c1)
    ops._lib.call("lz_gemm", a.data_ptr(), M, 0, b.data_ptr(), N, 0, 1, c3.data_ptr(), N, 0, 0, 0, M, N, K, 1.0, 0.0,
                  0, 0, ops.stream_ptr(a.device))
    assert torch.allclose(c1, c3, rtol=1e-4, atol=1e-3)


def test_gemm_and_attention_repeat_bit_identically():
    """Every kernel that stages operands with direct-to-LDS loads must wait for
    them before the barrier that publishes a stage; a missing wait reads a
    stage that is still landing, which shows up as run-to-run differences.
    Each product below (input gradient, split weight gradient, forward, the
    attention forward and backward) is repeated and must match bit for bit."""
    g = _seed(21)
    dy = torch.randn(2048, 4096, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.randn(4096, 2048, generator=g).to(torch.bfloat16).to(DEV)
    x = torch.randn(2048, 2048, generator=g).to(torch.bfloat16).to(DEV)
    runs = {
        "dgrad": lambda: ops.gemm(dy, w, True, False),
        "wgrad": lambda: ops.gemm(dy, x, False, False, out_dtype=torch.float32),
        "fwd": lambda: ops.gemm(x, w),
    }
    for name, fn in runs.items():
        first = fn().cpu()
        for _ in range(8):
            assert torch.equal(fn().cpu(), first), name
    B, S, H, KV, hd = 2, 1024, 8, 4, 128
    ld = (H + 2 * KV) * hd
    d = torch.randn(B * S, ld, generator=g).to(torch.bfloat16).to(DEV)
    q2, k2, v2 = d[:, : H * hd], d[:, H * hd : (H + KV) * hd], d[:, (H + KV) * hd :]
    do = torch.randn(B * S, H * hd, generator=g).to(torch.bfloat16).to(DEV)
    o0, lse0 = ops.attn_fwd(q2, k2, v2, B, S, H, KV, hd, hd**-0.5, None)
    grads0 = None
    for _ in range(6):
        o, lse = ops.attn_fwd(q2, k2, v2, B, S, H, KV, hd, hd**-0.5, None)
        assert torch.equal(o, o0) and torch.equal(lse, lse0)
        dqkv = torch.zeros_like(d)
        ops.attn_bwd(q2, k2, v2, o, do, lse, B, S, H, KV, hd, hd**-0.5, dqkv[:, : H * hd],
                     dqkv[:, H * hd : (H + KV) * hd], dqkv[:, (H + KV) * hd :])
        if grads0 is None:
            grads0 = dqkv.cpu()
        assert torch.equal(dqkv.cpu(), grads0)


def test_gemm_unaligned_mn_major_operands_fall_back():
    g = _seed(13)
    M, N, K = 37, 29, 45
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    b = torch.randn(N, K, generator=g).to(torch.bfloat16)
    ref = a.double() @ b.double().t()
    for ak in (True, False):
        for bk in (True, False):
            c = ops.gemm(_layout_operand(a, ak), _layout_operand(b, bk), ak, bk, out_dtype=torch.float32).cpu()
            assert torch.allclose(c.double(), ref, rtol=1e-5, atol=1e-3), (ak, bk)


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols,dtype", [(64, 64, torch.float32), (333, 768, torch.bfloat16),
                                             (16 * 1024, 2048, torch.bfloat16), (50, 100, torch.float32),
                                             (128, 4096, torch.bfloat16)])
def test_rmsnorm_fwd_bwd(rows, cols, dtype):
    g = _seed(rows + cols)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    w = (1.0 + 0.02 * torch.randn(cols, generator=g)).to(dtype)
    dy = torch.randn(rows, cols, generator=g).to(dtype)
    y, rstd = ops.rmsnorm_fwd(x.to(DEV), w.to(DEV), 1e-5)
    # reference: fp32 statistics, (x*r)*w in fp32, one rounding to the dtype
    xd, wd = x.double().requires_grad_(True), w.double().requires_grad_(True)
    yref = R.rmsnorm(xd, wd, 1e-5)
    if dtype == torch.float32:
        assert _rel_err(y, yref) < 1e-6
    else:
        assert float((y.cpu().double() - yref.detach()).abs().max()) <= 2 ** -8 * float(yref.abs().max())
    rref = torch.rsqrt(x.double().pow(2).mean(-1) + 1e-5)
    assert _rel_err(rstd, rref) < 1e-6
    dx, dw = ops.rmsnorm_bwd(x.to(DEV), w.to(DEV), rstd, dy.to(DEV))
    yref.backward(dy.double())
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert _rel_err(dx, xd.grad) < tol
    assert _rel_err(dw, wd.grad) < tol


@pytest.mark.parametrize("rows,cols", [(512, 256), (333, 768), (16 * 1024, 2048), (1000, 4096)])
def test_rmsnorm_bwd_repeats_and_accumulates(rows, cols):
    """The bf16 backward's dw (per-workgroup fp32 partial rows, then a
    fixed-order column sum) repeats bit for bit with a reused workspace, and
    dw_accumulate adds the new dw to the old one."""
    g = _seed(rows * 3 + cols)
    x = torch.randn(rows, cols, generator=g).to(torch.bfloat16).to(DEV)
    w = (1.0 + 0.02 * torch.randn(cols, generator=g)).to(torch.bfloat16).to(DEV)
    dy = torch.randn(rows, cols, generator=g).to(torch.bfloat16).to(DEV)
    _, rstd = ops.rmsnorm_fwd(x, w, 1e-5)
    runs = [ops.rmsnorm_bwd(x, w, rstd, dy) for _ in range(3)]
    for dx, dw in runs[1:]:
        assert torch.equal(dx, runs[0][0]) and torch.equal(dw, runs[0][1])
    ref = (dy.double() * x.double() * rstd.double()[:, None]).sum(0)
    assert _rel_err(runs[0][1], ref) < 1e-2
    base = torch.full((cols,), 0.5, dtype=torch.bfloat16, device=DEV)
    acc = base.clone()
    dx = torch.empty_like(x)
    lib = _lib.load()
    ws = ops._rmsnorm_workspace(DEV, int(lib.lz_rmsnorm_bwd_workspace(rows, cols)))
    _lib.call("lz_rmsnorm_bwd", x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr(), None, dx.data_ptr(),
              acc.data_ptr(), 1, ws.data_ptr(), ws.numel() * 4, 1, rows, cols, cols, cols, cols,
              ops.stream_ptr(DEV))
    # the fp32 sum plus the old bf16 value, rounded once: within a rounding of
    # the result and of dw from adding the rounded dw
    dw0 = runs[0][1].double()
    assert torch.allclose(acc.double(), base.double() + dw0, rtol=2 ** -8, atol=2 ** -8 * float(dw0.abs().max()))


# ---------------------------------------------------------------------------
# RoPE: bit-exact against the reference's bf16 op sequence given equal tables
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("S,hd,theta", [(1024, 128, 10000.0), (128, 32, 10000.0), (16, 16, 500000.0)])
def test_rope_matches_reference_ops(dtype, S, hd, theta):
    g = _seed(S + hd)
    B, nh = 2, 3
    cos, sin = R.rope_tables(S, hd, theta, dtype=dtype)
    # the kernel's table, from the same fp32 inv_freq buffer, agrees with the
    # reference table to one rounding of cos/sin; with a bf16 buffer (the
    # reference after Module.to(bfloat16)) positions and angles are bf16 too
    for angle_dtype in (torch.float32, torch.bfloat16):
        rc, rs = R.rope_tables(S, hd, theta, dtype=dtype, angle_dtype=angle_dtype)
        inv = R.inv_freq(hd, theta).to(angle_dtype).to(DEV)
        kc, ks = ops.rope_table(S, hd, inv, dtype)
        ulp = 2 ** -8 if (dtype == torch.bfloat16 or angle_dtype == torch.bfloat16) else 2 ** -23
        assert float((kc.cpu().double() - rc.double()).abs().max()) <= ulp
        assert float((ks.cpu().double() - rs.double()).abs().max()) <= ulp
        if dtype == torch.bfloat16:
            # after rounding to bf16 the device and host cos/sin agree almost everywhere
            assert float((kc.cpu() == rc).double().mean()) > 0.99
    x = torch.randn(B, S, nh, hd, generator=g).to(dtype)
    xg = x.clone().to(DEV)
    ops.rope_(xg.view(B * S, nh * hd), S, nh, hd, cos.to(DEV), sin.to(DEV))
    ref = R.apply_rope(x.transpose(1, 2), cos, sin).transpose(1, 2)
    assert torch.equal(xg.cpu(), ref)
    # backward = autograd of the same ops in the same dtype
    xr = x.transpose(1, 2).clone().requires_grad_(True)
    dy = torch.randn(B, nh, S, hd, generator=g).to(dtype)
    R.apply_rope(xr, cos, sin).backward(dy)
    dg = dy.transpose(1, 2).contiguous().to(DEV)
    ops.rope_(dg.view(B * S, nh * hd), S, nh, hd, cos.to(DEV), sin.to(DEV), backward=True)
    assert torch.equal(dg.cpu(), xr.grad.transpose(1, 2))


# ---------------------------------------------------------------------------
# SwiGLU pointwise
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("rows,cols,dtype", [(1024, 5632, torch.bfloat16), (77, 130, torch.bfloat16),
                                             (64, 96, torch.float32)])
def test_swiglu_fwd_bwd(rows, cols, dtype):
    g = _seed(rows * 3 + cols)
    gu = torch.randn(rows, 2 * cols, generator=g).to(dtype)
    dh = torch.randn(rows, cols, generator=g).to(dtype)
    gd = gu.to(DEV)
    h = ops.swiglu_fwd(gd[:, :cols], gd[:, cols:])
    gate, up = gu[:, :cols], gu[:, cols:]
    # reference op sequence in the activation dtype: silu rounded, product rounded
    href = F.silu(gate) * up
    diff = (h.cpu().double() - href.double()).abs()
    assert float(diff.max()) <= 2 ** -7 * float(href.double().abs().max() + 1)
    if dtype == torch.bfloat16:
        assert float((diff == 0).double().mean()) > 0.99
    dgu = torch.empty_like(gd)
    ops.swiglu_bwd(gd[:, :cols], gd[:, cols:], dh.to(DEV), dgu[:, :cols], dgu[:, cols:])
    gr = gate.double().requires_grad_(True)
    ur = up.double().requires_grad_(True)
    R.swiglu(gr, ur).backward(dh.double())
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert _rel_err(dgu[:, :cols], gr.grad) < tol
    assert _rel_err(dgu[:, cols:], ur.grad) < tol


@pytest.mark.parametrize("M,F_,K", [(256, 128, 64), (512, 384, 192), (768, 256, 2048)])
def test_gemm_swiglu_fused_matches_unfused(M, F_, K):
    """The fused gate|up GEMM + SwiGLU equals the unfused pair bit for bit
    (gate|up and h), with and without the gate|up output, and h stays within
    bf16 rounding of the float64 oracle on the same bf16 operands."""
    g = _seed(M + F_ + K)
    x = (0.5 * torch.randn(M, K, generator=g)).to(torch.bfloat16)
    w = (0.05 * torch.randn(2 * F_, K, generator=g)).to(torch.bfloat16)
    xd, wd = x.to(DEV), w.to(DEV)
    gu_ref = ops.gemm(xd, wd)
    h_ref = ops.swiglu_fwd(gu_ref[:, :F_], gu_ref[:, F_:])
    gu = torch.full((M, 2 * F_), 7.0, dtype=torch.bfloat16, device=DEV)
    h = ops.gemm_swiglu(xd, wd, gu=gu)
    assert torch.equal(gu.cpu(), gu_ref.cpu())
    assert torch.equal(h.cpu(), h_ref.cpu())
    h2 = ops.gemm_swiglu(xd, wd)
    assert torch.equal(h2.cpu(), h_ref.cpu())
    prod = x.double() @ w.double().t()
    want = R.swiglu(prod[:, :F_], prod[:, F_:])
    diff = (h.cpu().double() - want).abs()
    assert float(diff.max()) <= 2 ** -6 * float(want.abs().max() + 1)


@pytest.mark.parametrize("M,F_,K,pad", [(256, 256, 64, 0), (512, 768, 192, 8), (768, 512, 960, 0)])
def test_gemm_swiglu_bwd_fused_matches_unfused(M, F_, K, pad):
    """The down projection's input gradient with SwiGLU's backward in its
    epilogue equals gemm (W_down read N-major) followed by the SwiGLU backward
    kernel bit for bit, also on padded row strides, and the gradients stay
    within bf16 rounding of float64 autograd on the same bf16 operands.  (The
    fused kernel never splits K; K stays below 1024 here so that the unfused
    product is not split either and sums K in the same order.)"""
    g = _seed(M + F_ + K + pad)
    dy = torch.randn(M, K, generator=g).to(torch.bfloat16)
    wd = (0.05 * torch.randn(K, F_, generator=g)).to(torch.bfloat16)
    gu = torch.randn(M, 2 * F_ + pad, generator=g).to(torch.bfloat16)
    dyd, wdd, gud = dy.to(DEV), wd.to(DEV), gu.to(DEV)[:, : 2 * F_]
    dm = ops.gemm(dyd, wdd, b_kmajor=False)
    ref = torch.empty((M, 2 * F_), dtype=torch.bfloat16, device=DEV)
    ops.swiglu_bwd(gud[:, :F_], gud[:, F_:], dm, ref[:, :F_], ref[:, F_:])
    assert ops.swiglu_bwd_fusable(dyd, wdd, gud)
    out = torch.full((M, 2 * F_ + pad), 7.0, dtype=torch.bfloat16, device=DEV)
    got = ops.gemm_swiglu_bwd(dyd, wdd, gud, dgu=out[:, : 2 * F_])
    assert torch.equal(got.cpu(), ref.cpu())
    if pad:
        assert bool((out[:, 2 * F_:] == 7.0).all())
    assert torch.equal(ops.gemm_swiglu_bwd(dyd, wdd, gud).cpu(), ref.cpu())
    gate = gu[:, :F_].double().requires_grad_(True)
    up = gu[:, F_ : 2 * F_].double().requires_grad_(True)
    R.swiglu(gate, up).backward(dy.double() @ wd.double())
    assert _rel_err(got[:, :F_], gate.grad) < 1e-2
    assert _rel_err(got[:, F_:], up.grad) < 1e-2
    with pytest.raises(ValueError):
        ops.gemm_swiglu_bwd(dyd[:128], wdd, gud[:128])  # M not a multiple of 256


@pytest.mark.parametrize("M,N,nrope,K,S,hd", [(256, 512, 256, 64, 256, 128), (512, 1024, 768, 192, 128, 128),
                                               (768, 512, 512, 2048, 384, 128),
                                               # head dim 64: the 125M layout (12 q + 4 k heads rotated, 4 v heads),
                                               # and sequences shorter than a wave's 128 rows
                                               (2048, 1280, 1024, 768, 1024, 64), (768, 1280, 1024, 768, 96, 64),
                                               (256, 512, 256, 128, 64, 64)])
def test_gemm_rope_fused_matches_unfused(M, N, nrope, K, S, hd):
    """The fused QKV GEMM + RoPE equals gemm followed by the RoPE kernel bit
    for bit (rotated q/k columns and the plain v columns), and the rotation
    matches the float64 oracle on the same bf16 product within bf16
    rounding."""
    g = _seed(M + N + K + hd)
    x = (0.5 * torch.randn(M, K, generator=g)).to(torch.bfloat16)
    w = (0.05 * torch.randn(N, K, generator=g)).to(torch.bfloat16)
    xd, wd = x.to(DEV), w.to(DEV)
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    cos, sin = ops.rope_table(S, hd, inv.to(DEV), torch.bfloat16)
    ref = ops.gemm(xd, wd)
    ops.rope_(ref, S, nrope // hd, hd, cos, sin)
    got = ops.gemm_rope(xd, wd, cos, sin, S, nrope, hd)
    assert torch.equal(got.cpu(), ref.cpu())
    prod = (x.double() @ w.double().t()).view(M // S, S, N)
    heads = prod[:, :, :nrope].reshape(M // S, S, nrope // hd, hd).transpose(1, 2)
    c64 = cos.cpu().double()[None, None]
    s64 = sin.cpu().double()[None, None]
    want = heads * c64 + torch.cat([-heads[..., hd // 2 :], heads[..., : hd // 2]], -1) * s64
    got_h = got.cpu().double().view(M // S, S, N)[:, :, :nrope].reshape(M // S, S, nrope // hd, hd).transpose(1, 2)
    assert float((got_h - want).abs().max()) <= 2 ** -6 * float(want.abs().max() + 1)


def test_gemm_swiglu_rejects_unsupported_shapes():
    x = torch.zeros(300, 64, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(256, 64, dtype=torch.bfloat16, device=DEV)
    assert not ops.swiglu_fusable(x, w)
    with pytest.raises(ValueError):
        ops.gemm_swiglu(x, w)
    with pytest.raises(_lib.HipLibraryError):
        _lib.call("lz_gemm_swiglu", x.data_ptr(), 64, w.data_ptr(), 64, 0, 0, x.data_ptr(), 128, 300, 128, 64, 0)


# ---------------------------------------------------------------------------
# Attention
# ---------------------------------------------------------------------------
@pytest.mark.parametrize(
    "B,S,H,KV,hd",
    [(2, 128, 4, 2, 64), (1, 256, 4, 1, 128), (2, 200, 4, 4, 64), (1, 130, 2, 2, 128), (2, 64, 8, 4, 32),
     (2, 16, 4, 2, 16), (1, 1024, 16, 8, 128), (3, 200, 8, 2, 32), (2, 128, 8, 4, 32), (1, 1, 2, 1, 16),
     (1, 70, 2, 2, 16), (4, 1024, 8, 8, 32)],
)
def test_attention_fwd_bwd(B, S, H, KV, hd):
    g = _seed(B * S + H * hd)
    ld = (H + 2 * KV) * hd
    qkv = torch.randn(B * S, ld, generator=g).to(torch.bfloat16)
    d = qkv.to(DEV)
    q2, k2, v2 = d[:, : H * hd], d[:, H * hd : (H + KV) * hd], d[:, (H + KV) * hd :]
    scale = hd**-0.5
    path = ops.attn_path(torch.bfloat16, S, hd, ld, ld, ld, H * hd)
    assert path == (2 if hd in (64, 128) and S % 64 == 0 else 1 if hd in (64, 128) else 0)
    mfma = path == 1  # the transposed-operand path needs V^T, Q^T, K^T, dO^T
    vt = ops.transpose_heads(d, B, S, KV, hd, col0=(H + KV) * hd) if mfma else None
    o, lse = ops.attn_fwd(q2, k2, v2, B, S, H, KV, hd, scale, vt)

    def heads(t, n):
        return t.double().view(B, S, n, hd).transpose(1, 2).requires_grad_(True)

    qr, kr, vr = heads(qkv[:, : H * hd], H), heads(qkv[:, H * hd : (H + KV) * hd], KV), heads(qkv[:, (H + KV) * hd :], KV)
    oref = R.causal_gqa_attention(qr, kr, vr, scale)
    o4 = o.cpu().double().view(B, S, H, hd).transpose(1, 2)
    assert _rel_err(o4, oref) < 1e-2
    kk = kr.repeat_interleave(H // KV, dim=1)
    sc = (qr @ kk.transpose(-1, -2)) * scale
    sc = sc.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    lse_ref = torch.logsumexp(sc, dim=-1)
    assert float((lse.cpu().double() - lse_ref.detach()).abs().max()) < 2e-2

    do = torch.randn(B * S, H * hd, generator=g).to(torch.bfloat16)
    dqkv = torch.zeros_like(d)
    qt = kt = dot = None
    if mfma:
        qt = ops.transpose_heads(d, B, S, H, hd, col0=0)
        kt = ops.transpose_heads(d, B, S, KV, hd, col0=H * hd)
        dot = ops.transpose_heads(do.to(DEV), B, S, H, hd, col0=0)
    ops.attn_bwd(q2, k2, v2, o, do.to(DEV), lse, B, S, H, KV, hd, scale,
                 dqkv[:, : H * hd], dqkv[:, H * hd : (H + KV) * hd], dqkv[:, (H + KV) * hd :], qt=qt, kt=kt, dot=dot)
    oref.backward(do.double().view(B, S, H, hd).transpose(1, 2))
    dq = dqkv[:, : H * hd].cpu().double().view(B, S, H, hd).transpose(1, 2)
    dk = dqkv[:, H * hd : (H + KV) * hd].cpu().double().view(B, S, KV, hd).transpose(1, 2)
    dv = dqkv[:, (H + KV) * hd :].cpu().double().view(B, S, KV, hd).transpose(1, 2)
    assert _grad_err(dq, qr.grad, vr.grad) < 2e-2
    assert _grad_err(dk, kr.grad, vr.grad) < 2e-2
    assert _rel_err(dv, vr.grad) < 2e-2


def _attn_masks(kind, B, H, S, g):
    """Masks of the shapes a caller of the reference's attention passes."""
    if kind == "bool_padding":  # [B, 1, S, S]: causal, and each batch's last keys padded away
        causal = ~torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
        keep = torch.ones(B, 1, S, S, dtype=torch.bool)
        for b in range(B):
            keep[b, :, :, S - 3 * (b + 1):] = False
        m = causal & keep
        m[..., 0] = True  # every query keeps at least one key
        return m
    if kind == "float_2d":  # [S, S] additive: -inf above the diagonal, random biases below
        m = torch.randn(S, S, generator=g)
        return m.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    if kind == "bf16_full":  # [B, H, S, S] additive, no -inf (every key of every query)
        return torch.randn(B, H, S, S, generator=g).to(torch.bfloat16)
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["bool_padding", "float_2d", "bf16_full"])
@pytest.mark.parametrize("B,S,H,KV,hd,dtype", [(2, 64, 4, 2, 64, torch.bfloat16), (1, 48, 4, 4, 32, torch.float32),
                                               (2, 40, 6, 2, 128, torch.bfloat16)])
def test_attention_with_explicit_mask_vs_oracle(kind, B, S, H, KV, hd, dtype):
    """model/llama.py:109-117: SDPA with attn_mask (no causal mask): forward
    and gradients against the oracle's restatement in float64."""
    g = _seed(B * S + hd + len(kind))
    ld = (H + 2 * KV) * hd
    qkv = torch.randn(B * S, ld, generator=g).to(dtype)
    mask = _attn_masks(kind, B, H, S, g)
    d = qkv.to(DEV)
    q2, k2, v2 = d[:, : H * hd], d[:, H * hd : (H + KV) * hd], d[:, (H + KV) * hd :]
    scale = hd**-0.5
    o, lse = ops.attn_fwd_general(q2, k2, v2, B, S, H, KV, hd, scale, mask.to(DEV))

    def heads(t, n):
        return t.double().view(B, S, n, hd).transpose(1, 2).requires_grad_(True)

    qr, kr, vr = heads(qkv[:, : H * hd], H), heads(qkv[:, H * hd : (H + KV) * hd], KV), heads(qkv[:, (H + KV) * hd :], KV)
    mref = mask if mask.dtype == torch.bool else mask.double()
    oref = R.causal_gqa_attention(qr, kr, vr, scale, attn_mask=mref)
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-5
    assert _rel_err(o.cpu().double().view(B, S, H, hd).transpose(1, 2), oref) < tol
    do = torch.randn(B * S, H * hd, generator=g).to(dtype)
    dqkv = torch.zeros_like(d)
    ops.attn_bwd_general(q2, k2, v2, o, do.to(DEV), lse, B, S, H, KV, hd, scale, dqkv[:, : H * hd],
                        dqkv[:, H * hd : (H + KV) * hd], dqkv[:, (H + KV) * hd :], mask.to(DEV))
    oref.backward(do.double().view(B, S, H, hd).transpose(1, 2))
    dq = dqkv[:, : H * hd].cpu().double().view(B, S, H, hd).transpose(1, 2)
    dk = dqkv[:, H * hd : (H + KV) * hd].cpu().double().view(B, S, KV, hd).transpose(1, 2)
    dv = dqkv[:, (H + KV) * hd :].cpu().double().view(B, S, KV, hd).transpose(1, 2)
    gtol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert _grad_err(dq, qr.grad, vr.grad) < gtol
    assert _grad_err(dk, kr.grad, vr.grad) < gtol
    assert _rel_err(dv, vr.grad) < gtol


def test_attention_explicit_causal_mask_equals_causal():
    """An explicit causal bool mask reproduces the causal kernels (fp32: to
    rounding), and a mask that does not broadcast is refused."""
    g = _seed(77)
    B, S, H, KV, hd = 2, 96, 4, 2, 64
    d = torch.randn(B * S, (H + 2 * KV) * hd, generator=g).to(DEV)
    q2, k2, v2 = d[:, : H * hd], d[:, H * hd : (H + KV) * hd], d[:, (H + KV) * hd :]
    causal = ~torch.triu(torch.ones(S, S, dtype=torch.bool, device=DEV), 1)
    o1, l1 = ops.attn_fwd(q2, k2, v2, B, S, H, KV, hd, 0.125, None)
    o2, l2 = ops.attn_fwd_general(q2, k2, v2, B, S, H, KV, hd, 0.125, causal)
    assert _rel_err(o2, o1) < 1e-6 and _rel_err(l2, l1) < 1e-6
    with pytest.raises(ValueError):
        ops.attn_fwd_general(q2, k2, v2, B, S, H, KV, hd, 0.125, causal[:5])
    with pytest.raises(TypeError):
        ops.attn_fwd_general(q2, k2, v2, B, S, H, KV, hd, 0.125, causal.to(torch.int32))


@pytest.mark.parametrize("n", [1, 1000, 1 << 20, 1000003])
@pytest.mark.parametrize("p", [0.0, 0.1, 0.5, 0.97, 1.0])
def test_dropout_mask_matches_oracle_stream(n, p):
    """The GPU keep mask is the oracle's SplitMix64 stream, bit for bit."""
    key = ops.dropout_key(1234 + n, 8)
    keep = ops.dropout_mask(n, p, key, DEV).cpu().numpy().astype(bool)
    assert (keep == R.dropout_keep(key, n, p)).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,offset", [(4096 * 8, 0), (4096 * 8 + 5, 0), (777, 1), (1 << 16, 3)])
@pytest.mark.parametrize("p", [0.1, 0.5, 1.0])
def test_dropout_op_vs_oracle(dtype, n, offset, p):
    """y = x * keep / (1 - p) exactly (scale computed in fp32, product
    rounded once), on the 16-byte and element-wise paths (a view that starts
    `offset` elements into its buffer is not 16-byte aligned), in place and
    out of place; the same call on y's gradient applies the same mask."""
    g = _seed(n + offset)
    base = torch.randn(n + offset, generator=g).to(dtype)
    x = base.to(DEV)[offset:]
    key = ops.dropout_key(77, n)
    keep = torch.from_numpy(R.dropout_keep(key, n, p))
    scale = (1.0 / (1.0 - torch.tensor(p, dtype=torch.float32))) if p < 1.0 else torch.tensor(0.0)
    want = (base[offset:].float() * keep.float() * scale).to(dtype)
    y = ops.dropout_(x, p, key, out=torch.empty_like(x))
    assert torch.equal(y.cpu(), want)
    xi = x.clone()
    ops.dropout_(xi, p, key)
    assert torch.equal(xi.cpu(), want)
    assert torch.equal(x.cpu(), base[offset:])  # out-of-place left x alone


def test_dropout_fn_backward_and_seed_draws():
    """DropoutFn: the backward applies the forward's mask and scale; seeds
    come from the device generator (torch.manual_seed replays them, each call
    draws a new one) and the kept fraction is 1 - p."""
    from lzhip import functional as LF

    x = torch.randn(64, 1024, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    torch.manual_seed(3)
    y = LF.dropout(x, 0.25)
    y2 = LF.dropout(x, 0.25)
    torch.manual_seed(3)
    y3 = LF.dropout(x, 0.25)
    assert torch.equal(y, y3) and not torch.equal(y, y2)
    kept = (y != 0).float().mean().item()
    assert abs(kept - 0.75) < 0.01
    dy = torch.randn_like(y)
    y.backward(dy)
    keep = (y != 0)
    want = (dy.float() * keep.float() * (1 / torch.tensor(0.75))).to(torch.bfloat16)
    assert torch.equal(x.grad, want)
    assert LF.dropout(x, 0.3, training=False) is x and LF.dropout(x, 0.0) is x


@pytest.mark.parametrize("mask_kind", [None, "bool_padding", "float_2d"])
@pytest.mark.parametrize("B,S,H,KV,hd,dtype,p", [(2, 64, 4, 2, 64, torch.bfloat16, 0.2),
                                                 (1, 48, 4, 4, 32, torch.float32, 0.5),
                                                 (2, 40, 6, 2, 128, torch.bfloat16, 0.1)])
def test_attention_dropout_vs_oracle(mask_kind, B, S, H, KV, hd, dtype, p):
    """model/llama.py:105-117 in training mode (SDPA dropout_p): forward and
    gradients of attention with dropout against the oracle in float64 given
    the kernel's keep mask (element ((b*H + h)*S + s)*S + kv of the stream),
    causal or with an explicit mask."""
    g = _seed(B * S + hd + int(p * 10))
    ld = (H + 2 * KV) * hd
    qkv = torch.randn(B * S, ld, generator=g).to(dtype)
    mask = _attn_masks(mask_kind, B, H, S, g) if mask_kind else None
    d = qkv.to(DEV)
    q2, k2, v2 = d[:, : H * hd], d[:, H * hd : (H + KV) * hd], d[:, (H + KV) * hd :]
    scale = hd**-0.5
    key = ops.dropout_key(2024, B * S)
    keep = ops.dropout_mask(B * H * S * S, p, key, DEV).cpu().view(B, H, S, S)
    mdev = mask.to(DEV) if mask is not None else None
    o, lse = ops.attn_fwd_general(q2, k2, v2, B, S, H, KV, hd, scale, mdev, p, key)

    def heads(t, n):
        return t.double().view(B, S, n, hd).transpose(1, 2).requires_grad_(True)

    qr, kr, vr = heads(qkv[:, : H * hd], H), heads(qkv[:, H * hd : (H + KV) * hd], KV), heads(qkv[:, (H + KV) * hd :], KV)
    mref = None if mask is None else (mask if mask.dtype == torch.bool else mask.double())
    oref = R.causal_gqa_attention(qr, kr, vr, scale, attn_mask=mref, dropout_keep=keep, dropout_p=p)
    tol = 1e-2 if dtype == torch.bfloat16 else 1e-5
    assert _rel_err(o.cpu().double().view(B, S, H, hd).transpose(1, 2), oref) < tol
    # the normaliser is the undropped softmax's: lse equals the no-dropout call's
    _, lse0 = ops.attn_fwd_general(q2, k2, v2, B, S, H, KV, hd, scale, mdev)
    assert torch.equal(lse, lse0)
    do = torch.randn(B * S, H * hd, generator=g).to(dtype)
    dqkv = torch.zeros_like(d)
    ops.attn_bwd_general(q2, k2, v2, o, do.to(DEV), lse, B, S, H, KV, hd, scale, dqkv[:, : H * hd],
                         dqkv[:, H * hd : (H + KV) * hd], dqkv[:, (H + KV) * hd :], mdev, p, key)
    oref.backward(do.double().view(B, S, H, hd).transpose(1, 2))
    dq = dqkv[:, : H * hd].cpu().double().view(B, S, H, hd).transpose(1, 2)
    dk = dqkv[:, H * hd : (H + KV) * hd].cpu().double().view(B, S, KV, hd).transpose(1, 2)
    dv = dqkv[:, (H + KV) * hd :].cpu().double().view(B, S, KV, hd).transpose(1, 2)
    gtol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    assert _grad_err(dq, qr.grad, vr.grad) < gtol
    assert _grad_err(dk, kr.grad, vr.grad) < gtol
    assert _rel_err(dv, vr.grad) < gtol


@pytest.mark.parametrize("B,S,H,KV,hd,dtype", [(2, 256, 8, 4, 128, torch.bfloat16), (1, 128, 4, 2, 64, torch.bfloat16),
                                               (1, 200, 4, 2, 128, torch.bfloat16), (2, 64, 4, 2, 32, torch.bfloat16),
                                               (1, 96, 4, 2, 64, torch.float32)])
def test_attention_bwd_with_rope_equals_separate_rope(B, S, H, KV, hd, dtype):
    """attn_bwd(rope=(cos, sin)) returns exactly what attn_bwd followed by
    the RoPE backward pass on dq and dk returns, on every kernel path (the
    bf16 tile and transposed-operand paths fold the rotation into their
    stores; the others run the RoPE kernel after)."""
    g = _seed(B * S * hd + H)
    ld = (H + 2 * KV) * hd
    d = torch.randn(B * S, ld, generator=g).to(dtype).to(DEV)
    q2, k2, v2 = d[:, : H * hd], d[:, H * hd : (H + KV) * hd], d[:, (H + KV) * hd :]
    scale = hd**-0.5
    path = ops.attn_path(dtype, S, hd, ld, ld, ld, H * hd)
    vt = ops.transpose_heads(d, B, S, KV, hd, col0=(H + KV) * hd) if path == 1 else None
    o, lse = ops.attn_fwd(q2, k2, v2, B, S, H, KV, hd, scale, vt)
    do = torch.randn(B * S, H * hd, generator=g).to(dtype).to(DEV)
    tr = {}
    if path == 1:
        tr = dict(qt=ops.transpose_heads(d, B, S, H, hd, col0=0), kt=ops.transpose_heads(d, B, S, KV, hd, col0=H * hd),
                  dot=ops.transpose_heads(do, B, S, H, hd, col0=0))
    cos, sin = R.rope_tables(S, hd, 10_000.0, dtype=dtype)
    cos, sin = cos.to(DEV), sin.to(DEV)
    sep = torch.zeros_like(d)
    ops.attn_bwd(q2, k2, v2, o, do, lse, B, S, H, KV, hd, scale, sep[:, : H * hd], sep[:, H * hd : (H + KV) * hd],
                 sep[:, (H + KV) * hd :], **tr)
    ops.rope_(sep, S, H + KV, hd, cos, sin, backward=True)
    fused = torch.zeros_like(d)
    ops.attn_bwd(q2, k2, v2, o, do, lse, B, S, H, KV, hd, scale, fused[:, : H * hd], fused[:, H * hd : (H + KV) * hd],
                 fused[:, (H + KV) * hd :], rope=(cos, sin), **tr)
    assert torch.equal(fused.cpu(), sep.cpu()), path
    with pytest.raises(ValueError):
        ops.attn_bwd(q2, k2, v2, o, do, lse, B, S, H, KV, hd, scale, fused[:, : H * hd],
                     fused[:, H * hd : (H + KV) * hd], fused[:, (H + KV) * hd :], rope=(cos[:, : hd // 2], sin), **tr)


@pytest.mark.parametrize("B,S,H,hd,pad", [(2, 64, 4, 128, 0), (1, 96, 8, 64, 64), (2, 33, 3, 32, 0), (1, 40, 2, 256, 8),
                                          (2, 24, 4, 48, 0)])
def test_attention_delta(B, S, H, hd, pad):
    """delta[b, h, s] = sum_d O * dO (the softmax-backward row term), fp32
    sums of bf16 products: 1e-5 relative against float64, on the vector path
    (hd 32..256, strided rows) and the element-wise one (hd 48)."""
    g = _seed(B * S * H + hd)
    ld = H * hd + pad
    o = torch.randn(B * S, ld, generator=g).to(torch.bfloat16)
    do = torch.randn(B * S, ld, generator=g).to(torch.bfloat16)
    delta = torch.empty(B, H, S, dtype=torch.float32, device=DEV)
    od, dod = o.to(DEV), do.to(DEV)
    _lib.call("lz_attn_delta", od.data_ptr(), ld, dod.data_ptr(), ld, delta.data_ptr(), B, S, H, hd,
              ops.dtype_code(od), 0)
    want = (o[:, : H * hd].double() * do[:, : H * hd].double()).view(B, S, H, hd).sum(-1).permute(0, 2, 1)
    assert _rel_err(delta, want) < 1e-5


@pytest.mark.parametrize("B,S,H,KV,hd,dtype", [(2, 256, 4, 2, 128, torch.bfloat16), (1, 192, 6, 2, 64, torch.bfloat16),
                                               (1, 128, 4, 4, 64, torch.float16), (1, 320, 4, 2, 128, torch.bfloat16)])
def test_attention_bwd_with_o_matches_separate_delta(B, S, H, KV, hd, dtype):
    """lz_attn_bwd_with_o (delta computed by the dQ kernel, which then runs
    before dK/dV) against lz_attn_delta + lz_attn_bwd on the same inputs:
    delta to 1e-6 relative (the same fp32 sums over the head dim in another
    order) and dq/dk/dv to the 16-bit format's rounding of that difference;
    with RoPE tables both return the pre-RoPE gradients.  S = 320 leaves the
    last 128-query block half outside the sequence."""
    g = _seed(B * S * H + hd)
    ld = (H + 2 * KV) * hd
    qkv = torch.randn(B * S, ld, generator=g).to(dtype).to(DEV)
    q, k, v = qkv[:, : H * hd], qkv[:, H * hd : (H + KV) * hd], qkv[:, (H + KV) * hd :]
    scale = hd ** -0.5
    o, lse = ops.attn_fwd(q, k, v, B, S, H, KV, hd, scale, None)
    do = torch.randn(B * S, H * hd, generator=g).to(dtype).to(DEV)
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32, device=DEV) / hd))
    cos, sin = ops.rope_table(S, hd, inv, dtype)
    st = ops.stream_ptr(q.device)
    for tables in (None, (cos, sin)):
        rc, rs = (None, None) if tables is None else (tables[0].data_ptr(), tables[1].data_ptr())
        outs = []
        for fused in (True, False):
            dq = torch.empty(B * S, H * hd, dtype=dtype, device=DEV)
            dk = torch.empty(B * S, KV * hd, dtype=dtype, device=DEV)
            dv = torch.empty_like(dk)
            delta = torch.full((B, H, S), float("nan"), dtype=torch.float32, device=DEV)
            if fused:
                _lib.call("lz_attn_bwd_with_o", q.data_ptr(), ld, k.data_ptr(), ld, v.data_ptr(), ld, o.data_ptr(),
                          H * hd, do.data_ptr(), H * hd, lse.data_ptr(), delta.data_ptr(), dq.data_ptr(), H * hd,
                          dk.data_ptr(), KV * hd, dv.data_ptr(), KV * hd, B, S, H, KV, hd, scale, rc, rs,
                          ops.dtype_code(q), st)
            else:
                _lib.call("lz_attn_delta", o.data_ptr(), H * hd, do.data_ptr(), H * hd, delta.data_ptr(), B, S, H, hd,
                          ops.dtype_code(o), st)
                _lib.call("lz_attn_bwd", q.data_ptr(), ld, k.data_ptr(), ld, v.data_ptr(), ld, do.data_ptr(), H * hd,
                          lse.data_ptr(), delta.data_ptr(), None, None, None, dq.data_ptr(), H * hd, dk.data_ptr(),
                          KV * hd, dv.data_ptr(), KV * hd, B, S, H, KV, hd, scale, rc, rs, ops.dtype_code(q), st)
            outs.append((delta, dq, dk, dv))
        (d1, *g1), (d2, *g2) = outs
        assert bool(torch.isfinite(d1).all())
        assert _rel_err(d1, d2) < 1e-6
        for a, b in zip(g1, g2):
            assert _rel_err(a, b) < 1e-2 and float((a.float() - b.float()).abs().max()) <= 0.02 * float(b.float().abs().max())
    # shapes outside the tile kernels are refused, not taken another way
    with pytest.raises(RuntimeError, match="lz_attn_bwd_with_o"):
        _lib.call("lz_attn_bwd_with_o", q.data_ptr(), ld, k.data_ptr(), ld, v.data_ptr(), ld, o.data_ptr(), H * hd,
                  do.data_ptr(), H * hd, lse.data_ptr(), d1.data_ptr(), g1[0].data_ptr(), H * hd, g1[1].data_ptr(),
                  KV * hd, g1[2].data_ptr(), KV * hd, B, S - 1, H, KV, hd, scale, None, None, ops.dtype_code(q), st)


@pytest.mark.parametrize("hd,S,H,KV", [(32, 130, 4, 2), (16, 64, 2, 1), (32, 1, 2, 2)])
def test_attention_fp32_small_head(hd, S, H, KV):
    """Head dims 16 and 32 (a quad of lanes per row, rows staged through LDS) in
    fp32: output, lse and all three gradients within 1e-5 of float64, over
    several 64-row chunks, a ragged tail, GQA and a one-token sequence."""
    g = _seed(hd * S + H)
    B = 2
    q = torch.randn(B, S, H, hd, generator=g)
    k = torch.randn(B, S, KV, hd, generator=g)
    v = torch.randn(B, S, KV, hd, generator=g)
    do = torch.randn(B, S, H, hd, generator=g)
    scale = hd**-0.5
    qd, kd, vd = (t.reshape(B * S, -1).to(DEV) for t in (q, k, v))
    o, lse = ops.attn_fwd(qd, kd, vd, B, S, H, KV, hd, scale, None)
    qr, kr, vr = (t.double().transpose(1, 2).requires_grad_(True) for t in (q, k, v))
    oref = R.causal_gqa_attention(qr, kr, vr, scale)
    assert _rel_err(o.cpu().view(B, S, H, hd).transpose(1, 2), oref) < 1e-5
    kk = kr.detach().repeat_interleave(H // KV, dim=1)
    sc = (qr.detach() @ kk.transpose(-1, -2)) * scale
    sc = sc.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    assert float((lse.cpu().double() - torch.logsumexp(sc, dim=-1)).abs().max()) < 1e-5
    dq = torch.empty_like(qd)
    dk = torch.empty_like(kd)
    dv = torch.empty_like(vd)
    ops.attn_bwd(qd, kd, vd, o, do.reshape(B * S, -1).to(DEV), lse, B, S, H, KV, hd, scale, dq, dk, dv)
    oref.backward(do.double().transpose(1, 2))
    assert _grad_err(dq.cpu().view(B, S, H, hd).transpose(1, 2), qr.grad, vr.grad) < 1e-5
    assert _grad_err(dk.cpu().view(B, S, KV, hd).transpose(1, 2), kr.grad, vr.grad) < 1e-5
    assert _rel_err(dv.cpu().view(B, S, KV, hd).transpose(1, 2), vr.grad) < 1e-5


def test_attention_fp32_generic():
    g = _seed(5)
    B, S, H, KV, hd = 2, 40, 4, 2, 24
    q = torch.randn(B, S, H, hd, generator=g)
    k = torch.randn(B, S, KV, hd, generator=g)
    v = torch.randn(B, S, KV, hd, generator=g)
    o, lse = ops.attn_fwd(q.view(B * S, -1).to(DEV), k.view(B * S, -1).to(DEV), v.view(B * S, -1).to(DEV),
                          B, S, H, KV, hd, hd**-0.5, None)
    oref = R.causal_gqa_attention(q.double().transpose(1, 2), k.double().transpose(1, 2), v.double().transpose(1, 2))
    assert _rel_err(o.cpu().view(B, S, H, hd).transpose(1, 2), oref) < 1e-5


# ---------------------------------------------------------------------------
# Cross entropy
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,S,V,dtype", [(2, 17, 97, torch.float32), (4, 64, 32000, torch.bfloat16),
                                         (2, 9, 1000, torch.bfloat16)])
def test_cross_entropy_fwd_bwd(B, S, V, dtype):
    g = _seed(B * S + V)
    logits = (3 * torch.randn(B, S, V, generator=g)).to(dtype)
    labels = torch.randint(0, V, (B, S), generator=g)
    labels[0, 3] = -100
    lg = logits.to(DEV).view(B * S, V)
    lab = labels.to(DEV)
    lse, row_loss = ops.ce_fwd(lg, lab, S)
    loss, count = ops.ce_reduce(row_loss, lab, B * S, S, V, clamp=False)
    lr = logits.double().requires_grad_(True)
    ref = R.shifted_cross_entropy(lr, labels)
    assert abs(float(loss) - float(ref.detach())) <= 1e-5 * abs(float(ref.detach()))
    assert int(count) == int(labels[:, 1:].ne(-100).sum())
    ref_lib = F.cross_entropy(logits.double()[:, :-1].transpose(1, 2), labels[:, 1:], ignore_index=-100)
    assert abs(float(ref.detach()) - float(ref_lib)) < 1e-10
    ref.backward(torch.tensor(0.5, dtype=torch.float64))
    d = ops.ce_bwd(lg, lab, S, lse, torch.tensor([0.5], device=DEV), count)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert _rel_err(d.view(B, S, V), lr.grad) < tol
    # clamp semantics with no valid targets
    none = torch.full((B, S), -100, dtype=torch.long, device=DEV)
    _, rl = ops.ce_fwd(lg, none, S)
    l0, c0 = ops.ce_reduce(rl, none, B * S, S, V, clamp=True)
    assert float(l0) == 0.0 and float(c0) == 1.0


# ---------------------------------------------------------------------------
# Embedding
# ---------------------------------------------------------------------------
def test_embedding_fwd_exact_bwd_close():
    g = _seed(3)
    V, d, B, S = 1000, 256, 4, 64
    table = torch.randn(V, d, generator=g).to(torch.bfloat16)
    ids = torch.randint(0, V, (B, S), generator=g)
    ids[0, :8] = 5  # repeated ids
    out = ops.embedding_fwd(ids.to(DEV), table.to(DEV))
    assert torch.equal(out.cpu(), table[ids])
    dout = torch.randn(B * S, d, generator=g).to(torch.bfloat16)
    grad = ops.embedding_bwd(ids.to(DEV), dout.to(DEV), V, torch.bfloat16)
    ref = torch.zeros(V, d, dtype=torch.float64).index_add_(0, ids.view(-1), dout.double())
    assert float((grad.cpu().double() - ref).abs().max()) <= 2 ** -8 * float(ref.abs().max())
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    bad = ids.clone()
    bad[1, 1] = V + 5
    out2 = ops.embedding_fwd(bad.to(DEV), table.to(DEV), bad_flag=flag)
    assert int(flag.item()) == 1
    assert torch.count_nonzero(out2[1, 1]) == 0


# ---------------------------------------------------------------------------
# Optimizer path
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("n,gdtype", [(1_000_003, torch.float32), (262_147, torch.bfloat16), (5, torch.float32)])
def test_adamw_matches_reference_update(n, gdtype):
    g = _seed(n)
    p = 0.02 * torch.randn(n, generator=g)
    m = torch.zeros(n)
    v = torch.zeros(n)
    pd, md, vd = p.to(DEV), m.to(DEV), v.to(DEV)
    out = torch.empty(n, dtype=torch.bfloat16, device=DEV)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    for step in range(1, 11):
        gr = (1e-3 * torch.randn(n, generator=g)).to(gdtype)
        ops.adamw_(pd, md, vd, gr.to(DEV), step=step, p_out=out, **hp)
        R.adamw_update(p, m, v, gr.float(), step=step, **hp)
    assert _rel_err(pd, p) < 1e-5
    assert _rel_err(md, m) < 1e-5
    assert _rel_err(vd, v) < 1e-5
    assert torch.equal(out.cpu(), pd.cpu().to(torch.bfloat16))


def test_adamw_grad_scale_and_unaligned_views():
    g = _seed(9)
    n = 10_001
    p = 0.02 * torch.randn(n + 1, generator=g)
    gr = 1e-2 * torch.randn(n + 1, generator=g)
    pd = p.to(DEV)[1:]
    md = torch.zeros(n + 1, device=DEV)[1:]
    vd = torch.zeros(n + 1, device=DEV)[1:]
    scale = torch.tensor([0.25], device=DEV)
    ops.adamw_(pd, md, vd, gr.to(DEV)[1:], lr=1e-3, beta1=0.9, beta2=0.99, eps=1e-8, weight_decay=0.0, step=1,
               grad_scale=scale)
    pr, mr, vr = p[1:].clone(), torch.zeros(n), torch.zeros(n)
    R.adamw_update(pr, mr, vr, gr[1:] * 0.25, lr=1e-3, beta1=0.9, beta2=0.99, eps=1e-8, weight_decay=0.0, step=1)
    assert _rel_err(pd, pr) < 1e-5


def test_adamw_device_step_matches_host_step():
    """adamw_step_ (step count and bias-correction factors on the device) then
    adamw_ with those factors: bit-identical to adamw_ with the host step over
    10 steps, and the device counter reads 10 at the end."""
    g = _seed(21)
    n = 300_007
    p = 0.02 * torch.randn(n, generator=g)
    ph, mh, vh = p.to(DEV), torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)
    pd, md, vd = p.to(DEV), torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)
    step = torch.zeros(1, dtype=torch.int64, device=DEV)
    hyper = torch.zeros(3, dtype=torch.float32, device=DEV)
    hp = dict(beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    for t in range(1, 11):
        gr = (1e-3 * torch.randn(n, generator=g)).to(torch.bfloat16).to(DEV)
        ops.adamw_(ph, mh, vh, gr, lr=3e-4, step=t, **hp)
        ops.adamw_step_(step, 3e-4, 0.9, 0.95, 0.1, hyper)
        ops.adamw_(pd, md, vd, gr, lr=0.0, step=1, hyper=hyper, **hp)
    assert int(step.item()) == 10
    bc1, bc2 = 1 - 0.9 ** 10, 1 - 0.95 ** 10
    assert torch.allclose(hyper.cpu().double(), torch.tensor([-3e-4 / bc1, math.sqrt(bc2), 1 - 3e-5],
                                                             dtype=torch.float64), rtol=1e-6, atol=0)
    assert torch.equal(pd, ph) and torch.equal(md, mh) and torch.equal(vd, vh)


def test_adamw_multi_matches_per_tensor():
    """adamw_multi_ over 30 tensors (two launches of at most 24; sizes from 0
    to 100k across the 4096-element chunk boundaries) against adamw_ tensor by
    tensor over 3 steps with a grad scale: the same bits for p, m, v and the
    bf16 copy, for bf16 and fp32 gradients, with device-resident factors, and
    with tensors 16-byte aligned (four elements per access) or not (scalar);
    sumsq_multi_ against float64 and per-tensor sumsq_ to 1e-6 (fp32 per-thread
    partials)."""
    g = _seed(31)
    sizes = [0, 1, 7, 4095, 4096, 4097, 100_003] + [int(x) for x in torch.randint(1, 20000, (23,), generator=g)]
    hp = dict(beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    scale = torch.tensor([0.5], device=DEV)
    def at_offset(t, off):
        """t's values in a view `off` elements into a larger buffer (off=1:
        not 16-byte aligned, so the multi-tensor kernel takes its scalar loop)."""
        buf = torch.zeros(t.numel() + off, dtype=t.dtype, device=DEV)
        v = buf[off:]
        v.copy_(t.to(DEV))
        return v

    for gdt, with_out, use_hyper, off in ((torch.bfloat16, True, False, 0), (torch.float32, False, False, 0),
                                          (torch.bfloat16, True, True, 0), (torch.bfloat16, True, False, 1)):
        p0 = [0.02 * torch.randn(n, generator=g) for n in sizes]
        A = [[p.to(DEV), torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)] for p, n in zip(p0, sizes)]
        B = [[at_offset(p, off), at_offset(torch.zeros(n), off), at_offset(torch.zeros(n), off)]
             for p, n in zip(p0, sizes)]
        oa = [torch.zeros(n, dtype=torch.bfloat16, device=DEV) if with_out else None for n in sizes]
        ob = [at_offset(torch.zeros(n, dtype=torch.bfloat16), off) if with_out else None for n in sizes]
        step = torch.zeros(1, dtype=torch.int64, device=DEV)
        hyper = torch.zeros(3, dtype=torch.float32, device=DEV)
        for t in range(1, 4):
            grads = [(1e-3 * torch.randn(n, generator=g)).to(gdt).to(DEV) for n in sizes]
            for (pa, ma, va), gr, o in zip(A, grads, oa):
                if pa.numel():
                    ops.adamw_(pa, ma, va, gr, lr=3e-4, step=t, grad_scale=scale, p_out=o, **hp)
            if use_hyper:
                ops.adamw_step_(step, 3e-4, 0.9, 0.95, 0.1, hyper)
            ops.adamw_multi_([b[0] for b in B], [b[1] for b in B], [b[2] for b in B], grads, ob,
                             lr=3e-4, step=t, grad_scale=scale, hyper=hyper if use_hyper else None, **hp)
        for (pa, ma, va), (pb, mb, vb), x, y in zip(A, B, oa, ob):
            assert torch.equal(pa, pb) and torch.equal(ma, mb) and torch.equal(va, vb)
            if with_out:
                assert torch.equal(x, y)
        acc1 = torch.zeros(1, dtype=torch.float64, device=DEV)
        acc2 = torch.zeros(1, dtype=torch.float64, device=DEV)
        for gr in grads:
            if gr.numel():
                ops.sumsq_(gr, acc1)
        ops.sumsq_multi_(grads, acc2)
        # both sum fp32 partials per thread (over different partitions) in fp64
        ref = float(sum(gr.double().pow(2).sum() for gr in grads))
        assert abs(float(acc2.item()) - ref) <= 1e-6 * ref
        assert abs(float(acc1.item()) - float(acc2.item())) <= 1e-6 * ref


@pytest.mark.parametrize("n,gdtype,off", [(1_000_003, torch.float32, 0), (262_147, torch.bfloat16, 0),
                                          (3 * 512, torch.bfloat16, 0), (5, torch.float32, 0),
                                          (10_001, torch.bfloat16, 1)])
def test_adamw_norm_matches_adamw_and_sumsq(n, gdtype, off):
    """adamw_norm_ (the update plus the sum of squares of g from the same
    read) against adamw_ then float64 sums: p, m, v and the bf16 copy bit for
    bit over 3 steps with a grad scale; the accumulated sum to 1e-6 (fp32
    squares of 4 elements, float64 after), added onto what acc held, and the
    same bits on a second run over the same gradient (fixed summation order).
    off=1 puts every operand one element into its buffer: not 16-byte
    aligned, so the scalar update runs after a separate sum-of-squares pass."""
    g = _seed(n % 1000 + off)
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    scale = torch.tensor([0.5], device=DEV)

    def at_offset(t):
        buf = torch.zeros(t.numel() + off, dtype=t.dtype, device=DEV)
        buf[off:].copy_(t.to(DEV))
        return buf[off:]

    p0 = 0.02 * torch.randn(n, generator=g)
    pa, ma, va = p0.to(DEV), torch.zeros(n, device=DEV), torch.zeros(n, device=DEV)
    pb, mb, vb = at_offset(p0), at_offset(torch.zeros(n)), at_offset(torch.zeros(n))
    oa = torch.zeros(n, dtype=torch.bfloat16, device=DEV)
    ob = at_offset(torch.zeros(n, dtype=torch.bfloat16))
    ws = torch.full((ops.adamw_norm_workspace_words(n),), float("nan"), dtype=torch.float64, device=DEV)
    for t in range(1, 4):
        gr = (1e-3 * torch.randn(n, generator=g)).to(gdtype)
        gd = at_offset(gr)
        acc = torch.full((1,), 2.5, dtype=torch.float64, device=DEV)
        ops.adamw_(pa, ma, va, gr.to(DEV), step=t, grad_scale=scale, p_out=oa, **hp)
        ops.adamw_norm_(pb, mb, vb, gd, acc, ws, step=t, grad_scale=scale, p_out=ob, **hp)
        assert torch.equal(pa, pb) and torch.equal(ma, mb) and torch.equal(va, vb) and torch.equal(oa, ob)
        ref = float(gr.double().pow(2).sum())
        assert abs(float(acc.item()) - 2.5 - ref) <= 1e-6 * ref
        if off == 0:
            # same gradient, fresh copies of the state: the same sum bit for bit
            acc2 = torch.full((1,), 2.5, dtype=torch.float64, device=DEV)
            ops.adamw_norm_(pb.clone(), mb.clone(), vb.clone(), gd, acc2, ws, step=t, **hp)
            assert torch.equal(acc, acc2)
    with pytest.raises(RuntimeError, match="workspace"):
        ops.adamw_norm_(pb, mb, vb, gd, acc, ws[:1], step=4, **hp)


def test_sumsq_and_clip():
    g = _seed(4)
    a = torch.randn(3_000_001, generator=g)
    b = torch.randn(1001, generator=g).to(torch.bfloat16)
    acc = torch.zeros(1, dtype=torch.float64, device=DEV)
    ops.sumsq_(a.to(DEV), acc)
    ops.sumsq_(b.to(DEV), acc)
    ref = float(a.double().pow(2).sum() + b.double().pow(2).sum())
    assert abs(float(acc.item()) - ref) <= 1e-6 * ref
    norm = torch.empty(1, device=DEV)
    scale = torch.empty(1, device=DEV)
    ops.clip_finalize(acc, 1.0, norm, scale)
    n = math.sqrt(ref)
    assert abs(float(norm.item()) - n) <= 1e-6 * n
    assert abs(float(scale.item()) - 1.0 / (n + 1e-6)) <= 1e-6
    ops.clip_finalize(acc, 1e9, norm, scale)
    assert float(scale.item()) == 1.0
    ops.clip_finalize(acc, 0.0, norm, scale)
    assert float(scale.item()) == 1.0


def test_multi_tensor_gather_scatter_bit_exact():
    g = _seed(8)
    shapes = [(7,), (33, 5), (1,), (4096, 3), (2, 2, 2), (100_000,)]
    ts = [torch.randn(*s, generator=g).to(torch.bfloat16).to(DEV) for s in shapes]
    numels = [t.numel() for t in ts]
    offs = [sum(numels[:i]) for i in range(len(ts))]
    total = sum(numels)
    tensors = list(ts)
    tensors[2] = None  # a missing gradient reads as zeros
    table = ops.SegmentTable.from_tensors(tensors, offs, numels, DEV)
    flat = torch.empty(total, dtype=torch.bfloat16, device=DEV)
    ops.mt_gather(table, torch.bfloat16, flat, 0, total)
    ref = torch.cat([(torch.zeros(n, dtype=torch.bfloat16) if t is None else t.cpu().view(-1))
                     for t, n in zip(tensors, numels)])
    assert torch.equal(flat.cpu(), ref)
    # a bucket window in the middle, accumulated into fp32
    acc = torch.ones(5000, device=DEV)
    ops.mt_gather(table, torch.bfloat16, acc, 100, 5100, accumulate=True)
    assert torch.equal(acc.cpu(), ref[100:5100].float() + 1.0)
    # scatter fp32 -> bf16 storages
    src = torch.randn(total, generator=g).to(DEV)
    outs = [torch.empty(s, dtype=torch.bfloat16, device=DEV) for s in shapes]
    t2 = ops.SegmentTable.from_tensors(outs, offs, numels, DEV)
    ops.mt_scatter(src, t2, torch.bfloat16, 0, total)
    got = torch.cat([o.cpu().view(-1) for o in outs])
    assert torch.equal(got, src.cpu().to(torch.bfloat16))


def test_transpose_and_cast_exact():
    g = _seed(12)
    x = torch.randn(130, 70, generator=g).to(torch.bfloat16).to(DEV)
    assert torch.equal(ops.transpose2d(x).cpu(), x.cpu().t())
    B, S, nh, hd = 2, 65, 3, 32
    y = torch.randn(B * S, 5 * hd, generator=g).to(torch.bfloat16).to(DEV)
    t = ops.transpose_heads(y, B, S, nh, hd, col0=hd)
    ref = y.cpu()[:, hd : hd + nh * hd].view(B, S, nh, hd).permute(0, 2, 3, 1)
    assert torch.equal(t.cpu(), ref)
    f = torch.randn(1001, generator=g).to(DEV)
    assert torch.equal(ops.cast(f, torch.bfloat16).cpu(), f.cpu().to(torch.bfloat16))
    z = ops.zeros((37,), torch.float32, DEV)
    assert torch.count_nonzero(z) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_copy2d_exact(dtype):
    """Window copies, bit-exact: contiguous (one long row), strided windows on
    the 16-byte path, rows beyond one grid column (70 000 > 65 535) and
    unaligned shapes on the element-wise path."""
    g = _seed(13)
    cases = [((64, 256), (64, 256), 64, 256),      # contiguous
             ((40, 96), (40, 160), 40, 64),        # strided window, 16-byte path
             ((70000, 8), (70000, 16), 70000, 8),  # rows past one grid column
             ((33, 21), (33, 37), 33, 21)]         # element-wise path
    for (sr, sc), (dr, dc), rows, cols in cases:
        src = torch.randn(sr, sc, generator=g).to(dtype).to(DEV)
        dst = torch.full((dr, dc), -7.0, dtype=dtype, device=DEV)
        ops.copy2d(src[:rows, :cols], dst[:rows, :cols])
        want = torch.full((dr, dc), -7.0, dtype=dtype)
        want[:rows, :cols] = src.cpu()[:rows, :cols]
        assert torch.equal(dst.cpu(), want), (sr, sc, dr, dc)
    # a window that starts 4 elements in (not 16-byte aligned for bf16)
    src = torch.randn(16, 64, generator=g).to(dtype).to(DEV)
    dst = torch.zeros(16, 64, dtype=dtype, device=DEV)
    ops.copy2d(src[:, 4:36], dst[:, 4:36])
    want = torch.zeros(16, 64, dtype=dtype)
    want[:, 4:36] = src.cpu()[:, 4:36]
    assert torch.equal(dst.cpu(), want)
