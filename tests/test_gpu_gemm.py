"""GPU parity of the long-prompt projection GEMM (vx27_hip_gemm_bf16): the
weights bf16 in the tiled layout, each fp32 activation as two bf16 parts
hi = bf16(x), lo = bf16(x - hi), fp32 accumulation.

Two references in float64 from the same bf16 weights:
  - W (hi + lo): what the kernel multiplies, so the only difference is the
    fp32 accumulation: |d| <= 2e-6 * sum_k |W||x| (a dropped lo part would
    be ~2^-9 of it, a transposed or misplaced operand far more);
  - W x: the product the reference's fp32 matvec computes (vx27_pmat.c:98-101)
    on the same weights, within the split's bound, |d| <= 2^-15 * sum_k |W||x|.
Shapes leave the last token tile and the last row tile partial, and the row
strides exceed the rows: rows past R and columns past N of y keep their NaN
canaries.  The three-part exact GEMV (vx27_hip_gemv_bf16) agrees with it to
the same 2^-15 bound."""
import numpy as np
import pytest

from gpu_common import say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from vx27_amd import lib as L
    c = L.Ctx(0)
    yield c
    c.close()


def split2(x):
    """hi = bf16(x) (round to nearest even), lo = bf16(x - hi), as float32."""
    from vx27_amd import workloads as W
    hi = W.bf16_to_f32(W.bf16_bits(x))
    lo = W.bf16_to_f32(W.bf16_bits((x - hi).astype(np.float32)))
    return hi, lo


def run_gemm(ctx, Wb, x, x_stride=None, y_stride=None, rows_extra=3):
    from vx27_amd import lib as L
    N, K = Wb.shape
    R = x.shape[0]
    xs = x_stride or K
    ys = y_stride or N
    xp = np.zeros((R, xs), np.float32)
    xp[:, :K] = x
    wt = ctx.put_tiled(Wb)
    xb = ctx.put(xp)
    y0 = np.full((R + rows_extra, ys), np.nan, np.float32)
    yb = ctx.put(y0)
    L.check(L.lib().vx27_hip_gemm_bf16(ctx.h, wt.ptr, N, K, xb.ptr, xs, R, yb.ptr, ys), "gemm")
    y = yb.download((R + rows_extra, ys), np.float32)
    for bb in (wt, xb, yb):
        bb.free()
    assert np.isnan(y[R:]).all(), "rows past R written"
    assert np.isnan(y[:R, N:]).all(), "columns past N written"
    return y[:R, :N]


@pytest.mark.parametrize("N,K,R,xs,ys", [(528, 640, 300, None, None), (256, 128, 1, None, None),
                                         (4096, 1024, 512, 1028, 4100), (16, 64, 257, None, 20),
                                         (1040, 5120, 256, None, None)])
def test_gemm_vs_float64(ctx, N, K, R, xs, ys):
    from vx27_amd import workloads as W
    r = W.rng(11, f"gemm{N}x{K}x{R}")
    Wb = W.bf16_bits(W.normal(r, (N, K), 0.02))
    x = W.normal(r, (R, K))
    y = run_gemm(ctx, Wb, x, xs, ys)
    Wf = W.bf16_to_f32(Wb).astype(np.float64)
    hi, lo = split2(x)
    mag = np.abs(x).astype(np.float64) @ np.abs(Wf).T
    ref_split = (hi.astype(np.float64) + lo.astype(np.float64)) @ Wf.T
    ref = x.astype(np.float64) @ Wf.T
    e_split = float(np.max(np.abs(y - ref_split) / mag))
    e_plain = float(np.max(np.abs(y - ref) / mag))
    say(f"  gemm {N}x{K} R={R}: vs W(hi+lo) {e_split:.2e}, vs W x {e_plain:.2e} (of sum|W||x|)")
    assert e_split <= 2e-6
    assert e_plain <= 2.0 ** -15


def test_gemm_matches_exact_gemv(ctx):
    """The GEMM against the three-part exact GEMV on the real in-projection
    width (16480 rows, 5120 inputs) for 160 tokens."""
    from vx27_amd import lib as L, workloads as W
    r = W.rng(12, "gemm_vs_gemv")
    N, K, R = 16480, 5120, 160
    Wb = W.bf16_bits(W.normal(r, (N, K), 0.02))
    x = W.normal(r, (R, K))
    y = run_gemm(ctx, Wb, x)
    wb, xb, yb = ctx.put(Wb), ctx.put(x), ctx.buf(R * N * 4)
    L.check(L.lib().vx27_hip_gemv_bf16(ctx.h, wb.ptr, N, K, xb.ptr, K, R, yb.ptr, N), "gemv")
    yg = yb.download((R, N), np.float32)
    for bb in (wb, xb, yb):
        bb.free()
    mag = np.abs(x).astype(np.float64) @ np.abs(W.bf16_to_f32(Wb).astype(np.float64)).T
    e = float(np.max(np.abs(y - yg) / mag))
    say(f"  gemm vs exact gemv, {N}x{K} R={R}: {e:.2e} of sum|W||x|")
    assert e <= 2.0 ** -15


def test_gemm_deterministic(ctx):
    """The last partial round of tiles is split along k (here 5 tiles of 1040
    rows x 256 tokens in 20 parts) and its parts are added in part order, so
    two calls give the same bits."""
    from vx27_amd import workloads as W
    r = W.rng(13, "gemm_det")
    N, K, R = 1040, 5120, 256
    Wb = W.bf16_bits(W.normal(r, (N, K), 0.02))
    x = W.normal(r, (R, K))
    y1 = run_gemm(ctx, Wb, x)
    y2 = run_gemm(ctx, Wb, x)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
