"""GPU parity of the prefill matmul (literal int8, 32+ tokens) against the
oracle: the exact path (nhip_matmul_i8_dev) is bit-identical with
Scalar.MatMulRows' order; the fused epilogue (nhip_matmul_i8_fused_dev) is
within the required tolerance, max|y - y_ref| <= 1e-4 * RMS(y_ref)."""
import numpy as np
import pytest

from test_matmul_gpu import SENTINEL, int8_case, run_i8

pytestmark = pytest.mark.gpu


def run_fused(hip, weights, q, qs, tokens, ldy, r0, r1):
    dq, ds = hip.DeviceBuffer.from_array(q), hip.DeviceBuffer.from_array(qs)
    dy = hip.DeviceBuffer.from_array(np.full(tokens * ldy, SENTINEL, dtype=np.float32))
    hip.check(hip.lib().nhip_matmul_i8_fused_dev(weights.handle, dq.ptr, ds.ptr, tokens, dy.ptr, ldy, r0, r1, None))
    return dy.download(np.float32).reshape(tokens, ldy)


SHAPES = [(32, 64, 64), (64, 256, 512), (100, 80, 96), (65, 48, 32), (128, 1024, 2048), (512, 512, 2048),
          (200, 130, 4096), (33, 256, 384), (40, 1000, 256), (33, 640, 256)]


@pytest.mark.parametrize("tokens,rows,cols", SHAPES)
def test_gemm_exact_bit_exact(hip, orc, tokens, rows, cols):
    w, scales, x, q, qs = int8_case(orc, tokens * 7 + rows + cols, rows, cols, tokens)
    weights = hip.Weights.int8(w, scales)
    y = run_i8(hip, weights, q, qs, tokens, rows, 0, rows)
    want = np.full((tokens, rows), SENTINEL, dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, want, rows, 0, rows)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("tokens,rows,cols", SHAPES)
def test_gemm_fused_within_tolerance(hip, orc, tokens, rows, cols):
    w, scales, x, q, qs = int8_case(orc, tokens * 11 + rows + cols, rows, cols, tokens)
    weights = hip.Weights.int8(w, scales)
    y = run_fused(hip, weights, q, qs, tokens, rows, 0, rows)
    want = np.zeros((tokens, rows), dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, want, rows, 0, rows)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert np.max(np.abs(y.astype(np.float64) - want)) <= 1e-4 * rms
    # and against a float64 evaluation of the same integers
    hs = scales.view(np.float16).astype(np.float64).reshape(rows, cols // 32)
    d = np.einsum("tgk,ngk->tng", q.reshape(tokens, -1, 32).astype(np.int64),
                  w.reshape(rows, -1, 32).astype(np.int64)).astype(np.float64)
    exact = (d * hs[None, :, :]).sum(axis=2) * qs.astype(np.float64)[:, None]
    assert np.max(np.abs(y - exact)) <= 1e-4 * rms


@pytest.mark.parametrize("r0,r1", [(5, 77), (16, 32), (0, 1), (79, 80)])
def test_gemm_row_ranges_untouched(hip, orc, r0, r1):
    tokens, rows, cols = 70, 80, 256
    w, scales, x, q, qs = int8_case(orc, 3 + r0, rows, cols, tokens)
    weights = hip.Weights.int8(w, scales)
    ldy = rows + 3
    y = run_i8(hip, weights, q, qs, tokens, ldy, r0, r1)
    want = np.full((tokens, ldy), SENTINEL, dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, want, ldy, r0, r1)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    yf = run_fused(hip, weights, q, qs, tokens, ldy, r0, r1)
    assert np.all(yf[:, :r0] == SENTINEL) and np.all(yf[:, r1:] == SENTINEL)


def test_gemm_special_scales_exact(hip, orc):
    tokens, rows, cols = 96, 64, 512
    w, scales, x, q, qs = int8_case(orc, 808, rows, cols, tokens)
    scales = scales.copy()
    flat = scales.reshape(-1)
    flat[::7], flat[::11], flat[::13], flat[::19] = 0x8000, 0x0000, 0x0001, 0x7C00
    weights = hip.Weights.int8(w, scales)
    y = run_i8(hip, weights, q, qs, tokens, rows, 0, rows)
    want = np.zeros((tokens, rows), dtype=np.float32)
    orc.matmul_rows_i8(w, scales, q, qs, tokens, want, rows, 0, rows)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_gemm_prefill_config_full_size(hip, orc):
    """The prefill configuration at full size: M = 512 tokens, K = 2048,
    N = 8192.  Exact path bit-identical with Scalar.MatMulRows' order, fused
    path within 1e-4 * RMS; the oracle runs row-parallel on its pool (the
    same bits as one thread)."""
    tokens, rows, cols = 512, 8192, 2048
    w, scales, x, q, qs = int8_case(orc, 0x512, rows, cols, tokens)
    weights = hip.Weights.int8(w, scales)
    want = np.zeros((tokens, rows), dtype=np.float32)
    members = orc.lib().or_baseline_start(8)
    try:
        orc.lib().or_baseline_matmul_i8(orc.p(w), orc.p(scales), rows, cols, 32, orc.p(q), orc.p(qs), tokens,
                                        orc.p(want), rows, 0, rows)
    finally:
        orc.lib().or_baseline_stop()
    assert members == 8
    y = run_i8(hip, weights, q, qs, tokens, rows, 0, rows)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    yf = run_fused(hip, weights, q, qs, tokens, rows, 0, rows)
    rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
    assert np.max(np.abs(yf.astype(np.float64) - want)) <= 1e-4 * rms
