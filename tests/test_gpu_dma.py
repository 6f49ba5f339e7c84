"""GPU parity of the bf16 skinny kernel's LDS-DMA items (k_rows at M = 1: the
weight, scale and zero-point loads of each item go straight into LDS, D items
per wave, or into registers) through the C-ABI entry points that take M = 1:
gemv_w4a16 / _f32, the fused residual / swiglu / rmsnorm forms, the argmax
heads and the W8A16 GEMV (src/kernels/gemv_w4a16.cuh:88-92, :112-118,
:147-166; src/kernels/elementwise.cuh:34-43; src/model/model.cu:697-700,
:772-785).

Bar: bit-exact against the register-item kernel. For the same unit size and
waves both do the same per-unit arithmetic in the same order (only which
workgroup owns which unit differs), so any difference is a load or wait
error. k_rows serves M = 1 for the 8-bit head and for shapes the
integer-MFMA decode kernel does not take; the oracle checks of every path
are in test_gpu_parity, test_gpu_fused and test_gpu_w8; one more here per
shape class (the GEMV bars: max-rel 1e-2, mean-abs 1e-3)."""
import numpy as np
import pytest

from gpu_util import dev, empty, host, repack_from_logical

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import torch

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    import w4a16_hip

    w4a16_hip.lib()
    return w4a16_hip


@pytest.fixture(scope="module")
def scratch(hip):
    s = hip.gemv_scratch_alloc(17408, 248320, 128, 16)
    yield s
    hip.gemv_scratch_free(s)


def _sync():
    import torch

    torch.cuda.synchronize()


def _gen(hip, N, K, seed):
    """Device-generated AWQ tensor, repacked (large shapes without the oracle)."""
    import torch

    G = K // 128
    q = torch.empty(K // 8 * N, dtype=torch.int32, device="cuda")
    s = torch.empty(G * N, dtype=torch.int16, device="cuda")
    z = torch.empty(G * N // 8, dtype=torch.int32, device="cuda")
    hip.gen_awq_k(q, s, z, N, K, seed, 3)
    w = hip.awq_alloc_fused(N, K)
    hip.awq_repack_awq_into(w, 0, q, s, z, N, hip.LAYOUT_AWQ_K)
    _sync()
    return w


def _x(hip, n, sid):
    import torch

    x = torch.empty(n, dtype=torch.int16, device="cuda")
    hip.gen_bf16(x, n, 0, sid, 0)
    return x


def _both(hip, run):
    """run() with k_rows register items (32-row units, 8 waves) and with its
    LDS-DMA items at every depth and at the policy's; every result must equal
    the first. Set through the library's tuning override, reset afterwards."""
    hip.tune_decode(2, S=2, W=8)
    try:
        want = run()
        for depth in (2, 3, 4, 0):
            hip.tune_decode(1, D=depth)
            got = run()
            assert np.array_equal(got, want), depth
    finally:
        hip.tune_decode(0)


# the model's projections, one group (G < waves), an odd group count, few units
# and the 8-way shards
SHAPES = [(7168, 5120), (5120, 4096), (34816, 5120), (5120, 17408), (64, 128), (192, 384),
          (640, 1280), (896, 5120), (4352, 5120), (5120, 512), (5120, 2176)]


@pytest.mark.parametrize("N,K", SHAPES)
def test_dma_gemv(hip, scratch, N, K):
    w, x = _gen(hip, N, K, seed=N + K), _x(hip, K, 7000 + K)
    print(f"dma gemv {N}x{K}", flush=True)

    def bf16():
        y = empty((1, N), np.uint16)
        hip.gemv_w4a16(y, w, x, scratch)
        _sync()
        return host(y, np.uint16)

    def f32():
        y = empty((1, N), np.float32)
        hip.gemv_w4a16_f32(y, w, x, scratch)
        _sync()
        return host(y, np.float32)

    _both(hip, bf16)
    _both(hip, f32)
    hip.awq_free(w)


@pytest.mark.parametrize("N,K", [(5120, 4096), (5120, 17408), (320, 640)])
def test_dma_residual(hip, scratch, N, K):
    w, x, h0 = _gen(hip, N, K, seed=N), _x(hip, K, 11), _x(hip, N, 12)
    print(f"dma residual {N}x{K}", flush=True)

    def run():
        h = h0.clone()
        hip.gemv_residual_w4a16(h, w, x, 1, scratch)
        _sync()
        return host(h, np.uint16)

    _both(hip, run)
    hip.awq_free(w)


@pytest.mark.parametrize("N,K", [(34816, 5120), (256, 640), (4352, 5120)])
def test_dma_swiglu(hip, scratch, N, K):
    w, x = _gen(hip, N, K, seed=N + 1), _x(hip, K, 13)
    print(f"dma swiglu {N}x{K}", flush=True)

    def run():
        y = empty((1, N // 2), np.uint16)
        hip.gemv_swiglu_w4a16(y, w, x, 1, scratch)
        _sync()
        return host(y, np.uint16)

    _both(hip, run)
    hip.awq_free(w)


@pytest.mark.parametrize("N,K", [(7168, 5120), (896, 5120), (128, 256)])
def test_dma_rmsnorm(hip, scratch, N, K):
    import torch

    w, h = _gen(hip, N, K, seed=N + 2), _x(hip, K, 14)
    nw = _x(hip, K, 15)
    nw.copy_((nw.view(torch.bfloat16) * 0.1).view(torch.int16))
    print(f"dma rmsnorm {N}x{K}", flush=True)

    def run():
        y = empty((1, N), np.uint16)
        hip.gemv_rmsnorm_w4a16(y, w, h, nw, 1e-6, 1, scratch)
        _sync()
        return host(y, np.uint16)

    _both(hip, run)
    hip.awq_free(w)


@pytest.mark.parametrize("N", [248320, 4096, 64])
def test_dma_argmax(hip, scratch, N):
    K = 5120
    w, x = _gen(hip, N, K, seed=N + 3), _x(hip, K, 16)
    print(f"dma argmax {N}", flush=True)

    def run():
        idx = empty((1,), np.int32)
        hip.gemv_argmax_w4a16(idx, w, x, 1, scratch)
        _sync()
        return host(idx, np.int32)

    _both(hip, run)
    hip.awq_free(w)


@pytest.mark.parametrize("N,K", [(31040, 5120), (640, 1280)])
def test_dma_w8(hip, scratch, N, K):
    src = _x(hip, N * K, 17)
    w = hip.quantize_w8a16(src, N, K)
    x = _x(hip, K, 18)
    del src
    print(f"dma w8 {N}x{K}", flush=True)

    def bf16():
        y = empty((1, N), np.uint16)
        hip.gemv_w8a16(y, w, x, scratch)
        _sync()
        return host(y, np.uint16)

    def argmax():
        idx = empty((1,), np.int32)
        hip.gemv_argmax_w8a16(idx, w, x, 1, scratch)
        _sync()
        return host(idx, np.int32)

    _both(hip, bf16)
    _both(hip, argmax)
    hip.w8a16_free(w)


@pytest.mark.parametrize("N,K", [(5120, 4096), (1024, 2048), (64, 128)])
def test_dma_vs_oracle(hip, orc, scratch, N, K):
    q, zp, s = orc.gen_weights(N, K, seed=N + 1)
    x = orc.gen_x(1, K, seed=1)
    w = repack_from_logical(hip, orc, q, zp, s)
    y = empty((1, N), np.uint16)
    hip.gemv_w4a16(y, w, dev(x), scratch)
    _sync()
    m = orc.parity_metrics(host(y, np.uint16), orc.matmul_f64(x, q, zp, s))
    print(f"dma oracle {N}x{K}: {m}", flush=True)
    assert m["max_rel"] <= 1e-2 and m["mean_abs_vs_bf16_ref"] <= 1e-3, m
    hip.awq_free(w)


# ------------------------------------------------- M > 1 (verify, heads)
def _both_m(hip, run, rows=2):
    """M > 1: LDS-DMA weight items (activations loaded with each item) against
    register items, 8 waves, 32-row units (rows=2) or the policy's unit size
    (rows=None: 64-row units for outputs with at least as many tiles as CUs)."""
    S = rows or 0
    hip.tune_decode(2, S=S, W=8)
    try:
        want = run()
        for depth in (2, 3, 4, 0):
            hip.tune_decode(1, S=S, D=depth)
            got = run()
            assert np.array_equal(got, want), depth
    finally:
        hip.tune_decode(0)


@pytest.mark.parametrize("M", [2, 9, 16])
@pytest.mark.parametrize("N,K", [(7168, 5120), (5120, 17408), (192, 384), (34816, 5120)])
def test_dma_verify(hip, scratch, N, K, M):
    w = _gen(hip, N, K, seed=N + K + M)
    x, h0 = _x(hip, M * K, 20 + M), _x(hip, M * N, 30 + M)
    print(f"dma verify M={M} {N}x{K}", flush=True)

    def gemm():
        y = empty((M, N), np.uint16)
        hip.gemm_small_w4a16(y, w, x, M, scratch)
        _sync()
        return host(y, np.uint16)

    def residual():
        h = h0.clone()
        hip.gemv_residual_w4a16(h, w, x, M, scratch)
        _sync()
        return host(h, np.uint16)

    def argmax():
        idx = empty((M,), np.int32)
        hip.gemv_argmax_w4a16(idx, w, x, M, scratch)
        _sync()
        return host(idx, np.int32)

    for rows in (2, None):
        _both_m(hip, gemm, rows)
        _both_m(hip, residual, rows)
        _both_m(hip, argmax, rows)
    if M == 2 and N % 128 == 0:
        def swiglu():
            y = empty((M, N // 2), np.uint16)
            hip.gemv_swiglu_w4a16(y, w, x, M, scratch)
            _sync()
            return host(y, np.uint16)

        _both_m(hip, swiglu)
    hip.awq_free(w)


@pytest.mark.parametrize("M", [2, 9])
def test_dma_w8_verify(hip, scratch, M):
    N, K = 31040, 5120
    src = _x(hip, N * K, 19)
    w = hip.quantize_w8a16(src, N, K)
    x = _x(hip, M * K, 21)
    del src

    def gemm():
        y = empty((M, N), np.uint16)
        hip.gemm_small_w8a16(y, w, x, M, scratch)
        _sync()
        return host(y, np.uint16)

    def argmax():
        idx = empty((M,), np.int32)
        hip.gemv_argmax_w8a16(idx, w, x, M, scratch)
        _sync()
        return host(idx, np.int32)

    for rows in (2, None):
        _both_m(hip, gemm, rows)
        _both_m(hip, argmax, rows)
    hip.w8a16_free(w)


# ------------------------------------------- M > 1 with the rows staged in LDS
def _staged_vs_per_item(hip, run):
    """run() with the policy (the activation rows staged in LDS where they fit
    and the workgroups own several units; else, with 3 to 6 units per
    workgroup, the group-major kernel k_rows_gm), with per-item activation
    loads (qw4_tune_decode mode 4), with register items (mode 2) and with the
    group-major kernel off (mode 5): every result equal. The per-row sums run
    over the same groups in the same wave order in every form, so any
    difference is a staging, padding, slot-reuse or wait error."""
    try:
        hip.tune_decode(0)
        want = run()
        for mode in (4, 2, 5):
            hip.tune_decode(mode)
            got = run()
            assert np.array_equal(got, want), mode
    finally:
        hip.tune_decode(0)


# gate|up (544 tiles), a head-like 16384-row output, a short-K one; the 5120-row
# output has fewer tiles than half the CUs and keeps the per-item loads. Where
# the rows do not fit the staging (M = 12 / 16 on gate|up, the 3- and
# 6-units-per-workgroup shapes) the group-major kernel runs.
STAGED = [(34816, 5120), (16384, 1024), (20480, 384), (5120, 4096), (24576, 5120),
          (49152, 5120)]


@pytest.mark.parametrize("M", [2, 9, 12, 16])
@pytest.mark.parametrize("N,K", STAGED)
def test_staged_rows(hip, scratch, N, K, M):
    w, x, h0 = _gen(hip, N, K, seed=N + M), _x(hip, M * K, 900 + M), _x(hip, M * N, 901)
    print(f"staged rows M={M} {N}x{K}", flush=True)

    def bf16():
        y = empty((M, N), np.uint16)
        hip.gemm_small_w4a16(y, w, x, M, scratch)
        _sync()
        return host(y, np.uint16)

    def residual():
        h = h0.clone()
        hip.gemv_residual_w4a16(h, w, x, M, scratch)
        _sync()
        return host(h, np.uint16)

    def swiglu():
        y = empty((M, N // 2), np.uint16)
        hip.gemv_swiglu_w4a16(y, w, x, M, scratch)
        _sync()
        return host(y, np.uint16)

    def argmax():
        idx = empty((M,), np.int32)
        hip.gemv_argmax_w4a16(idx, w, x, M, scratch)
        _sync()
        return host(idx, np.int32)

    for run in (bf16, residual, swiglu, argmax):
        _staged_vs_per_item(hip, run)
    hip.awq_free(w)


def test_staged_rows_vs_oracle(hip, orc, scratch):
    """One staged shape against the oracle (the GEMV bars)."""
    N, K, M = 16384, 1024, 9
    q, zp, s = orc.gen_weights(N, K, seed=77)
    w = repack_from_logical(hip, orc, q, zp, s)
    x = orc.gen_x(M, K, seed=78)
    y = empty((M, N), np.uint16)
    hip.gemm_small_w4a16(y, w, dev(x), M, scratch)
    _sync()
    m = orc.parity_metrics(host(y, np.uint16), orc.matmul_f64(x, q, zp, s))
    print(f"staged rows vs oracle: {m}", flush=True)
    assert m["max_rel"] <= 1e-2 and m["mean_abs_vs_bf16_ref"] <= 1e-3, m
    hip.awq_free(w)
