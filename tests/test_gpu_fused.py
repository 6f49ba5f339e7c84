"""GPU parity of the layer steps around the projections and of their fused
forms, through the C-ABI (src/kernels/elementwise.cu:8-49;
src/model/model.cu:697-700, :772-785), and of the linear() dispatcher
(model.cu:522-565).

Bars: residual_add is bit-exact against the oracle (one fp32 add of two bf16
values, rounded once); rmsnorm and swiglu within one bf16 ulp with < 1% of
elements off (the fp32 sum order and the device expf / rsqrtf differ from
numpy's); every fused entry point is bit-exact against the same steps run
unfused on the GPU, and within the GEMV bars (max-rel 1e-2, mean-abs 1e-3) of
the oracle composition (fp64 projection, rounded where the reference rounds);
swiglu's large products get an ulp bar instead of the absolute mean
(_check_ulp)."""
import numpy as np
import pytest

from gpu_util import dev, empty, host, repack_from_logical

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.fixture(scope="module")
def hip():
    import torch

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    import w4a16_hip

    w4a16_hip.lib()
    return w4a16_hip


@pytest.fixture(scope="module")
def scratch(hip):
    s = hip.gemv_scratch_alloc(17408, 34816, 128, 16)
    yield s
    hip.gemv_scratch_free(s)


def _sync():
    import torch

    torch.cuda.synchronize()


def _ulp_close(orc, got, want):
    g = orc.bf16_to_f32(got).astype(np.float64)
    w = orc.bf16_to_f32(want).astype(np.float64)
    assert np.all(np.abs(g - w) <= np.abs(w) * 2.0 ** -7 + 1e-30)
    assert np.mean(got != want) < 0.01


def _check(orc, y, ref, tag):
    """The GEMV bars: max-rel <= 1e-2, mean-abs <= 1e-3 against the bf16-rounded
    oracle composition."""
    m = orc.parity_metrics(y, ref)
    print(f"{tag}: {m}", flush=True)
    assert m["max_rel"] <= 1e-2, (tag, m)
    assert m["mean_abs_vs_bf16_ref"] <= 1e-3, (tag, m)


def _check_ulp(orc, y, ref, tag):
    """For swiglu outputs (a product, |y| up to ~50 where a bf16 ulp is 0.25, so
    an absolute mean bar would count single rounding flips): max-rel <= 1e-2 and
    99% of the elements within 1 ulp of the bf16-rounded oracle composition
    (a small output can sit a few ulps off: the rounding of its gate and up
    inputs moves it by their ulps, not its own)."""
    m = orc.parity_metrics(y, ref)
    yf = orc.bf16_to_f32(y).astype(np.float64)
    rb = orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(ref, np.float32))).astype(np.float64)
    ulp = np.maximum(np.abs(rb), 2.0 ** -126) * 2.0 ** -7
    off = np.abs(yf - rb) / ulp
    m["max_ulp"], m["frac_over_1ulp"] = float(off.max()), float(np.mean(off > 1.0))
    print(f"{tag}: {m}", flush=True)
    assert m["max_rel"] <= 1e-2, (tag, m)
    assert m["frac_over_1ulp"] <= 0.01, (tag, m)


def _norm_w(orc, K, seed):
    # small weights around 0 (the checkpoint's norm weights enter as 1 + w)
    return orc.f32_to_bf16(orc.bf16_to_f32(orc.gen_x(1, K, seed=seed)[0]) * np.float32(0.1))


# ------------------------------------------------------ stand-alone steps
@pytest.mark.parametrize("rows,dim", [(1, 5120), (9, 4096), (16, 17408), (3, 136), (2, 8704)])
def test_rmsnorm(hip, orc, rows, dim):
    x, w = orc.gen_x(rows, dim, seed=dim + rows), _norm_w(orc, dim, 11)
    out = empty((rows, dim), np.uint16)
    hip.rmsnorm(out, dev(x), dev(w), rows, dim, EPS)
    _sync()
    _ulp_close(orc, host(out, np.uint16), orc.rmsnorm_bf16(x, w, EPS))


@pytest.mark.parametrize("n", [5120, 9 * 5120 + 3, 1])
def test_residual_add(hip, orc, n):
    a, b = orc.gen_x(1, n, seed=1)[0], orc.gen_x(1, n, seed=2)[0]
    da = dev(a)
    hip.residual_add(da, dev(b), n)
    _sync()
    assert np.array_equal(host(da, np.uint16), orc.residual_add_bf16(a, b))


@pytest.mark.parametrize("rows,inter", [(1, 17408), (12, 256), (16, 8)])
def test_swiglu(hip, orc, rows, inter):
    f = orc.gen_x(rows, 2 * inter, seed=inter)
    out = empty((rows, inter), np.uint16)
    hip.swiglu(out, dev(f), rows, inter)
    _sync()
    _ulp_close(orc, host(out, np.uint16), orc.swiglu_bf16(f, inter))


# ------------------------------------------------------------ fused forms
def _plain(hip, y, w, x, M, s):
    if M == 1:
        hip.gemv_w4a16(y, w, x, s)
    else:
        hip.gemm_small_w4a16(y, w, x, M, s)


@pytest.mark.parametrize("M", [1, 2, 9, 16])
@pytest.mark.parametrize("N,K", [(5120, 4096), (5120, 17408), (320, 640)])
def test_gemv_residual(hip, orc, scratch, M, N, K):
    q, zp, s = orc.gen_weights(N, K, seed=M + N, tensor=1)
    w = repack_from_logical(hip, orc, q, zp, s)
    x, h0 = orc.gen_x(M, K, seed=M), orc.gen_x(M, N, seed=M + 100)
    dx = dev(x)
    y = empty((M, N), np.uint16)
    _plain(hip, y, w, dx, M, scratch)
    dh = dev(h0)
    hip.gemv_residual_w4a16(dh, w, dx, M, scratch)
    _sync()
    got = host(dh, np.uint16)
    assert np.array_equal(got, orc.residual_add_bf16(h0, host(y, np.uint16)))
    # the reference rounds the projection to bf16, then adds in fp32 and rounds
    ref = orc.residual_add_bf16(h0, orc.f32_to_bf16(orc.matmul_f64(x, q, zp, s).astype(np.float32)))
    _check(orc, got, orc.bf16_to_f32(ref), f"gemv_residual M={M} {N}x{K}")
    hip.awq_free(w)


@pytest.mark.parametrize("M", [1, 3, 9, 16])
@pytest.mark.parametrize("inter,K", [(17408, 5120), (4352, 5120), (256, 1024)])
def test_gemv_swiglu(hip, orc, scratch, M, inter, K):
    q, zp, s = orc.gen_weights(2 * inter, K, seed=inter + M, tensor=2)
    w = repack_from_logical(hip, orc, q, zp, s)
    x = orc.gen_x(M, K, seed=M + 7)
    dx = dev(x)
    yf = empty((M, 2 * inter), np.uint16)
    _plain(hip, yf, w, dx, M, scratch)
    ys = empty((M, inter), np.uint16)
    hip.swiglu(ys, yf, M, inter)
    y = empty((M, inter), np.uint16)
    hip.gemv_swiglu_w4a16(y, w, dx, M, scratch)   # fused at any M
    y2 = empty((M, inter), np.uint16)
    tmp = empty((M, 2 * inter), np.uint16)
    hip.gemv_swiglu_w4a16(y2, w, dx, M, scratch, tmp=tmp)   # through tmp for M > 2
    _sync()
    got = host(y, np.uint16)
    assert np.array_equal(got, host(ys, np.uint16))
    assert np.array_equal(host(y2, np.uint16), got)
    # the reference rounds gate and up to bf16, then swiglu in fp32
    gu = orc.f32_to_bf16(orc.matmul_f64(x, q, zp, s).astype(np.float32))
    _check_ulp(orc, got, orc.bf16_to_f32(orc.swiglu_bf16(gu, inter)), f"gemv_swiglu M={M} inter={inter}")
    hip.awq_free(w)


# one group (waves without chunks), more chunks than the 1024 virtual threads
# of the sum order (1088), and a 16-wave decode launch (K = 17408)
@pytest.mark.parametrize("M", [1, 2, 3, 9, 16])
@pytest.mark.parametrize("N,K", [(7168, 5120), (34816, 5120), (640, 1024), (256, 128),
                                 (1024, 8704), (5120, 17408)])
def test_gemv_rmsnorm(hip, orc, scratch, M, N, K):
    q, zp, s = orc.gen_weights(N, K, seed=N + M, tensor=3)
    w = repack_from_logical(hip, orc, q, zp, s)
    h, nw = orc.gen_x(M, K, seed=M + 3), _norm_w(orc, K, 5)
    dh, dnw = dev(h), dev(nw)
    xn = empty((M, K), np.uint16)
    hip.rmsnorm(xn, dh, dnw, M, K, EPS)
    y0 = empty((M, N), np.uint16)
    _plain(hip, y0, w, xn, M, scratch)
    y = empty((M, N), np.uint16)
    tmp = empty((M, K), np.uint16)
    hip.gemv_rmsnorm_w4a16(y, w, dh, dnw, EPS, M, scratch, tmp=tmp)
    _sync()
    got = host(y, np.uint16)
    assert np.array_equal(got, host(y0, np.uint16))
    xr = orc.rmsnorm_bf16(h, nw, EPS)
    _check(orc, got, orc.matmul_f64(xr, q, zp, s), f"gemv_rmsnorm M={M} {N}x{K}")
    hip.awq_free(w)


def test_gemv_rmsnorm_m1_without_tmp(hip, orc, scratch):
    """M = 1 at K = 17408: beyond the decode kernel's staging, so with tmp the
    call runs rmsnorm + decode GEMV (bitwise the unfused steps, checked in
    test_gemv_rmsnorm); without tmp it runs the bf16 skinny kernel with the row
    normalized in LDS, held to the GEMV bars against the oracle composition."""
    N, K, M = 5120, 17408, 1
    q, zp, s = orc.gen_weights(N, K, seed=2, tensor=6)
    w = repack_from_logical(hip, orc, q, zp, s)
    h, nw = orc.gen_x(M, K, seed=9), _norm_w(orc, K, 4)
    y = empty((M, N), np.uint16)
    hip.gemv_rmsnorm_w4a16(y, w, dev(h), dev(nw), EPS, M, scratch)
    _sync()
    xr = orc.rmsnorm_bf16(h, nw, EPS)
    _check(orc, host(y, np.uint16), orc.matmul_f64(xr, q, zp, s), "gemv_rmsnorm M=1 no tmp")
    hip.awq_free(w)


def test_gemv_rmsnorm_needs_tmp_when_not_staged(hip, orc, scratch):
    """M = 16 rows of K = 5120 do not fit the LDS staging: without tmp the call
    reports a shape error instead of computing something else."""
    N, K, M = 640, 5120, 16
    q, zp, s = orc.gen_weights(N, K, seed=1, tensor=4)
    w = repack_from_logical(hip, orc, q, zp, s)
    y = empty((M, N), np.uint16)
    with pytest.raises(hip.W4A16Error):
        hip.gemv_rmsnorm_w4a16(y, w, dev(orc.gen_x(M, K, seed=1)), dev(_norm_w(orc, K, 1)), EPS,
                               M, scratch)
    hip.awq_free(w)


# ------------------------------------------------------------- dispatcher
@pytest.fixture(scope="module")
def workspace(hip):
    ws = hip.gemm_workspace_alloc(256 << 20)
    yield ws
    hip.gemm_workspace_free(ws)


def test_linear_paths(hip, orc, scratch, workspace):
    """linear() picks the GEMV (T = 1), 16-row skinny chunks (T <= max_t) or the
    prefill GEMM, and matches each path run directly."""
    N, K = 1024, 2048   # 1.1 MB: skinny passes up to 16 * 9 rows
    q, zp, s = orc.gen_weights(N, K, seed=8, tensor=5)
    w = repack_from_logical(hip, orc, q, zp, s)
    mt = hip.linear_max_t(w)
    for T in sorted({1, 2, 16, 17, 40, mt, mt + 1, 300}):
        x = orc.gen_x(T, K, seed=T)
        dx = dev(x)
        y = empty((T, N), np.uint16)
        hip.linear_w4a16(y, w, dx, T, scratch, workspace)
        y0 = empty((T, N), np.uint16)
        if T == 1:
            hip.gemv_w4a16(y0, w, dx, scratch)
        elif T <= mt:
            for i in range(0, T, 16):
                n = min(16, T - i)
                hip.gemm_small_w4a16(y0[i:i + n], w, dx[i:i + n], n, scratch)
        else:
            hip.gemm_w4a16(y0, w, dx, T, workspace)
        _sync()
        got = host(y, np.uint16)
        assert np.array_equal(got, host(y0, np.uint16)), T
        ref = orc.matmul_f64(x, q, zp, s, round_w=T > mt)
        _check(orc, got, ref, f"linear T={T}")
    hip.awq_free(w)
