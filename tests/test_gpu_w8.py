"""GPU parity of the 8-bit lm_head path (the reference's W8A16Weights,
src/kernels/gemv_w4a16.cuh:147-166) against the CPU oracle, through the C-ABI.

Tolerances:
  * quantized bytes, scales and dequantized rows: bit-exact against the
    oracle's restatement of k_quant_w8 (gemv_w4a16.cu:478-495);
  * bf16 GEMV / verify outputs: max-rel <= 1e-2 against the fp64 product of the
    oracle's q * s and mean-abs <= 1e-3 against its bf16 rounding (the 4-bit
    path's bar, tests/gate_gemv.cu:115);
  * argmax: exact index wherever the fp64 top-2 margin exceeds the fp32
    accumulation bound 1e-4 * max|logit|.
"""
import numpy as np
import pytest

from gpu_util import dev, download, empty, host

pytestmark = pytest.mark.gpu

MAXREL_BF16 = 1e-2
MEANABS_BF16 = 1e-3


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


def _unpack_layout(w, N, K):
    """Device blocks -> logical (q int8 [N][K], s u16 [N][G]). The block
    layout is [tile][g][j][position][32 B] with position p holding row
    4 (p % 16) + p / 16 of the tile and byte b of chunk j at k = 128 g + 32 j + b;
    scales are [tile][g][64 rows]."""
    G = K // 128
    raw = download(w.qweight, N * K).reshape(N // 64, G, 4, 64, 32)
    p = np.arange(64)
    rows = 4 * (p % 16) + p // 16
    logical = np.empty((N // 64, 64, G, 4, 32), np.uint8)
    logical[:, rows] = raw.transpose(0, 3, 1, 2, 4)
    q = (logical.reshape(N, K).astype(np.int16) - 128).astype(np.int8)
    s = download(w.scale, N * G * 2).view(np.uint16).reshape(N // 64, G, 64)
    s = s.transpose(0, 2, 1).reshape(N, G)
    return q, s


def _edge_source(orc, N, K, seed):
    """Random bf16 weights with the quantizer's edge cases written in: an
    all-zero group (scale 0), a group whose max is 127 so w * 127 / max hits
    exact halves (round-half-even), a group with one huge value, negative max."""
    w = orc.gen_bf16(N * K, seed, 40, 0).reshape(N, K).copy()
    f = orc.bf16_to_f32(w)
    if N >= 4 and K >= 256:
        f[0, :128] = 0.0
        halves = np.arange(-63.5, 64.5, 1.0, dtype=np.float32)[:127]
        f[1, 128:255] = halves
        f[1, 255] = 127.0
        f[2, :128] *= 1e-3
        f[2, 5] = 3.0e4
        f[3, 128:256] = -np.abs(f[3, 128:256])
        f[3, 200] = -50.0
    return orc.f32_to_bf16(f)


def _dequant_ref(orc, q, s):
    N, K = q.shape
    sf = np.repeat(orc.bf16_to_f32(s), 128, axis=1)
    return orc.f32_to_bf16(q.astype(np.float32) * sf)


@pytest.mark.parametrize("N,K", [(64, 128), (64, 512), (192, 1024), (320, 5120), (128, 2176)])
def test_w8_quantize_bitexact(hip, orc, N, K):
    import torch

    src = _edge_source(orc, N, K, seed=N + K)
    w = hip.quantize_w8a16(dev(src), N, K)
    torch.cuda.synchronize()
    assert w.total_bytes() == N * K + N * (K // 128) * 2
    q_ref, s_ref = orc.w8_quantize(src)
    q, s = _unpack_layout(w, N, K)
    assert np.array_equal(s, s_ref)
    assert np.array_equal(q, q_ref)
    if N >= 4 and K >= 256:
        assert s_ref[0, 0] == 0 and not q_ref[0, :128].any()
        assert q_ref[1, 128:255].tolist() == np.round(np.arange(-63.5, 63.5)).astype(int).tolist()
    out = empty((N, K), np.uint16)
    hip.w8a16_dequant_rows(out, w, 0, N)
    torch.cuda.synchronize()
    assert np.array_equal(host(out, np.uint16), _dequant_ref(orc, q_ref, s_ref))
    # a window of rows
    part = empty((N // 2, K), np.uint16)
    hip.w8a16_dequant_rows(part, w, N // 4, N // 2)
    torch.cuda.synchronize()
    assert np.array_equal(host(part, np.uint16), _dequant_ref(orc, q_ref, s_ref)[N // 4: N // 4 + N // 2])
    hip.w8a16_free(w)
    assert w.qweight is None and w.out_f == 0


def test_w8_bad_arguments(hip, orc):
    import torch

    src = torch.zeros(64 * 256, dtype=torch.int16, device="cuda")
    for args, status in (((64, 256, 64), hip.QW4_ERR_GROUP), ((32, 256, 128), hip.QW4_ERR_SHAPE),
                         ((64, 200, 128), hip.QW4_ERR_SHAPE)):
        with pytest.raises(hip.W4A16Error) as e:
            hip.quantize_w8a16(src, args[0], args[1], args[2])
        assert e.value.status == status
    w = hip.quantize_w8a16(src, 64, 256)
    s = hip.gemv_scratch_alloc(256, 64, 128, 1)
    y = empty((2, 64), np.uint16)
    x = torch.zeros(2 * 256, dtype=torch.int16, device="cuda")
    with pytest.raises(hip.W4A16Error) as e:   # M above the scratch's max_m
        hip.gemm_small_w8a16(y, w, x, 2, s)
    assert e.value.status == hip.QW4_ERR_SCRATCH
    with pytest.raises(hip.W4A16Error) as e:
        hip.w8a16_dequant_rows(empty((64, 256), np.uint16), w, 32, 64)
    assert e.value.status == hip.QW4_ERR_SHAPE
    torch.cuda.synchronize()
    hip.gemv_scratch_free(s)
    hip.w8a16_free(w)


def _run(hip, orc, scratch, N, K, M, seed):
    import torch

    src = orc.gen_bf16(N * K, seed, 41, 0).reshape(N, K)
    x = orc.gen_x(M, K, seed=seed, tensor=9)
    w = hip.quantize_w8a16(dev(src), N, K)
    y = empty((M, N), np.uint16)
    dx = dev(x)
    if M == 1:
        hip.gemv_w8a16(y, w, dx, scratch)
    else:
        hip.gemm_small_w8a16(y, w, dx, M, scratch)
    torch.cuda.synchronize()
    q, s = orc.w8_quantize(src)
    return w, dx, y, orc.w8_matmul_f64(x, q, s)


@pytest.mark.parametrize("M", [1, 2, 9, 16])
# (31040, 5120) at M = 2 and (16384, 1024) at every M > 1 run the verify kernel
# with the activation rows staged in LDS (the default path, "dec")
@pytest.mark.parametrize("N,K", [(64, 512), (5120, 5120), (31040, 5120), (640, 2176),
                                 (16384, 1024)])
def test_w8_gemv_and_verify(hip, orc, scratch, decode_path, N, K, M):
    import torch

    w, dx, y, ref = _run(hip, orc, scratch, N, K, M, seed=N + M)
    m = orc.parity_metrics(host(y, np.uint16), ref)
    print(f"w8 M={M} {N}x{K}: {m}", flush=True)
    assert m["max_rel"] <= MAXREL_BF16, m
    assert m["mean_abs_vs_bf16_ref"] <= MEANABS_BF16, m
    first = host(y, np.uint16).copy()
    for _ in range(5):
        if M == 1:
            hip.gemv_w8a16(y, w, dx, scratch)
        else:
            hip.gemm_small_w8a16(y, w, dx, M, scratch)
    torch.cuda.synchronize()
    assert np.array_equal(host(y, np.uint16), first)
    hip.w8a16_free(w)


@pytest.mark.parametrize("M", [1, 9])
def test_w8_lm_head_argmax_full_vocab(hip, orc, scratch, decode_path, M):
    """The reference's default head (lm_head_bits 8, model.cu:796-815, :1044-1047)
    at the full vocabulary: quantize 248320 x 5120 on the GPU (bytes and scales
    bit-exact against the oracle), then the fused GEMV + fp32 row-argmax."""
    import torch

    N, K = 248320, 5120
    src = empty((N * K,), np.uint16)
    hip.gen_bf16(src, N * K, 3, 42, 0)
    w = hip.quantize_w8a16(src, N, K)
    del src
    x = orc.gen_x(M, K, seed=3, tensor=10)
    dx = dev(x)
    idx = empty((M,), np.int32)
    hip.gemv_argmax_w8a16(idx, w, dx, M, scratch)
    torch.cuda.synchronize()
    got = host(idx, np.int32)
    q_ref, s_ref = orc.w8_quantize(orc.gen_bf16(N * K, 3, 42, 0).reshape(N, K))
    q, s = _unpack_layout(w, N, K)
    assert np.array_equal(s, s_ref)
    assert np.array_equal(q, q_ref)
    del q, s
    ref = orc.w8_matmul_f64(x, q_ref, s_ref)
    want, margin = orc.argmax_rows_f64(ref)
    bound = 1e-4 * np.max(np.abs(ref), axis=1)
    for m in range(M):
        print(f"row {m}: idx {got[m]} want {want[m]} margin {margin[m]:.4g} bound {bound[m]:.3g}",
              flush=True)
        if margin[m] > bound[m]:
            assert got[m] == want[m]
        else:
            assert ref[m, got[m]] >= ref[m, want[m]] - bound[m]
    # logits path of the same weights agrees with the fused argmax
    y = empty((M, N), np.uint16)
    hip.gemm_small_w8a16(y, w, dx, M, scratch) if M > 1 else hip.gemv_w8a16(y, w, dx, scratch)
    torch.cuda.synchronize()
    mets = orc.parity_metrics(host(y, np.uint16), ref)
    assert mets["max_rel"] <= MAXREL_BF16, mets
    hip.gemv_argmax_w8a16(idx, w, dx, M, scratch)
    torch.cuda.synchronize()
    assert np.array_equal(host(idx, np.int32), got)
    hip.w8a16_free(w)
