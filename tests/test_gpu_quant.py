"""GPU parity of the INT4 lm_head quantizer (the reference's quantize_w4a16_raw
/ k_quant_i4, src/model/model.cu:140-186) against the CPU oracle, through the
C-ABI: the device quantizer writes the repacked layout directly; the oracle's
compressed-tensors tensors of the same source, repacked by the (separately
pinned) repack, must give the same bytes -- packed words, the 160-byte
scale/zero-point records and the zero-point array -- bit for bit. Then the
quantized head through the GEMV and the fused argmax against the oracle's
product (the GEMV bars) and exact indices where the top-2 margin exceeds the
fp32 accumulation bound."""
import numpy as np
import pytest

from gpu_util import dev, empty, host, weights_buffers

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import torch

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    import w4a16_hip

    w4a16_hip.lib()
    return w4a16_hip


def _source(orc, N, K, seed):
    """bf16 rows with the quantizer's edge cases: a constant positive, a
    constant negative, an all-zero and an evenly spaced group."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.03).astype(np.float32)
    w[1, :128] = 0.5
    w[2, 128:256] = -1.25
    w[3, :128] = 0.0
    w[4, :128] = (np.arange(128) % 16 - 7) * 2.0 ** -6
    return orc.f32_to_bf16(w)


@pytest.mark.parametrize("N,K", [(512, 1024), (4096, 5120)])
def test_quantize_w4a16_bitexact(hip, orc, N, K):
    import torch

    src = _source(orc, N, K, seed=N + K)
    wq = hip.quantize_w4a16_raw(dev(src), N, K)
    torch.cuda.synchronize()
    packed, scale, zp = orc.quant_i4(src)
    wr = hip.awq_repack(dev(packed), dev(scale), dev(zp), N, K)
    torch.cuda.synchronize()
    got, want = weights_buffers(wq, N, K), weights_buffers(wr, N, K)
    for name, a, b in zip(("qweight", "scale records", "zeros"), got, want):
        assert np.array_equal(a, b), name
    hip.awq_free(wq)
    hip.awq_free(wr)


def test_quantized_head_gemv_and_argmax(hip, orc):
    """One GPU's 8-way shard of the 248320-row head (31040 x 5120): GEMV and
    fused argmax of the device-quantized weights against the oracle."""
    import torch

    N, K = 31040, 5120
    src = _source(orc, N, K, seed=5)
    w = hip.quantize_w4a16_raw(dev(src), N, K)
    q, zp, s = orc.unpack_ct(*orc.quant_i4(src), N, K)
    scr = hip.gemv_scratch_alloc(K, N, 128, 16)
    for M in (1, 9):
        x = orc.gen_x(M, K, seed=M, tensor=9)
        dx = dev(x)
        y = empty((M, N), np.uint16)
        idx = empty((M,), np.int32)
        hip.gemm_small_w4a16(y, w, dx, M, scr)
        hip.gemv_argmax_w4a16(idx, w, dx, M, scr)
        torch.cuda.synchronize()
        ref = orc.matmul_f64(x, q, zp, s)
        m = orc.parity_metrics(host(y, np.uint16), ref)
        print(f"quantized head M={M}: {m}", flush=True)
        assert m["max_rel"] <= 1e-2 and m["mean_abs_vs_bf16_ref"] <= 1e-3, m
        want, margin = orc.argmax_rows_f64(ref)
        got = host(idx, np.int32)
        bound = 1e-4 * np.max(np.abs(ref), axis=1)
        for r in range(M):
            if margin[r] > bound[r]:
                assert got[r] == want[r], (M, r)
    hip.gemv_scratch_free(scr)
    hip.awq_free(w)
