"""Non-finite activations through the decode (M = 1, k_dec) and verify (M = 9,
k_rows) kernels, through the C-ABI.

The reference's fp32 GEMV adds per group p = sum_k (128 + q) x then subtracts
(128 + zp) * sum_k x (src/kernels/gemv_w4a16.cu:136-147): an Inf or NaN
activation in a group makes that group's term Inf - Inf = NaN (or NaN), so
every output of that activation row is NaN. Checked here: the poisoned row is
NaN at every output (where the fp64 oracle's direct dot product is non-finite
too), and the other rows of the same call equal the oracle within the bf16
bar (max-rel 1e-2, mean-abs 1e-3) and are bitwise equal to the same call with
the poisoned row made finite.
"""
import numpy as np
import pytest

from gpu_util import dev, empty, host, repack_from_logical

pytestmark = pytest.mark.gpu

BF16_INF = 0x7F80
BF16_NINF = 0xFF80
BF16_NAN = 0x7FC0


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


def _call(hip, scratch, w, x, M, N):
    import torch

    y = empty((M, N), np.uint16)
    if M == 1:
        hip.gemv_w4a16(y, w, dev(x), scratch)
    else:
        hip.gemm_small_w4a16(y, w, dev(x), M, scratch)
    torch.cuda.synchronize()
    return host(y, np.uint16).reshape(M, N)


def _bf16_to_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("M", [1, 9])
@pytest.mark.parametrize("N,K", [(5120, 4096), (7168, 5120), (5120, 17408)])
@pytest.mark.parametrize("bad", [BF16_INF, BF16_NINF, BF16_NAN, "inf-ninf"])
def test_nonfinite_activation(hip, orc, scratch, M, N, K, bad):
    q, zp, s = orc.gen_weights(N, K, seed=7)
    w = repack_from_logical(hip, orc, q, zp, s, "awq_k")
    x = orc.gen_x(M, K, seed=7).copy()
    row = M // 2
    clean = _call(hip, scratch, w, x, M, N)
    xb = x.copy()
    if bad == "inf-ninf":   # +Inf and -Inf in one group: the dot product itself is NaN
        xb[row, 300] = BF16_INF
        xb[row, 301] = BF16_NINF
    else:
        xb[row, 300] = bad
    got = _call(hip, scratch, w, xb, M, N)
    print(f"M={M} {N}x{K} bad={bad}: row {row} NaN count {np.isnan(_bf16_to_f64(got[row])).sum()}",
          flush=True)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = orc.matmul_f64(xb, q, zp, s)
    assert not np.isfinite(ref[row]).any()
    assert np.isnan(_bf16_to_f64(got[row])).all()
    others = [m for m in range(M) if m != row]
    if others:
        assert np.array_equal(got[others], clean[others])
        m = orc.parity_metrics(got[others], ref[others])
        assert m["max_rel"] <= 1e-2 and m["mean_abs_vs_bf16_ref"] <= 1e-3, m
    hip.awq_free(w)


def test_subnormal_group_is_bounded(hip, orc, scratch):
    """A group whose largest |x| is an fp32 subnormal contributes at most
    ~2^-100 per output in the decode kernel (its fixed-point scale caps at
    2^126); the reference's fp32 sum keeps such terms. The output of an
    all-subnormal x must therefore be within 1e-30 of the oracle (both are ~0
    against any normal activation's scale)."""
    N, K = 5120, 4096
    q, zp, s = orc.gen_weights(N, K, seed=3)
    w = repack_from_logical(hip, orc, q, zp, s, "awq_k")
    x = orc.gen_x(1, K, seed=3).copy()
    x[0, :] = (x[0, :] & 0x807F) | 0x0001   # exponent 0: every element subnormal
    got = _bf16_to_f64(_call(hip, scratch, w, x, 1, N))
    ref = orc.matmul_f64(x, q, zp, s)
    assert np.isfinite(got).all()
    assert np.max(np.abs(got - ref)) < 1e-30
    hip.awq_free(w)
