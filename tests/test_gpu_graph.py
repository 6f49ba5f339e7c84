"""Graph capture and replay of the path's entry points (the reference captures
its decode step in a CUDA graph, src/model/model.cu:880-946, and requires the
kernels to be capturable: no sync, no allocation, self-resetting scratch).

One hipGraph holds a decode GEMV (LDS-DMA items), a verify GEMM (M = 9), both
argmax heads, the fused residual / swiglu / rmsnorm steps, the W8 GEMV and a
prefill GEMM whose tiles are split (split-K partials + fixup). It is replayed
several times with eager work and synchronisations between the replays; every
replay must equal the eager results bitwise (the split counters, argmax keys
and fixed-point words reset themselves, and the summation order is fixed)."""
import numpy as np
import pytest

from gpu_util import empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip():
    import torch

    assert torch.cuda.is_available(), "GPU test run without a GPU"
    import w4a16_hip

    w4a16_hip.lib()
    return w4a16_hip


def _gen(hip, N, K, seed):
    import torch

    G = K // 128
    q = torch.empty(K // 8 * N, dtype=torch.int32, device="cuda")
    s = torch.empty(G * N, dtype=torch.int16, device="cuda")
    z = torch.empty(G * N // 8, dtype=torch.int32, device="cuda")
    hip.gen_awq_k(q, s, z, N, K, seed, 3)
    w = hip.awq_alloc_fused(N, K)
    hip.awq_repack_awq_into(w, 0, q, s, z, N, hip.LAYOUT_AWQ_K)
    torch.cuda.synchronize()
    return w


def _x(hip, n, sid):
    import torch

    x = torch.empty(n, dtype=torch.int16, device="cuda")
    hip.gen_bf16(x, n, 0, sid, 0)
    return x


def test_graph_replays_match_eager(hip):
    import torch

    hip.tune_decode(0)
    hip.tune_gemm(-1)
    s = hip.gemv_scratch_alloc(17408, 34816, 128, 16)
    ws = hip.gemm_workspace_alloc(256 << 20)
    wq = _gen(hip, 7168, 5120, 1)      # qkv
    wd = _gen(hip, 5120, 17408, 2)     # down
    wg = _gen(hip, 34816, 5120, 3)     # gate|up
    wh = _gen(hip, 4096, 5120, 4)      # a head
    src = _x(hip, 4096 * 5120, 5)
    w8 = hip.quantize_w8a16(src, 4096, 5120)
    del src
    x5, x9 = _x(hip, 5120, 6), _x(hip, 9 * 5120, 7)
    x17 = _x(hip, 17408, 8)
    a_pf = _x(hip, 512 * 17408, 9)     # down M=512: every tile split (split-K, 6 k-slices)
    h0 = _x(hip, 5120, 10)
    nw = torch.zeros(5120, dtype=torch.int16, device="cuda")
    outs = {
        "gemv": empty((1, 7168), np.uint16), "verify": empty((9, 7168), np.uint16),
        "head": empty((9,), np.int32), "head1": empty((1,), np.int32),
        "res": empty((5120,), np.uint16), "swiglu": empty((1, 17408), np.uint16),
        "norm": empty((1, 7168), np.uint16), "w8": empty((1, 4096), np.uint16),
        "w8head": empty((1,), np.int32), "prefill": empty((512, 5120), np.uint16),
    }

    def run():
        hip.gemv_w4a16(outs["gemv"], wq, x5, s)
        hip.gemm_small_w4a16(outs["verify"], wq, x9, 9, s)
        hip.gemv_argmax_w4a16(outs["head"], wh, x9, 9, s)
        hip.gemv_argmax_w4a16(outs["head1"], wh, x5, 1, s)
        outs["res"].copy_(h0)
        hip.gemv_residual_w4a16(outs["res"], wd, x17, 1, s)
        hip.gemv_swiglu_w4a16(outs["swiglu"], wg, x5, 1, s)
        hip.gemv_rmsnorm_w4a16(outs["norm"], wq, x5, nw, 1e-6, 1, s)
        hip.gemv_w8a16(outs["w8"], w8, x5, s)
        hip.gemv_argmax_w8a16(outs["w8head"], w8, x5, 1, s)
        hip.gemm_w4a16(outs["prefill"], wd, a_pf, 512, ws)

    def snap():
        torch.cuda.synchronize()
        return {k: v.clone() for k, v in outs.items()}

    run()
    want = snap()
    for v in outs.values():
        v.zero_()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for rep in range(4):
        for v in outs.values():
            v.zero_()
        g.replay()
        got = snap()
        for k in want:
            assert torch.equal(got[k], want[k]), (rep, k)
        # eager work between replays, on the same scratch and workspace
        run()
        eager = snap()
        for k in want:
            assert torch.equal(eager[k], want[k]), (rep, k, "eager")
    print("graph replays:", 4, {k: tuple(v.shape) for k, v in want.items()}, flush=True)
    assert int(host(want["head1"], np.int32)[0]) >= 0
    del g
    for w in (wq, wd, wg, wh):
        hip.awq_free(w)
    hip.w8a16_free(w8)
    hip.gemm_workspace_free(ws)
    hip.gemv_scratch_free(s)
