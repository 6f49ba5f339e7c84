"""qw4_gemv_argmax_noalloc (no reference counterpart: the argmax head for callers
that cannot allocate) against the existing entry point qw4_gemv_argmax on the
same inputs, bit-exact indices: two calls in a row, the second smaller (a
head-sized M = 9 call on the bf16 skinny kernel, then an M = 1 call on the
integer-MFMA decode kernel), so the second starts from the state the first
left in the shared static scratch; sizes beyond the maximum are rejected. Also:
the first call of the process made under graph capture, then the graph
replayed several times (the entry point records no set-up work, and each
replay resets the keys it used), and an M = 16 call (every key row used)
followed by an M = 1 call."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import host

pytestmark = pytest.mark.gpu


def _gen(hip, N, K, seed):
    import torch

    G = K // 128
    q = torch.empty(K // 8 * N, dtype=torch.int32, device="cuda")
    s = torch.empty(G * N, dtype=torch.int16, device="cuda")
    z = torch.empty(G * N // 8, dtype=torch.int32, device="cuda")
    hip.gen_awq_k(q, s, z, N, K, seed, 7)
    w = hip.awq_alloc_fused(N, K)
    hip.awq_repack_awq_into(w, 0, q, s, z, N, hip.LAYOUT_AWQ_K)
    torch.cuda.synchronize()
    return w


def _want(hip, w, x, M):
    import torch

    scr = hip.gemv_scratch_alloc(5120, 31040, 128, 16)
    idx = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    hip.gemv_argmax_w4a16(idx, w, x, M, scr)
    torch.cuda.synchronize()
    hip.gemv_scratch_free(scr)
    return host(idx, np.int32).copy()


def test_noalloc_first_call_under_capture():
    import torch

    import w4a16_hip as hip

    L = hip.lib()
    hip.tune_decode(0)
    N, K, M = 31040, 5120, 9
    w = _gen(hip, N, K, 5)
    x = torch.empty(M * K, dtype=torch.int16, device="cuda")
    hip.gen_bf16(x, M * K, 0, 905, 0)
    want = _want(hip, w, x, M)
    idx = torch.full((M,), -1, dtype=torch.int32, device="cuda")
    g = torch.cuda.CUDAGraph()
    print("noalloc argmax: first call under capture", flush=True)
    with torch.cuda.graph(g):
        st = L.qw4_gemv_argmax_noalloc(idx.data_ptr(), C.byref(w), x.data_ptr(), M,
                                       torch.cuda.current_stream().cuda_stream)
    assert st == hip.QW4_OK
    for rep in range(3):
        idx.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(idx, np.int32), want), rep
        junk = torch.ones(1 << 20, device="cuda").sum()   # eager work between replays
        torch.cuda.synchronize()
    del g
    hip.awq_free(w)


def test_noalloc_m16_then_m1():
    import torch

    import w4a16_hip as hip

    L = hip.lib()
    hip.tune_decode(0)
    stream = torch.cuda.current_stream().cuda_stream
    for N, K, M, seed in [(4096, 5120, 16, 11), (4096, 5120, 1, 12), (31040, 5120, 16, 13),
                          (5120, 4096, 1, 14)]:
        w = _gen(hip, N, K, seed)
        x = torch.empty(M * K, dtype=torch.int16, device="cuda")
        hip.gen_bf16(x, M * K, 0, 950 + seed, 0)
        want = _want(hip, w, x, M)
        idx = torch.full((M,), -1, dtype=torch.int32, device="cuda")
        print(f"noalloc argmax {N}x{K} M={M}", flush=True)
        assert L.qw4_gemv_argmax_noalloc(idx.data_ptr(), C.byref(w), x.data_ptr(), M,
                                         stream) == hip.QW4_OK
        torch.cuda.synchronize()
        assert np.array_equal(host(idx, np.int32), want), (N, K, M)
        hip.awq_free(w)


def test_noalloc_argmax_matches_scratch_entry():
    import torch

    import w4a16_hip as hip

    L = hip.lib()
    hip.tune_decode(0)
    cases = [(31040, 5120, 9, 1), (4096, 2048, 1, 2)]   # the second call smaller
    ws, xs, want = [], [], []
    scr = hip.gemv_scratch_alloc(5120, 31040, 128, 16)
    for N, K, M, seed in cases:
        w = _gen(hip, N, K, seed)
        x = torch.empty(M * K, dtype=torch.int16, device="cuda")
        hip.gen_bf16(x, M * K, 0, 900 + seed, 0)
        idx = torch.full((M,), -1, dtype=torch.int32, device="cuda")
        hip.gemv_argmax_w4a16(idx, w, x, M, scr)
        torch.cuda.synchronize()
        ws.append(w)
        xs.append(x)
        want.append(host(idx, np.int32).copy())
    hip.gemv_scratch_free(scr)
    stream = torch.cuda.current_stream().cuda_stream
    got = []
    for (N, K, M, seed), w, x in zip(cases, ws, xs):   # two calls in a row
        idx = torch.full((M,), -1, dtype=torch.int32, device="cuda")
        print(f"noalloc argmax {N}x{K} M={M}", flush=True)
        assert L.qw4_gemv_argmax_noalloc(idx.data_ptr(), C.byref(w), x.data_ptr(), M,
                                         stream) == hip.QW4_OK
        got.append(idx)
    torch.cuda.synchronize()
    for (N, K, M, seed), g, r in zip(cases, got, want):
        assert np.array_equal(host(g, np.int32), r), (N, K, M)
        assert np.all((r >= 0) & (r < N))
    # beyond the 16 rows the static keys hold: rejected before any launch
    idx = torch.empty(17, dtype=torch.int32, device="cuda")
    assert L.qw4_gemv_argmax_noalloc(idx.data_ptr(), C.byref(ws[1]), xs[1].data_ptr(), 17,
                                     stream) == hip.QW4_ERR_M
    for w in ws:
        hip.awq_free(w)
