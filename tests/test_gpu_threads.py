"""Host threads launching at once (the reference's lazily initialised statics,
gemv_w4a16.cu:281-297, race; here every per-device cache is filled under
std::call_once or is an atomic): two threads, each on its own stream, run
decode GEMVs, fused steps and verify GEMMs of their own weights through the
C-ABI concurrently from the first launch on; every output must equal the
same call made alone afterwards (bitwise: the kernels are deterministic)."""
import threading

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
    hip.gen_awq_k(q, s, z, N, K, seed, 5)
    w = hip.awq_alloc_fused(N, K)
    hip.awq_repack_awq_into(w, 0, q, s, z, N, hip.LAYOUT_AWQ_K)
    torch.cuda.synchronize()
    return w


def test_two_threads_launch_at_once():
    import torch

    import w4a16_hip as hip

    hip.lib()
    hip.tune_decode(0)
    shapes = [(7168, 5120), (5120, 17408)]
    ws = [_gen(hip, N, K, 11 + i) for i, (N, K) in enumerate(shapes)]
    scr = [hip.gemv_scratch_alloc(17408, 7168, 128, 16) for _ in shapes]
    xs = []
    for i, (N, K) in enumerate(shapes):
        x = torch.empty(9 * K, dtype=torch.int16, device="cuda")
        hip.gen_bf16(x, 9 * K, 0, 300 + i, 0)
        xs.append(x)
    streams = [torch.cuda.Stream() for _ in shapes]
    outs = [[None] * 3 for _ in shapes]
    errors = []
    barrier = threading.Barrier(len(shapes))

    def work(i):
        try:
            N, K = shapes[i]
            ys = [torch.empty(N, dtype=torch.int16, device="cuda"),
                  torch.empty(9 * N, dtype=torch.int16, device="cuda"),
                  torch.empty(N, dtype=torch.float32, device="cuda")]
            barrier.wait()
            with torch.cuda.stream(streams[i]):
                st = streams[i].cuda_stream
                for _ in range(20):
                    hip.gemv_w4a16(ys[0], ws[i], xs[i], scr[i], stream=st)
                    hip.gemm_small_w4a16(ys[1], ws[i], xs[i], 9, scr[i], stream=st)
                    hip.gemv_w4a16_f32(ys[2], ws[i], xs[i], scr[i], stream=st)
            streams[i].synchronize()
            outs[i] = [host(ys[0], np.uint16), host(ys[1], np.uint16), host(ys[2], np.float32)]
        except Exception as e:   # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(shapes))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i, (N, K) in enumerate(shapes):
        y0 = torch.empty(N, dtype=torch.int16, device="cuda")
        y1 = torch.empty(9 * N, dtype=torch.int16, device="cuda")
        y2 = torch.empty(N, dtype=torch.float32, device="cuda")
        hip.gemv_w4a16(y0, ws[i], xs[i], scr[i])
        hip.gemm_small_w4a16(y1, ws[i], xs[i], 9, scr[i])
        hip.gemv_w4a16_f32(y2, ws[i], xs[i], scr[i])
        torch.cuda.synchronize()
        assert np.array_equal(outs[i][0], host(y0, np.uint16)), shapes[i]
        assert np.array_equal(outs[i][1], host(y1, np.uint16)), shapes[i]
        assert np.array_equal(outs[i][2], host(y2, np.float32)), shapes[i]
    for w in ws:
        hip.awq_free(w)
    for s in scr:
        hip.gemv_scratch_free(s)
