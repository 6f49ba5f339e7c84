"""Helpers shared by the GPU tests: move oracle arrays to the device and build
repacked weights through the C-ABI."""
from __future__ import annotations

import numpy as np

_TORCH_VIEW = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32,
               np.dtype(np.int32): np.int32, np.dtype(np.uint8): np.uint8,
               np.dtype(np.float32): np.float32}


def dev(a: np.ndarray):
    import torch

    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(_TORCH_VIEW[a.dtype]).copy()).cuda()


def host(t, dtype) -> np.ndarray:
    return t.detach().cpu().numpy().view(dtype)


def empty(shape, dtype):
    import torch

    tdt = {np.uint16: torch.int16, np.uint32: torch.int32, np.int32: torch.int32,
           np.float32: torch.float32, np.uint8: torch.uint8}[dtype]
    return torch.empty(shape, dtype=tdt, device="cuda")


def repack_from_logical(hip, orc, q, zp, s, layout: str = "ct"):
    """Upload one logical tensor in the given source layout and repack it."""
    N, K = q.shape
    if layout == "ct":
        p, sc, z = orc.pack_ct(q, zp, s)
        bufs = (dev(p), dev(sc), dev(z))
        w = hip.awq_repack(*bufs, N, K)
    else:
        pack = orc.pack_awq_k if layout == "awq_k" else orc.pack_awq_n
        p, sc, z = pack(q, zp, s)
        bufs = (dev(p), dev(sc), dev(z))
        w = hip.awq_alloc_fused(N, K)
        hip.awq_repack_awq_into(w, 0, *bufs, N,
                                hip.LAYOUT_AWQ_K if layout == "awq_k" else hip.LAYOUT_AWQ_N)
    import torch

    torch.cuda.synchronize()
    return w


def weights_buffers(w, N: int, K: int):
    """Copy the three repacked device buffers back to host (for layout checks)."""
    import ctypes as C

    import torch

    G = K // 128
    out = []
    for ptr, n in ((w.qweight, N * K // 2), (w.scale, N * G * 5 // 2), (w.zeros, N * G // 2)):
        buf = torch.empty(n, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        hipMemcpy = C.CDLL("libamdhip64.so").hipMemcpy
        hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        assert hipMemcpy(buf.data_ptr(), ptr, n, 3) == 0   # device to device
        torch.cuda.synchronize()
        out.append(buf.cpu().numpy())
    return out


def download(ptr: int, nbytes: int) -> np.ndarray:
    """Copy nbytes of device memory at a raw pointer to a host uint8 array."""
    import ctypes as C

    import torch

    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    hipMemcpy = C.CDLL("libamdhip64.so").hipMemcpy
    hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    assert hipMemcpy(buf.data_ptr(), ptr, nbytes, 3) == 0   # device to device
    torch.cuda.synchronize()
    return buf.cpu().numpy()
