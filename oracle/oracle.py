"""ctypes binding of the CPU oracle (oracle.c). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker. The product library never imports it.

Array conventions are the logical tensor of oracle.h:
  q  uint8 [N, K]   stored nibble 0..15
  zp uint8 [N, G]   stored nibble 0..15
  s  uint16 [N, G]  bf16 bits
  x  uint16 [M, K]  bf16 bits
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libref_unpack.so")

_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")

_lib = None


def build() -> None:
    """Compile liboracle.so (and oracle/_ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)
    if os.path.exists("/root/reference/src/loader/w4a16_unpack.h"):
        subprocess.run(["make", "-s", "-C", _HERE, "ref"], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = C.CDLL(_LIB_PATH)
    sz, i, u64 = C.c_size_t, C.c_int, C.c_uint64
    L.or_gen_u4.argtypes = [_u8p, sz, u64, u64, u64]
    L.or_gen_bf16.argtypes = [_u16p, sz, u64, u64, u64, i]
    L.or_mix64.argtypes = [u64]
    L.or_mix64.restype = u64
    L.or_key.argtypes = [u64, u64]
    L.or_key.restype = u64
    L.or_normal.argtypes = [u64, u64]
    L.or_normal.restype = C.c_float
    for name in ("or_pack_ct", "or_pack_awq_k", "or_pack_awq_n"):
        getattr(L, name).argtypes = [_u8p, _u8p, _u16p, i, i, i, _u32p, _u16p, _u32p]
    for name in ("or_unpack_ct", "or_unpack_awq_k", "or_unpack_awq_n"):
        getattr(L, name).argtypes = [_u32p, _u16p, _u32p, i, i, i, _u8p, _u8p, _u16p]
    L.or_ct_q.argtypes = [_u32p, C.c_int64, C.c_int64, C.c_int64]
    L.or_ct_q.restype = C.c_int32
    L.or_ct_zp.argtypes = [_u32p, C.c_int64, C.c_int64, C.c_int64]
    L.or_ct_zp.restype = C.c_int32
    L.or_dequant_f32.argtypes = [_u8p, _u8p, _u16p, i, i, i, i, i, _f32p]
    L.or_dequant_bf16.argtypes = [_u8p, _u8p, _u16p, i, i, i, i, i, _u16p]
    L.or_matmul_f64.argtypes = [_u16p, i, _u8p, _u8p, _u16p, i, i, i, _f64p, i]
    L.or_matmul_bf16w_f64.argtypes = [_u16p, i, _u8p, _u8p, _u16p, i, i, i, _f64p, i]
    L.or_cpu_w4a16_matmul.argtypes = [_u16p, i, _u32p, _u16p, _u32p, i, i, i, _u16p, i]
    L.or_cpu_w4a16_matmul.restype = i
    L.or_argmax_rows_f64.argtypes = [_f64p, i, i, _i32p, _f64p]
    L.or_argmax_rows_f32.argtypes = [_f32p, i, i, _i32p]
    L.or_argmax_rows_bf16.argtypes = [_u16p, i, i, _i32p]
    L.or_w8_quantize.argtypes = [_u16p, i, i, i, _i8p, _u16p]
    L.or_quant_i4.argtypes = [_u16p, i, i, i, _u32p, _u16p, _u32p]
    L.or_w8_matmul_f64.argtypes = [_u16p, i, _i8p, _u16p, i, i, i, _f64p, i]
    L.or_f32_to_bf16.argtypes = [C.c_float]
    L.or_f32_to_bf16.restype = C.c_uint16
    _lib = L
    return L


def ref_lib():
    """The reference's own w4a16_unpack.h compiled into oracle/_ref (or None)."""
    if not os.path.exists(_REF_PATH):
        return None
    L = C.CDLL(_REF_PATH)
    L.ref_w4_q.argtypes = [_u32p, C.c_int64, C.c_int64, C.c_int64]
    L.ref_w4_q.restype = C.c_int32
    L.ref_w4_zp.argtypes = [_u32p, C.c_int64, C.c_int64, C.c_int64]
    L.ref_w4_zp.restype = C.c_int32
    return L


def nthreads() -> int:
    try:
        return max(1, min(len(os.sched_getaffinity(0)), 16))
    except AttributeError:  # pragma: no cover
        return max(1, min(os.cpu_count() or 1, 16))


# ------------------------------------------------------------------ bf16
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """RNE (tests/gate_gemv.cu:23-29), vectorised; finite inputs."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u >> 16) & 1
    return ((u + 0x7FFF + r) >> 16).astype(np.uint16)


# ------------------------------------------------------------- generator
def gen_u4(count: int, seed: int, stream: int, offset: int = 0) -> np.ndarray:
    out = np.empty(count, np.uint8)
    lib().or_gen_u4(out, count, seed, stream, offset)
    return out


def gen_bf16(count: int, seed: int, stream: int, kind: int, offset: int = 0) -> np.ndarray:
    out = np.empty(count, np.uint16)
    lib().or_gen_bf16(out, count, seed, stream, offset, kind)
    return out


STREAM_Q, STREAM_ZP, STREAM_S, STREAM_X = 0, 1, 2, 3


def stream_id(tensor: int, kind: int) -> int:
    """Stream numbering shared with the HIP generator: tensor * 8 + kind."""
    return tensor * 8 + kind


def gen_weights(N: int, K: int, group: int = 128, seed: int = 0, tensor: int = 0):
    G = K // group
    q = gen_u4(N * K, seed, stream_id(tensor, STREAM_Q)).reshape(N, K)
    zp = gen_u4(N * G, seed, stream_id(tensor, STREAM_ZP)).reshape(N, G)
    s = gen_bf16(N * G, seed, stream_id(tensor, STREAM_S), 1).reshape(N, G)
    return q, zp, s


def gen_x(M: int, K: int, seed: int = 0, tensor: int = 0) -> np.ndarray:
    return gen_bf16(M * K, seed, stream_id(tensor, STREAM_X), 0).reshape(M, K)


# --------------------------------------------------------------- layouts
def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def pack_ct(q, zp, s, group=128):
    N, K = q.shape
    G = K // group
    packed = np.empty((N, K // 8), np.uint32)
    scale = np.empty((N, G), np.uint16)
    zpw = np.empty((N // 8, G), np.uint32)
    lib().or_pack_ct(_c(q, np.uint8), _c(zp, np.uint8), _c(s, np.uint16), N, K, group,
                     packed, scale, zpw)
    return packed, scale, zpw


def unpack_ct(packed, scale, zpw, N, K, group=128):
    G = K // group
    q = np.empty((N, K), np.uint8)
    zp = np.empty((N, G), np.uint8)
    s = np.empty((N, G), np.uint16)
    lib().or_unpack_ct(_c(packed, np.uint32), _c(scale, np.uint16), _c(zpw, np.uint32),
                       N, K, group, q, zp, s)
    return q, zp, s


def pack_awq_k(q, zp, s, group=128):
    N, K = q.shape
    G = K // group
    qw = np.empty((K // 8, N), np.uint32)
    sc = np.empty((G, N), np.uint16)
    zw = np.empty((G, N // 8), np.uint32)
    lib().or_pack_awq_k(_c(q, np.uint8), _c(zp, np.uint8), _c(s, np.uint16), N, K, group,
                        qw, sc, zw)
    return qw, sc, zw


def unpack_awq_k(qw, sc, zw, N, K, group=128):
    G = K // group
    q = np.empty((N, K), np.uint8)
    zp = np.empty((N, G), np.uint8)
    s = np.empty((N, G), np.uint16)
    lib().or_unpack_awq_k(_c(qw, np.uint32), _c(sc, np.uint16), _c(zw, np.uint32),
                          N, K, group, q, zp, s)
    return q, zp, s


def pack_awq_n(q, zp, s, group=128):
    N, K = q.shape
    G = K // group
    qw = np.empty((K, N // 8), np.uint32)
    sc = np.empty((G, N), np.uint16)
    zw = np.empty((G, N // 8), np.uint32)
    lib().or_pack_awq_n(_c(q, np.uint8), _c(zp, np.uint8), _c(s, np.uint16), N, K, group,
                        qw, sc, zw)
    return qw, sc, zw


def unpack_awq_n(qw, sc, zw, N, K, group=128):
    G = K // group
    q = np.empty((N, K), np.uint8)
    zp = np.empty((N, G), np.uint8)
    s = np.empty((N, G), np.uint16)
    lib().or_unpack_awq_n(_c(qw, np.uint32), _c(sc, np.uint16), _c(zw, np.uint32),
                          N, K, group, q, zp, s)
    return q, zp, s


# --------------------------------------------------------------- dequant
def dequant_f32(q, zp, s, group=128, row0=0, nrows=None):
    N, K = q.shape
    nrows = N - row0 if nrows is None else nrows
    w = np.empty((nrows, K), np.float32)
    lib().or_dequant_f32(_c(q, np.uint8), _c(zp, np.uint8), _c(s, np.uint16), N, K, group,
                         row0, nrows, w)
    return w


def dequant_bf16(q, zp, s, group=128, row0=0, nrows=None):
    N, K = q.shape
    nrows = N - row0 if nrows is None else nrows
    w = np.empty((nrows, K), np.uint16)
    lib().or_dequant_bf16(_c(q, np.uint8), _c(zp, np.uint8), _c(s, np.uint16), N, K, group,
                          row0, nrows, w)
    return w


# ---------------------------------------------------------------- matmul
def matmul_f64(x, q, zp, s, group=128, round_w=False, threads=None):
    x = _c(np.atleast_2d(x), np.uint16)
    M, K = x.shape
    N = q.shape[0]
    y = np.empty((M, N), np.float64)
    fn = lib().or_matmul_bf16w_f64 if round_w else lib().or_matmul_f64
    fn(x, M, _c(q, np.uint8), _c(zp, np.uint8), _c(s, np.uint16), N, K, group, y,
       threads or nthreads())
    return y


def quant_i4(w_bf16, group=128):
    """INT4 g128 asymmetric quantizer (k_quant_i4, src/model/model.cu:140-172):
    bf16 [N][K] -> compressed-tensors tensors (packed u32 [N][K/8], scale bf16
    bits [N][G], zero points u32 [N/8][G]; nibbles 0..15)."""
    w = _c(w_bf16, np.uint16)
    N, K = w.shape
    G = K // group
    packed = np.empty((N, K // 8), np.uint32)
    scale = np.empty((N, G), np.uint16)
    zp = np.empty((N // 8, G), np.uint32)
    lib().or_quant_i4(w, N, K, group, packed, scale, zp)
    return packed, scale, zp


def w8_quantize(w_bf16, group=128):
    """W8A16 quantizer (k_quant_w8, gemv_w4a16.cu:478-495): bf16 [N][K] ->
    (q int8 [N][K], s bf16 bits [N][G])."""
    w = _c(w_bf16, np.uint16)
    N, K = w.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((N, K // group), np.uint16)
    lib().or_w8_quantize(w, N, K, group, q, s)
    return q, s


def w8_matmul_f64(x, q, s, group=128, threads=None):
    """fp64 y = x @ (q * s)^T for W8A16 weights."""
    x = _c(np.atleast_2d(x), np.uint16)
    M, K = x.shape
    N = q.shape[0]
    y = np.empty((M, N), np.float64)
    lib().or_w8_matmul_f64(x, M, _c(q, np.int8), _c(s, np.uint16), N, K, group, y,
                           threads or nthreads())
    return y


def cpu_w4a16_matmul(x, packed, scale, zpw, N, K, group=128, threads=None):
    """CPU baseline over A0 tensors; returns (y_bf16, threads_used)."""
    x = _c(np.atleast_2d(x), np.uint16)
    M = x.shape[0]
    y = np.empty((M, N), np.uint16)
    used = lib().or_cpu_w4a16_matmul(x, M, _c(packed, np.uint32), _c(scale, np.uint16),
                                     _c(zpw, np.uint32), N, K, group, y,
                                     threads or nthreads())
    return y, used


def argmax_rows_f64(v):
    v = _c(np.atleast_2d(v), np.float64)
    rows, n = v.shape
    idx = np.empty(rows, np.int32)
    margin = np.empty(rows, np.float64)
    lib().or_argmax_rows_f64(v, rows, n, idx, margin)
    return idx, margin


def argmax_rows_f32(v):
    v = _c(np.atleast_2d(v), np.float32)
    rows, n = v.shape
    idx = np.empty(rows, np.int32)
    lib().or_argmax_rows_f32(v, rows, n, idx)
    return idx


def argmax_rows_bf16(v):
    v = _c(np.atleast_2d(v), np.uint16)
    rows, n = v.shape
    idx = np.empty(rows, np.int32)
    lib().or_argmax_rows_bf16(v, rows, n, idx)
    return idx


# ------------------------------------------------- layer steps either side
# numpy restatements of the reference's elementwise kernels; bf16 in/out as
# uint16 bits, fp32 arithmetic as the reference does it.
def rmsnorm_bf16(x, w, eps):
    """src/kernels/elementwise.cu:8-31: per row, inv = rsqrt(sum(x^2) / dim + eps)
    (fp32 sum; here accumulated in float64, then rounded to fp32), then
    bf16(x * inv * (1 + w)) in fp32."""
    xf = bf16_to_f32(np.atleast_2d(x))
    wf = bf16_to_f32(np.asarray(w)).astype(np.float32)
    ss = np.sum(xf.astype(np.float64) ** 2, axis=1).astype(np.float32)
    inv = (np.float32(1.0) / np.sqrt(ss / np.float32(xf.shape[1]) + np.float32(eps))).astype(np.float32)
    out = (xf * inv[:, None]).astype(np.float32) * (np.float32(1.0) + wf)[None, :]
    return f32_to_bf16(out.astype(np.float32))


def swiglu_bf16(fused, inter):
    """src/kernels/elementwise.cu:40-49: bf16(g / (1 + exp(-g)) * u), fp32."""
    f = bf16_to_f32(np.atleast_2d(fused)).astype(np.float32)
    g, u = f[:, :inter], f[:, inter:2 * inter]
    with np.errstate(over="ignore"):
        out = (g / (np.float32(1.0) + np.exp(-g))) * u
    return f32_to_bf16(out.astype(np.float32))


def residual_add_bf16(out, x):
    """src/kernels/elementwise.cu:34-37: bf16(out + x) in fp32."""
    return f32_to_bf16((bf16_to_f32(out) + bf16_to_f32(x)).astype(np.float32))


# ------------------------------------------------------------- tolerances
def parity_metrics(y_bf16: np.ndarray, ref: np.ndarray) -> dict:
    """max-rel = max|y - ref| / max|ref| against the unrounded reference
    (tests/gate_gemv.cu:115, tests/gate_gemm.cu:91); mean-abs against the
    bf16-rounded reference and, for transparency, against the unrounded one."""
    y = bf16_to_f32(y_bf16).astype(np.float64)
    ref = np.asarray(ref, np.float64)
    ref_b = bf16_to_f32(f32_to_bf16(ref.astype(np.float32))).astype(np.float64)
    mx = float(np.max(np.abs(ref))) if ref.size else 0.0
    return {
        "max_rel": float(np.max(np.abs(y - ref))) / mx if mx > 0 else 0.0,
        "mean_abs_vs_bf16_ref": float(np.mean(np.abs(y - ref_b))) if ref.size else 0.0,
        "mean_abs_vs_ref": float(np.mean(np.abs(y - ref))) if ref.size else 0.0,
    }
