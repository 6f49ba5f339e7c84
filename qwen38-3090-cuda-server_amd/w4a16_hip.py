"""Python host binding of libqwen_w4a16.so (the C-ABI in include/qwen_w4a16.h).

The function names mirror the reference's C++ entry points (namespace qwen in
src/kernels/gemv_w4a16.cuh, gemm_w4a16.cuh and elementwise.cuh) so callers and
tests read like the reference's own gates. Device memory and streams come from
torch tensors (plumbing only); every compute call goes through the HIP library,
and there is no fallback: if the library is missing, loading fails loudly.

Errors: the reference prints and aborts; here a non-zero status raises
W4A16Error carrying the status code and message.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqwen_w4a16.so")

QW4_OK = 0
QW4_ERR_NULL = 1
QW4_ERR_SHAPE = 2
QW4_ERR_GROUP = 3
QW4_ERR_M = 4
QW4_ERR_SCRATCH = 5
QW4_ERR_ALIGN = 6
QW4_ERR_HIP = 7
QW4_ERR_NOMEM = 8
QW4_ERR_LAYOUT = 9
QW4_ERR_IO = 10
QW4_ERR_NOTFOUND = 11
LAYOUT_AWQ_K = 1
LAYOUT_AWQ_N = 2

# Every symbol include/qwen_w4a16.h declares.
EXPORTS = (
    "qw4_status_string", "qw4_last_hip_error", "qw4_version", "qw4_weights_bytes",
    "qw4_weights_alloc", "qw4_weights_free", "qw4_repack_ct_into", "qw4_repack_ct",
    "qw4_repack_awq_into", "qw4_dequant_rows", "qw4_scratch_alloc", "qw4_scratch_free",
    "qw4_partial_check", "qw4_choose_splits", "qw4_gemv", "qw4_gemv_f32", "qw4_gemm_small",
    "qw4_gemm_mma", "qw4_gemv_argmax", "qw4_workspace_alloc", "qw4_workspace_free",
    "qw4_gemm", "qw4_argmax", "qw4_argmax_rows", "qw4_gen_bf16", "qw4_gen_awq_k",
    "qw4_stream_read", "qw4_st_open", "qw4_st_open_dir", "qw4_st_close", "qw4_st_count",
    "qw4_st_find", "qw4_st_last_error", "qw4_load_ct_fused",
    "qw4_w8_quantize", "qw4_w8_free", "qw4_w8_bytes", "qw4_w8_dequant_rows", "qw4_w8_gemv",
    "qw4_w8_gemm_small", "qw4_w8_gemv_argmax",
    "qw4_rmsnorm", "qw4_residual_add", "qw4_swiglu", "qw4_gemv_residual", "qw4_gemv_swiglu",
    "qw4_gemv_rmsnorm", "qw4_linear", "qw4_linear_max_t", "qw4_mfma_peak", "qw4_tune_decode",
    "qw4_tune_gemm", "qw4_tune_linear", "qw4_gemv_argmax_noalloc",
    "qw4_quantize_w4a16",
)

# safetensors dtype order (qw4_st_tensor.dtype)
ST_DTYPES = ("BF16", "F16", "F32", "F64", "I8", "U8", "I16", "I32", "I64", "BOOL", "F8_E4M3",
             "F8_E5M2")


class W4A16Error(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        msg = lib().qw4_status_string(status).decode()
        if status in (QW4_ERR_IO, QW4_ERR_NOTFOUND) or (
                status == QW4_ERR_SHAPE and where.startswith(("load_ct_fused", "SafeTensors"))):
            detail = lib().qw4_st_last_error().decode()
            if detail:
                msg += f": {detail}"
        if status == QW4_ERR_HIP:
            msg += f" (hipError {lib().qw4_last_hip_error()})"
        super().__init__(f"{where}: {msg} [status {status}]")


class W4A16Weights(C.Structure):
    """qw4_weights / the reference's W4A16Weights (gemv_w4a16.cuh:50-60)."""
    _fields_ = [("qweight", C.c_void_p), ("scale", C.c_void_p), ("zeros", C.c_void_p),
                ("out_f", C.c_int32), ("in_f", C.c_int32), ("group_size", C.c_int32),
                ("num_groups", C.c_int32)]

    def total_bytes(self) -> int:
        return lib().qw4_weights_bytes(C.byref(self))


class W8A16Weights(C.Structure):
    """qw4_w8_weights / the reference's W8A16Weights (gemv_w4a16.cuh:147-154)."""
    _fields_ = [("qweight", C.c_void_p), ("scale", C.c_void_p),
                ("out_f", C.c_int32), ("in_f", C.c_int32), ("group_size", C.c_int32),
                ("num_groups", C.c_int32)]

    def total_bytes(self) -> int:
        return lib().qw4_w8_bytes(C.byref(self))


class GemvScratch(C.Structure):
    """qw4_scratch / the reference's GemvScratch (gemv_w4a16.cuh:94-104)."""
    _fields_ = [("partial", C.c_void_p), ("counters", C.c_void_p), ("keys", C.c_void_p),
                ("partial_elems", C.c_size_t), ("max_in", C.c_int32), ("max_out", C.c_int32),
                ("max_m", C.c_int32), ("max_tiles", C.c_int32)]


class GemmWorkspace(C.Structure):
    """qw4_workspace / the reference's GemmWorkspace (gemm_w4a16.cuh:30-35)."""
    _fields_ = [("buf", C.c_void_p), ("bytes", C.c_size_t)]


class StTensor(C.Structure):
    """qw4_st_tensor: one tensor of an open safetensors set (host view)."""
    _fields_ = [("dtype", C.c_int32), ("ndim", C.c_int32), ("shape", C.c_int64 * 8),
                ("data", C.c_void_p), ("nbytes", C.c_size_t)]


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} not built: run __graft_entry__.build() "
                          "(python qwen38-3090-cuda-server_amd/build.py)")
    L = C.CDLL(LIB_PATH)
    vp, i, sz, u64 = C.c_void_p, C.c_int, C.c_size_t, C.c_uint64
    W, S, WS = C.POINTER(W4A16Weights), C.POINTER(GemvScratch), C.POINTER(GemmWorkspace)
    W8 = C.POINTER(W8A16Weights)
    sig = {
        "qw4_status_string": ([i], C.c_char_p),
        "qw4_last_hip_error": ([], i),
        "qw4_version": ([], i),
        "qw4_weights_bytes": ([W], sz),
        "qw4_weights_alloc": ([W, i, i, i, vp], i),
        "qw4_weights_free": ([W], i),
        "qw4_repack_ct_into": ([W, i, vp, vp, vp, i, vp], i),
        "qw4_repack_ct": ([W, vp, vp, vp, i, i, i, vp], i),
        "qw4_repack_awq_into": ([W, i, vp, vp, vp, i, i, vp], i),
        "qw4_dequant_rows": ([vp, W, i, i, vp], i),
        "qw4_scratch_alloc": ([S, i, i, i, i], i),
        "qw4_scratch_free": ([S], i),
        "qw4_partial_check": ([S, i, i, i], i),
        "qw4_choose_splits": ([i, i], i),
        "qw4_gemv": ([vp, W, vp, S, vp], i),
        "qw4_gemv_f32": ([vp, W, vp, S, vp], i),
        "qw4_gemm_small": ([vp, W, vp, i, S, vp], i),
        "qw4_gemm_mma": ([vp, W, vp, i, S, vp], i),
        "qw4_gemv_argmax": ([vp, W, vp, i, S, vp], i),
        "qw4_workspace_alloc": ([WS, sz], i),
        "qw4_workspace_free": ([WS], i),
        "qw4_gemm": ([vp, W, vp, i, WS, vp], i),
        "qw4_argmax": ([vp, vp, i, vp, vp], i),
        "qw4_argmax_rows": ([vp, vp, i, i, vp], i),
        "qw4_gen_bf16": ([vp, sz, u64, u64, u64, i, vp], i),
        "qw4_gen_awq_k": ([vp, vp, vp, i, i, u64, u64, vp], i),
        "qw4_stream_read": ([vp, sz, vp, i, vp], i),
        "qw4_st_open": ([C.POINTER(vp), C.POINTER(C.c_char_p), i], i),
        "qw4_st_open_dir": ([C.POINTER(vp), C.c_char_p], i),
        "qw4_st_close": ([vp], i),
        "qw4_st_count": ([vp], i),
        "qw4_st_find": ([vp, C.c_char_p, C.POINTER(StTensor)], i),
        "qw4_st_last_error": ([], C.c_char_p),
        "qw4_load_ct_fused": ([W, vp, C.POINTER(C.c_char_p), i, i, i, vp], i),
        "qw4_w8_quantize": ([W8, vp, i, i, i, vp], i),
        "qw4_w8_free": ([W8], i),
        "qw4_w8_bytes": ([W8], sz),
        "qw4_w8_dequant_rows": ([vp, W8, i, i, vp], i),
        "qw4_w8_gemv": ([vp, W8, vp, S, vp], i),
        "qw4_w8_gemm_small": ([vp, W8, vp, i, S, vp], i),
        "qw4_w8_gemv_argmax": ([vp, W8, vp, i, S, vp], i),
        "qw4_rmsnorm": ([vp, vp, vp, i, i, C.c_float, vp], i),
        "qw4_residual_add": ([vp, vp, sz, vp], i),
        "qw4_swiglu": ([vp, vp, i, i, vp], i),
        "qw4_gemv_residual": ([vp, W, vp, i, S, vp], i),
        "qw4_gemv_swiglu": ([vp, W, vp, i, vp, S, vp], i),
        "qw4_gemv_rmsnorm": ([vp, W, vp, vp, C.c_float, i, vp, S, vp], i),
        "qw4_linear": ([vp, W, vp, i, S, WS, vp], i),
        "qw4_linear_max_t": ([W], i),
        "qw4_tune_decode": ([i, i, i, i, i], i),
        "qw4_mfma_peak": ([vp, i, i, vp], i),
        "qw4_tune_gemm": ([i, i], i),
        "qw4_gemv_argmax_noalloc": ([vp, W, vp, i, vp], i),
        "qw4_quantize_w4a16": ([W, vp, i, i, i, vp], i),
        "qw4_tune_linear": ([i], i),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _chk(status: int, where: str) -> None:
    if status != QW4_OK:
        raise W4A16Error(status, where)


def _ptr(t) -> int | None:
    if t is None:
        return None
    return t.data_ptr() if hasattr(t, "data_ptr") else int(t)


def _need(t, nbytes: int, where: str) -> None:
    """Host-side bounds check before a launch: a torch tensor argument must hold
    at least nbytes (raw integer pointers cannot be checked and are trusted)."""
    if t is not None and hasattr(t, "numel") and hasattr(t, "element_size"):
        have = t.numel() * t.element_size()
        if have < nbytes:
            raise ValueError(f"{where}: buffer holds {have} bytes, needs {nbytes}")


def _stream(stream) -> int | None:
    if stream is None:
        import torch

        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


# ------------------------------------------------------------- weights
def awq_alloc_fused(total_out_f: int, in_f: int, group_size: int = 128, stream=None) -> W4A16Weights:
    """awq_alloc_fused (gemv_w4a16.cuh:81-82)."""
    w = W4A16Weights()
    _chk(lib().qw4_weights_alloc(C.byref(w), total_out_f, in_f, group_size, _stream(stream)),
         "awq_alloc_fused")
    return w


def awq_repack_into(w: W4A16Weights, row_offset: int, packed, scale, zp, out_f: int,
                    stream=None) -> None:
    """awq_repack_into (gemv_w4a16.cuh:83-85): compressed-tensors source tensors."""
    G = w.in_f // 128
    _need(packed, out_f * w.in_f // 2, "awq_repack_into packed")
    _need(scale, out_f * G * 2, "awq_repack_into scale")
    _need(zp, out_f // 8 * G * 4, "awq_repack_into zp")
    _chk(lib().qw4_repack_ct_into(C.byref(w), row_offset, _ptr(packed), _ptr(scale), _ptr(zp),
                                  out_f, _stream(stream)), "awq_repack_into")


def awq_repack(packed, scale, zp, out_f: int, in_f: int, group_size: int = 128,
               stream=None) -> W4A16Weights:
    """awq_repack (gemv_w4a16.cuh:70-75)."""
    G = in_f // group_size if group_size else 0
    _need(packed, out_f * in_f // 2, "awq_repack packed")
    _need(scale, out_f * G * 2, "awq_repack scale")
    _need(zp, out_f // 8 * G * 4, "awq_repack zp")
    w = W4A16Weights()
    _chk(lib().qw4_repack_ct(C.byref(w), _ptr(packed), _ptr(scale), _ptr(zp), out_f, in_f,
                             group_size, _stream(stream)), "awq_repack")
    return w


def awq_repack_awq_into(w: W4A16Weights, row_offset: int, qweight, scales, zeros, out_f: int,
                        layout: int = LAYOUT_AWQ_K, stream=None) -> None:
    """AWQ-order sources (BASELINE layout along K, or AutoAWQ along N)."""
    G = w.in_f // 128
    _need(qweight, out_f * w.in_f // 2, "awq_repack_awq_into qweight")
    _need(scales, out_f * G * 2, "awq_repack_awq_into scales")
    _need(zeros, out_f // 8 * G * 4, "awq_repack_awq_into zeros")
    _chk(lib().qw4_repack_awq_into(C.byref(w), row_offset, _ptr(qweight), _ptr(scales),
                                   _ptr(zeros), out_f, layout, _stream(stream)),
         "awq_repack_awq_into")


def awq_free(w: W4A16Weights) -> None:
    """awq_free (gemv_w4a16.cuh:86)."""
    _chk(lib().qw4_weights_free(C.byref(w)), "awq_free")


def w4a16_dequant_rows(dst, w: W4A16Weights, row0: int, nrows: int, stream=None) -> None:
    """w4a16_dequant_rows (gemm_w4a16.cuh:45-48)."""
    _need(dst, max(nrows, 0) * w.in_f * 2, "w4a16_dequant_rows dst")
    _chk(lib().qw4_dequant_rows(_ptr(dst), C.byref(w), row0, nrows, _stream(stream)),
         "w4a16_dequant_rows")


# ------------------------------------------------------------- scratch
def gemv_scratch_alloc(max_in: int, max_out: int, min_group: int = 128, max_m: int = 1) -> GemvScratch:
    """gemv_scratch_alloc (gemv_w4a16.cuh:106-107)."""
    s = GemvScratch()
    _chk(lib().qw4_scratch_alloc(C.byref(s), max_in, max_out, min_group, max_m),
         "gemv_scratch_alloc")
    return s


def gemv_scratch_free(s: GemvScratch) -> None:
    _chk(lib().qw4_scratch_free(C.byref(s)), "gemv_scratch_free")


def gemv_partial_check(s: GemvScratch, splits: int, out_f: int, M: int) -> None:
    _chk(lib().qw4_partial_check(C.byref(s), splits, out_f, M), "gemv_partial_check")


def gemv_choose_splits(out_f: int, num_groups: int) -> int:
    return lib().qw4_choose_splits(out_f, num_groups)


def gemm_workspace_alloc(nbytes: int = 0) -> GemmWorkspace:
    ws = GemmWorkspace()
    _chk(lib().qw4_workspace_alloc(C.byref(ws), nbytes), "gemm_workspace_alloc")
    return ws


def gemm_workspace_free(ws: GemmWorkspace) -> None:
    _chk(lib().qw4_workspace_free(C.byref(ws)), "gemm_workspace_free")


# ------------------------------------------------------------- compute
def gemv_w4a16(y, w: W4A16Weights, x, s: GemvScratch, stream=None) -> None:
    """gemv_w4a16 (gemv_w4a16.cuh:130-131): y[out] = W @ x, bf16."""
    _need(y, w.out_f * 2, "gemv_w4a16 y")
    _need(x, w.in_f * 2, "gemv_w4a16 x")
    _chk(lib().qw4_gemv(_ptr(y), C.byref(w), _ptr(x), C.byref(s), _stream(stream)), "gemv_w4a16")


def gemv_w4a16_f32(y, w: W4A16Weights, x, s: GemvScratch, stream=None) -> None:
    """gemv_w4a16_f32 (gemv_w4a16.cuh:132-133)."""
    _need(y, w.out_f * 4, "gemv_w4a16_f32 y")
    _need(x, w.in_f * 2, "gemv_w4a16_f32 x")
    _chk(lib().qw4_gemv_f32(_ptr(y), C.byref(w), _ptr(x), C.byref(s), _stream(stream)),
         "gemv_w4a16_f32")


def gemm_small_w4a16(y, w: W4A16Weights, x, M: int, s: GemvScratch, stream=None) -> None:
    """gemm_small_w4a16 (gemv_w4a16.cuh:124-125): Y[M,out] = X[M,in] @ W^T."""
    _need(y, max(M, 0) * w.out_f * 2, "gemm_small_w4a16 y")
    _need(x, max(M, 0) * w.in_f * 2, "gemm_small_w4a16 x")
    _chk(lib().qw4_gemm_small(_ptr(y), C.byref(w), _ptr(x), M, C.byref(s), _stream(stream)),
         "gemm_small_w4a16")


def gemm_mma_w4a16(y, w: W4A16Weights, x, M: int, s: GemvScratch, stream=None) -> None:
    """gemm_mma_w4a16 (gemv_w4a16.cuh:187-188)."""
    _need(y, max(M, 0) * w.out_f * 2, "gemm_mma_w4a16 y")
    _need(x, max(M, 0) * w.in_f * 2, "gemm_mma_w4a16 x")
    _chk(lib().qw4_gemm_mma(_ptr(y), C.byref(w), _ptr(x), M, C.byref(s), _stream(stream)),
         "gemm_mma_w4a16")


def gemv_argmax_w4a16(idx, w: W4A16Weights, x, M: int, s: GemvScratch, stream=None) -> None:
    """lm_head GEMV + fused fp32 row-argmax (model.cu:796-815 + elementwise.cuh:39-43)."""
    _need(idx, max(M, 0) * 4, "gemv_argmax_w4a16 idx")
    _need(x, max(M, 0) * w.in_f * 2, "gemv_argmax_w4a16 x")
    _chk(lib().qw4_gemv_argmax(_ptr(idx), C.byref(w), _ptr(x), M, C.byref(s), _stream(stream)),
         "gemv_argmax_w4a16")


# ------------------------------------------- layer steps either side
def gemv_argmax_w4a16_noalloc(idx, w: W4A16Weights, x, M: int, stream=None) -> None:
    """qw4_gemv_argmax_noalloc: the fused argmax head with the library's static
    scratch (no allocation, no scratch argument; overlapping calls race)."""
    _need(idx, M * 4, "gemv_argmax_w4a16_noalloc idx")
    _need(x, M * w.in_f * 2, "gemv_argmax_w4a16_noalloc x")
    _chk(lib().qw4_gemv_argmax_noalloc(_ptr(idx), C.byref(w), _ptr(x), M, _stream(stream)),
         "gemv_argmax_w4a16_noalloc")


def rmsnorm(out, x, w, rows: int, dim: int, eps: float, stream=None) -> None:
    """rmsnorm (elementwise.cuh:8-13): out = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w))."""
    _need(out, rows * dim * 2, "rmsnorm out")
    _need(x, rows * dim * 2, "rmsnorm x")
    _need(w, dim * 2, "rmsnorm w")
    _chk(lib().qw4_rmsnorm(_ptr(out), _ptr(x), _ptr(w), rows, dim, eps, _stream(stream)),
         "rmsnorm")


def residual_add(out, x, n: int, stream=None) -> None:
    """residual_add (elementwise.cuh:15-17): out[i] = bf16(out[i] + x[i])."""
    _need(out, n * 2, "residual_add out")
    _need(x, n * 2, "residual_add x")
    _chk(lib().qw4_residual_add(_ptr(out), _ptr(x), n, _stream(stream)), "residual_add")


def swiglu(out, fused, rows: int, inter: int, stream=None) -> None:
    """swiglu (elementwise.cuh:19-22): out[r] = bf16(silu(gate[r]) * up[r])."""
    _need(out, rows * inter * 2, "swiglu out")
    _need(fused, rows * 2 * inter * 2, "swiglu fused")
    _chk(lib().qw4_swiglu(_ptr(out), _ptr(fused), rows, inter, _stream(stream)), "swiglu")


def gemv_residual_w4a16(h, w: W4A16Weights, x, M: int, s: GemvScratch, stream=None) -> None:
    """linear then residual_add (model.cu:779-784): h = bf16(h + bf16(x @ W^T))."""
    _need(h, max(M, 0) * w.out_f * 2, "gemv_residual h")
    _need(x, max(M, 0) * w.in_f * 2, "gemv_residual x")
    _chk(lib().qw4_gemv_residual(_ptr(h), C.byref(w), _ptr(x), M, C.byref(s), _stream(stream)),
         "gemv_residual")


def gemv_swiglu_w4a16(y, w: W4A16Weights, x, M: int, s: GemvScratch, tmp=None,
                      stream=None) -> None:
    """linear over a fused [gate | up] weight then swiglu (model.cu:776-778)."""
    _need(y, max(M, 0) * (w.out_f // 2) * 2, "gemv_swiglu y")
    _need(x, max(M, 0) * w.in_f * 2, "gemv_swiglu x")
    if tmp is not None:
        _need(tmp, max(M, 0) * w.out_f * 2, "gemv_swiglu tmp")
    _chk(lib().qw4_gemv_swiglu(_ptr(y), C.byref(w), _ptr(x), M, _ptr(tmp), C.byref(s),
                               _stream(stream)), "gemv_swiglu")


def gemv_rmsnorm_w4a16(y, w: W4A16Weights, h, norm_w, eps: float, M: int, s: GemvScratch,
                       tmp=None, stream=None) -> None:
    """rmsnorm then linear (model.cu:697-700, :773-777)."""
    _need(y, max(M, 0) * w.out_f * 2, "gemv_rmsnorm y")
    _need(h, max(M, 0) * w.in_f * 2, "gemv_rmsnorm h")
    _need(norm_w, w.in_f * 2, "gemv_rmsnorm norm_w")
    if tmp is not None:
        _need(tmp, max(M, 0) * w.in_f * 2, "gemv_rmsnorm tmp")
    _chk(lib().qw4_gemv_rmsnorm(_ptr(y), C.byref(w), _ptr(h), _ptr(norm_w), eps, M, _ptr(tmp),
                                C.byref(s), _stream(stream)), "gemv_rmsnorm")


def linear_w4a16(y, w: W4A16Weights, x, T: int, s: GemvScratch, ws: GemmWorkspace | None = None,
                 stream=None) -> None:
    """linear() with lin_path() (model.cu:522-565, :643-658)."""
    _need(y, max(T, 0) * w.out_f * 2, "linear y")
    _need(x, max(T, 0) * w.in_f * 2, "linear x")
    _chk(lib().qw4_linear(_ptr(y), C.byref(w), _ptr(x), T, C.byref(s),
                          C.byref(ws) if ws is not None else None, _stream(stream)), "linear")


def tune_decode(mode: int = 0, S: int = 0, W: int = 0, D: int = 0, P: int = 0) -> None:
    """Tuning and test override of the skinny launches (qw4_tune_decode): mode 0
    the library's policy, 1 k_rows at M = 1 (D: LDS-DMA depth), 2 k_rows with
    register items (S, W: unit size and waves), 3 k_dec of shape S / W / D,
    4 the policy without staging M > 1 activations in LDS, 5 the policy without
    the group-major M > 1 kernel; P forces k_dec's workgroups (0 = policy)."""
    _chk(lib().qw4_tune_decode(mode, S, W, D, P), "tune_decode")


def tune_gemm(schedule: int = -1, variant: int = 0) -> None:
    """Prefill override (qw4_tune_gemm): schedule -1 cost model, 0 per tile,
    1 stream-K, 2 hybrid, 3 split-K; variant 0 the default 4-wave kernel, 1 8 waves on
    32-row tile halves, 2 8 waves on whole tiles (bitwise-equal results)."""
    _chk(lib().qw4_tune_gemm(schedule, variant), "tune_gemm")


def tune_linear(max_t: int = 0) -> None:
    """qw4_linear crossover override (qw4_tune_linear), 0 = the measured rule."""
    _chk(lib().qw4_tune_linear(max_t), "tune_linear")


def linear_max_t(w: W4A16Weights) -> int:
    """Rows up to which linear() uses 16-row skinny passes for this weight."""
    return lib().qw4_linear_max_t(C.byref(w))


# ------------------------------------------------------- 8-bit lm_head
def quantize_w4a16_raw(src, rows: int, cols: int, group: int = 128, stream=None) -> W4A16Weights:
    """quantize_w4a16_raw (src/model/model.cu:174-186): bf16 [rows][cols] -> INT4
    g128 asymmetric, repacked (the reference's INT4 lm_head)."""
    _need(src, rows * cols * 2, "quantize_w4a16_raw src")
    w = W4A16Weights()
    _chk(lib().qw4_quantize_w4a16(C.byref(w), _ptr(src), rows, cols, group, _stream(stream)),
         "quantize_w4a16_raw")
    return w


def quantize_w8a16(src, out_f: int, in_f: int, group_size: int = 128, stream=None) -> W8A16Weights:
    """quantize_w8a16 (gemv_w4a16.cuh:156-157): bf16 [out_f][in_f] -> 8-bit weights."""
    _need(src, out_f * in_f * 2, "quantize_w8a16 src")
    w = W8A16Weights()
    _chk(lib().qw4_w8_quantize(C.byref(w), _ptr(src), out_f, in_f, group_size, _stream(stream)),
         "quantize_w8a16")
    return w


def w8a16_free(w: W8A16Weights) -> None:
    """w8a16_free (gemv_w4a16.cuh:166)."""
    _chk(lib().qw4_w8_free(C.byref(w)), "w8a16_free")


def w8a16_dequant_rows(dst, w: W8A16Weights, row0: int, nrows: int, stream=None) -> None:
    _need(dst, max(nrows, 0) * w.in_f * 2, "w8a16_dequant_rows dst")
    _chk(lib().qw4_w8_dequant_rows(_ptr(dst), C.byref(w), row0, nrows, _stream(stream)),
         "w8a16_dequant_rows")


def gemv_w8a16(y, w: W8A16Weights, x, s: GemvScratch, stream=None) -> None:
    """gemv_w8a16 (gemv_w4a16.cuh:158-159)."""
    _need(y, w.out_f * 2, "gemv_w8a16 y")
    _need(x, w.in_f * 2, "gemv_w8a16 x")
    _chk(lib().qw4_w8_gemv(_ptr(y), C.byref(w), _ptr(x), C.byref(s), _stream(stream)),
         "gemv_w8a16")


def gemm_small_w8a16(y, w: W8A16Weights, x, M: int, s: GemvScratch, stream=None) -> None:
    """gemm_small_w8a16 (gemv_w4a16.cuh:163-164)."""
    _need(y, max(M, 0) * w.out_f * 2, "gemm_small_w8a16 y")
    _need(x, max(M, 0) * w.in_f * 2, "gemm_small_w8a16 x")
    _chk(lib().qw4_w8_gemm_small(_ptr(y), C.byref(w), _ptr(x), M, C.byref(s), _stream(stream)),
         "gemm_small_w8a16")


def gemv_argmax_w8a16(idx, w: W8A16Weights, x, M: int, s: GemvScratch, stream=None) -> None:
    """8-bit lm_head + fused fp32 row-argmax (model.cu:796-815, lm_head_bits 8)."""
    _need(idx, max(M, 0) * 4, "gemv_argmax_w8a16 idx")
    _need(x, max(M, 0) * w.in_f * 2, "gemv_argmax_w8a16 x")
    _chk(lib().qw4_w8_gemv_argmax(_ptr(idx), C.byref(w), _ptr(x), M, C.byref(s),
                                  _stream(stream)), "gemv_argmax_w8a16")


def gemm_w4a16(Cm, w: W4A16Weights, A, M: int, ws: GemmWorkspace | None = None, stream=None) -> None:
    """gemm_w4a16 (gemm_w4a16.cuh:40-43): C[M,out] = A[M,in] @ W^T."""
    _need(Cm, max(M, 0) * w.out_f * 2, "gemm_w4a16 C")
    _need(A, max(M, 0) * w.in_f * 2, "gemm_w4a16 A")
    wsp = C.byref(ws) if ws is not None else None
    _chk(lib().qw4_gemm(_ptr(Cm), C.byref(w), _ptr(A), M, wsp, _stream(stream)), "gemm_w4a16")


def argmax(out, x, n: int, scratch, stream=None) -> None:
    """argmax (elementwise.cuh:39-40) over bf16 logits."""
    _need(out, 4, "argmax out")
    _need(x, n * 2, "argmax x")
    _need(scratch, 512 * 4, "argmax scratch")
    _chk(lib().qw4_argmax(_ptr(out), _ptr(x), n, _ptr(scratch), _stream(stream)), "argmax")


def argmax_rows(out, x, rows: int, n: int, stream=None) -> None:
    """argmax_rows (elementwise.cuh:41-43)."""
    _need(out, rows * 4, "argmax_rows out")
    _need(x, rows * n * 2, "argmax_rows x")
    _chk(lib().qw4_argmax_rows(_ptr(out), _ptr(x), rows, n, _stream(stream)), "argmax_rows")


# ------------------------------------------------------ synthetic inputs
def gen_bf16(out, count: int, seed: int, stream_id: int, kind: int, offset: int = 0,
             stream=None) -> None:
    _need(out, count * 2, "gen_bf16 out")
    _chk(lib().qw4_gen_bf16(_ptr(out), count, seed, stream_id, offset, kind, _stream(stream)),
         "gen_bf16")


def gen_awq_k(qweight, scales, zeros, out_f: int, in_f: int, seed: int, tensor: int,
              stream=None) -> None:
    G = in_f // 128
    _need(qweight, in_f // 8 * out_f * 4, "gen_awq_k qweight")
    _need(scales, G * out_f * 2, "gen_awq_k scales")
    _need(zeros, G * out_f // 8 * 4, "gen_awq_k zeros")
    _chk(lib().qw4_gen_awq_k(_ptr(qweight), _ptr(scales), _ptr(zeros), out_f, in_f, seed,
                             tensor, _stream(stream)), "gen_awq_k")


def mfma_peak(sink, blocks: int, iters: int, stream=None) -> None:
    """MFMA microbenchmark: blocks x 4 waves x iters x 8 bf16 32x32x16 MFMAs."""
    _need(sink, blocks * 4, "mfma_peak sink")
    _chk(lib().qw4_mfma_peak(_ptr(sink), blocks, iters, _stream(stream)), "mfma_peak")


def stream_read(src, nbytes: int, sink, blocks: int, stream=None) -> None:
    """Streaming-read microbenchmark kernel (HBM read bandwidth denominator)."""
    _need(src, nbytes, "stream_read src")
    _need(sink, blocks * 4, "stream_read sink")
    _chk(lib().qw4_stream_read(_ptr(src), nbytes, _ptr(sink), blocks, _stream(stream)),
         "stream_read")


# ------------------------------------------------------------ checkpoints
class SafeTensors:
    """The reference's qwen::SafeTensors (src/loader/safetensors.h:44-75) over
    the C-ABI: files are mmap'd by the library; get() returns a numpy view of
    the mapping (valid until close())."""

    def __init__(self, paths=None, dir=None):
        self._h = C.c_void_p()
        if dir is not None:
            _chk(lib().qw4_st_open_dir(C.byref(self._h), dir.encode()), "SafeTensors.open_dir")
        else:
            arr = (C.c_char_p * len(paths))(*[p.encode() for p in paths])
            _chk(lib().qw4_st_open(C.byref(self._h), arr, len(paths)), "SafeTensors.open_files")

    def close(self) -> None:
        if self._h:
            lib().qw4_st_close(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return lib().qw4_st_count(self._h)

    def info(self, name: str) -> StTensor:
        t = StTensor()
        _chk(lib().qw4_st_find(self._h, name.encode(), C.byref(t)), f"SafeTensors.find({name})")
        return t

    def has(self, name: str) -> bool:
        t = StTensor()
        return lib().qw4_st_find(self._h, name.encode(), C.byref(t)) == QW4_OK

    def get(self, name: str):
        import numpy as np

        t = self.info(name)
        np_dt = {"BF16": np.uint16, "F16": np.float16, "F32": np.float32, "F64": np.float64,
                 "I8": np.int8, "U8": np.uint8, "I16": np.int16, "I32": np.int32,
                 "I64": np.int64, "BOOL": np.bool_, "F8_E4M3": np.uint8,
                 "F8_E5M2": np.uint8}[ST_DTYPES[t.dtype]]
        shape = tuple(t.shape[k] for k in range(t.ndim))
        buf = (C.c_uint8 * t.nbytes).from_address(t.data) if t.nbytes else b""
        return np.frombuffer(buf, dtype=np_dt).reshape(shape)

    def dtype(self, name: str) -> str:
        return ST_DTYPES[self.info(name).dtype]

    def load_ct_fused(self, prefixes, in_f: int, group_size: int = 128, stream=None) -> W4A16Weights:
        """fuse() (src/model/model.cu:103-128): repack the compressed-tensors
        projections `prefixes` into one W4A16 tensor, rows in order."""
        w = W4A16Weights()
        arr = (C.c_char_p * len(prefixes))(*[p.encode() for p in prefixes])
        _chk(lib().qw4_load_ct_fused(C.byref(w), self._h, arr, len(prefixes), in_f, group_size,
                                     _stream(stream)), "load_ct_fused")
        return w
