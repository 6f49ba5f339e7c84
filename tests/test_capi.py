"""The C-ABI library loads, exports every symbol include/qwen_w4a16.h declares,
and rejects bad arguments with status codes before touching the GPU (CPU only:
no call here launches work)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qwen_w4a16.h")


@pytest.fixture(scope="module")
def hip():
    import w4a16_hip

    w4a16_hip.lib()
    return w4a16_hip


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qw4_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree(hip):
    assert declared_functions() == sorted(hip.EXPORTS)


def test_every_declared_symbol_exported(hip):
    L = C.CDLL(hip.LIB_PATH)
    for name in declared_functions():
        assert hasattr(L, name), name


def test_status_strings(hip):
    L = hip.lib()
    for code in range(10):
        assert L.qw4_status_string(code)
    assert L.qw4_status_string(0) == b"ok"


def _fake_weights(hip, out_f=128, in_f=512, group=128):
    w = hip.W4A16Weights()
    w.qweight, w.scale, w.zeros = 0x1000, 0x2000, 0x3000   # never dereferenced
    w.out_f, w.in_f, w.group_size, w.num_groups = out_f, in_f, group, in_f // group
    return w


def _fake_scratch(hip, max_m=16, tiles=4):
    s = hip.GemvScratch()
    s.partial, s.counters, s.keys = 0x4000, 0x5000, 0x6000
    s.partial_elems, s.max_in, s.max_out, s.max_m, s.max_tiles = 1 << 20, 512, 256, max_m, tiles
    return s


def test_argument_errors_before_any_launch(hip):
    L = hip.lib()
    w, s = _fake_weights(hip), _fake_scratch(hip)
    x, y = C.c_void_p(0x10000), C.c_void_p(0x20000)
    # M out of range (reference: gemv_w4a16.cu:429 aborts on M outside 2..16)
    assert L.qw4_gemm_small(y, C.byref(w), x, 17, C.byref(s), None) == hip.QW4_ERR_M
    assert L.qw4_gemm_small(y, C.byref(w), x, 0, C.byref(s), None) == hip.QW4_ERR_M
    assert L.qw4_gemv_argmax(y, C.byref(w), x, 17, C.byref(s), None) == hip.QW4_ERR_M
    # group other than 128 (reference: gemv_w4a16.cu:392 aborts)
    wg = _fake_weights(hip, group=64)
    assert L.qw4_gemv(y, C.byref(wg), x, C.byref(s), None) == hip.QW4_ERR_GROUP
    # shapes the layout cannot hold
    assert L.qw4_gemv(y, C.byref(_fake_weights(hip, out_f=96)), x, C.byref(s), None) == hip.QW4_ERR_SHAPE
    bad_k = _fake_weights(hip, in_f=640)
    bad_k.in_f = 600                       # not a whole number of 128-wide groups
    assert L.qw4_gemv(y, C.byref(bad_k), x, C.byref(s), None) == hip.QW4_ERR_SHAPE
    bad_g = _fake_weights(hip, in_f=640)
    bad_g.num_groups = 4                   # inconsistent with in_f
    assert L.qw4_gemv(y, C.byref(bad_g), x, C.byref(s), None) == hip.QW4_ERR_SHAPE
    # scratch too small for the output rows / M (reference: gemv_partial_check aborts)
    small = _fake_scratch(hip, max_m=4, tiles=1)
    assert L.qw4_gemv(y, C.byref(w), x, C.byref(small), None) == hip.QW4_ERR_SCRATCH
    assert L.qw4_gemm_small(y, C.byref(w), x, 9, C.byref(_fake_scratch(hip, max_m=4)), None) == hip.QW4_ERR_SCRATCH
    # misaligned activations
    assert L.qw4_gemv(y, C.byref(w), C.c_void_p(0x10002), C.byref(s), None) == hip.QW4_ERR_ALIGN
    # null pointers
    assert L.qw4_gemv(None, C.byref(w), x, C.byref(s), None) == hip.QW4_ERR_NULL
    assert L.qw4_gemm(y, C.byref(w), x, 0, None, None) == hip.QW4_ERR_M
    assert L.qw4_repack_ct_into(C.byref(w), 32, x, x, x, 64, None) == hip.QW4_ERR_SHAPE   # offset % 64
    assert L.qw4_repack_ct_into(C.byref(w), 64, x, x, x, 128, None) == hip.QW4_ERR_SHAPE  # overflow
    assert L.qw4_repack_awq_into(C.byref(w), 0, x, x, x, 128, 7, None) == hip.QW4_ERR_LAYOUT
    assert L.qw4_dequant_rows(y, C.byref(w), 100, 64, None) == hip.QW4_ERR_SHAPE
    assert L.qw4_argmax_rows(y, x, 1, 0, None) == hip.QW4_ERR_SHAPE
    assert L.qw4_partial_check(C.byref(small), 4, 128, 1) == hip.QW4_ERR_SCRATCH


def test_python_binding_raises(hip):
    w, s = _fake_weights(hip), _fake_scratch(hip)
    with pytest.raises(hip.W4A16Error) as e:
        hip.gemm_small_w4a16(0x20000, w, 0x10000, 17, s, stream=0)
    assert e.value.status == hip.QW4_ERR_M


def test_choose_splits(hip):
    # whole units per workgroup: no output is split across workgroups
    for n, g in ((248320, 40), (5120, 40), (7168, 40), (5120, 32), (5120, 136), (34816, 40),
                 (64, 4), (64, 136)):
        assert hip.gemv_choose_splits(n, g) == 1


def test_cpp_layer_exports_every_declared_function(hip):
    """include/qwen_w4a16.hpp (the reference-compatible namespace qwen layer):
    every declared function is defined in the library."""
    import subprocess

    text = re.sub(r"//.*", "", open(os.path.join(ROOT, "include", "qwen_w4a16.hpp")).read())
    names = set(re.findall(r"^(?:void|int|size_t)\s+([a-z_0-9]+)\s*\(", text, flags=re.M))
    out = subprocess.run(["nm", "-DC", hip.LIB_PATH], capture_output=True, text=True).stdout
    defined = set(re.findall(r" T qwen::([a-z_0-9]+)\(", out))
    assert len(names) >= 20 and names <= defined, names - defined


def test_linear_threshold_by_weight_size(hip):
    """linear()'s skinny/prefill crossover per weight (host-only call): the
    model's projections get 48 (gate|up), 64 (down), 96 (qkv), 112 (o_proj);
    qw4_tune_linear overrides it (the reference's QWEN_MMA_MAX_T)."""
    hip.tune_linear(0)
    want = {(34816, 5120): 48, (5120, 17408): 64, (7168, 5120): 96, (5120, 4096): 112}
    for (n, k), t in want.items():
        w = hip.W4A16Weights()
        w.out_f, w.in_f, w.group_size, w.num_groups = n, k, 128, k // 128
        assert hip.linear_max_t(w) == t, (n, k)
    hip.tune_linear(33)
    try:
        assert hip.linear_max_t(w) == 33
    finally:
        hip.tune_linear(0)
    assert hip.linear_max_t(w) == want[(n, k)]


def test_host_paths_from_many_threads(hip):
    """The host-side launch policy and argument checks called from many threads
    at once (ctypes releases the GIL, so the calls overlap): every thread gets
    the single-threaded answers. The per-device caches behind them are filled
    under std::call_once or are atomics (the reference's lazy statics,
    gemv_w4a16.cu:281-297, would race here)."""
    import threading

    L = hip.lib()
    hip.tune_linear(0)
    shapes = [(34816, 5120), (5120, 17408), (7168, 5120), (5120, 4096)]

    def answers():
        out = []
        for n, k in shapes:
            w = hip.W4A16Weights()
            w.out_f, w.in_f, w.group_size, w.num_groups = n, k, 128, k // 128
            out.append(hip.linear_max_t(w))
            out.append(hip.gemv_choose_splits(n, k // 128))
        w, s = _fake_weights(hip), _fake_scratch(hip)
        x, y = C.c_void_p(0x10000), C.c_void_p(0x20000)
        out.append(L.qw4_gemm_small(y, C.byref(w), x, 17, C.byref(s), None))
        out.append(L.qw4_gemv(y, C.byref(_fake_weights(hip, group=64)), x, C.byref(s), None))
        out.append(L.qw4_gemv(y, C.byref(w), C.c_void_p(0x10002), C.byref(s), None))
        out.append(L.qw4_status_string(hip.QW4_ERR_SHAPE))
        return out

    want = answers()
    got, errors = [None] * 16, []
    start = threading.Barrier(16)

    def work(i):
        try:
            start.wait()
            for _ in range(50):
                r = answers()
                if r != want:
                    got[i] = r
                    return
            got[i] = want
        except Exception as e:   # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(i,)) for i in range(16)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert all(g == want for g in got), got


def test_weights_beyond_32bit_offsets_refused(hip):
    """The skinny kernels address packed weights through 32-bit buffer offsets:
    a tensor of 4 GiB or more of packed words is refused before any launch
    (QW4_ERR_SHAPE), and one just below the limit passes the size check (it
    then fails on the scratch capacity, still before a launch)."""
    L = hip.lib()
    x, y = C.c_void_p(0x10000), C.c_void_p(0x20000)
    big = _fake_weights(hip, out_f=131072, in_f=65536)            # 4 GiB of packed words
    s = _fake_scratch(hip, tiles=131072 // 64)
    s.max_in, s.max_out = 65536, 131072
    assert L.qw4_gemv(y, C.byref(big), x, C.byref(s), None) == hip.QW4_ERR_SHAPE
    assert L.qw4_gemm_small(y, C.byref(big), x, 9, C.byref(s), None) == hip.QW4_ERR_SHAPE
    below = _fake_weights(hip, out_f=131072 - 64, in_f=65536)
    small = _fake_scratch(hip, tiles=1)
    assert L.qw4_gemv(y, C.byref(below), x, C.byref(small), None) == hip.QW4_ERR_SCRATCH
