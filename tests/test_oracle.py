"""Pins the CPU oracle before anything is checked against it (CPU only).

Each test anchors an oracle function on something other than the oracle's own
formula: the reference's committed compressed-tensors fixtures, the reference's
own unpack header compiled into oracle/_ref, hand-computed known answers, closed
forms, or an independent numpy brute force.
"""
import json
import os
import struct

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden")


# --------------------------------------------------------------------- bf16
def test_bf16_rne_known_answers(orc):
    f = np.array([1.0, 1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, -2.5, 65280.0, 1e-4], np.float32)
    got = orc.f32_to_bf16(f)
    # 1+2^-8 is a tie -> even (0x3f80); 1+3*2^-8 is a tie -> even (0x3f82)
    assert list(got[:5]) == [0x3F80, 0x3F80, 0x3F82, 0xC020, 0x477F]
    # 1e-4 = 0x38D1B717 -> round up of 0xB717 > 0x8000 -> 0x38D2
    assert got[5] == 0x38D2
    for v in f:
        assert orc.lib().or_f32_to_bf16(float(v)) == orc.f32_to_bf16(np.array([v], np.float32))[0]


# ---------------------------------------------------------------- generator
def _py_mix64(z):
    M = (1 << 64) - 1
    z &= M
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return z ^ (z >> 31)


def test_generator_matches_independent_python(orc):
    M = (1 << 64) - 1
    seed, stream = 0, 5
    key = _py_mix64((seed * 0xD1B54A32D192ED03 + stream) & M)
    assert orc.lib().or_key(seed, stream) == key
    draws = [_py_mix64((key + (i + 1) * 0x9E3779B97F4A7C15) & M) for i in range(64)]
    assert list(orc.gen_u4(64, seed, stream)) == [d >> 60 for d in draws]
    # Irwin-Hall(12) normal from three draws per element
    for i in range(5):
        s = 0
        for t in range(3):
            r = _py_mix64((key + (3 * i + t + 1) * 0x9E3779B97F4A7C15) & M)
            s += (r & 0xFFFF) + ((r >> 16) & 0xFFFF) + ((r >> 32) & 0xFFFF) + (r >> 48)
        want = np.float32((s + 6) / 65536.0 - 6.0)
        assert np.float32(orc.lib().or_normal(key, i)) == want


def test_generator_moments(orc):
    n = 1 << 20
    x = orc.bf16_to_f32(orc.gen_bf16(n, 0, 3, 0)).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.var() - 1.0) < 1e-2
    s = orc.bf16_to_f32(orc.gen_bf16(n, 0, 2, 1)).astype(np.float64)
    # |N(0, 0.02)| + 1e-4 has mean 0.02*sqrt(2/pi) + 1e-4
    assert s.min() >= 1e-4 * 0.99 and abs(s.mean() - (0.02 * np.sqrt(2 / np.pi) + 1e-4)) < 2e-4
    u = orc.gen_u4(n, 0, 0)
    counts = np.bincount(u, minlength=16)
    assert counts.size == 16 and np.all(np.abs(counts / n - 1 / 16) < 2e-3)


# -------------------------------------------------- reference fixtures (A0)
def _solve_group(q, f, orc):
    """Find (zp in [-8,7], bf16 s) with float(q - zp) * s == f bit-exactly."""
    for zp in range(-8, 8):
        d = (q.astype(np.int32) - zp).astype(np.float32)
        nz = d != 0
        if np.any(~nz & (f != 0)):
            continue
        if not np.any(nz):
            return zp, 0x3F80
        s16 = orc.f32_to_bf16(np.array([f[nz][0] / d[nz][0]], np.float32))[0]
        s = orc.bf16_to_f32(np.array([s16], np.uint16))[0]
        if np.array_equal((d * s).view(np.uint32), f.view(np.uint32)):
            return zp, int(s16)
    return None


@pytest.mark.parametrize("idx", range(7))
def test_ct_fixture_dequant_bitexact(orc, idx):
    """tests/fixtures/dequant (written by the reference's tools/dump_dequant_ref.py
    from compressed_tensors.unpack_from_int32): re-pack each 64x512 tile in the A0
    layout and require unpack + dequant to reproduce the library's values bit for bit
    (the check of tests/gate_dequant.cpp:71-87)."""
    man = json.load(open(os.path.join(GOLD, "ct_dequant", "manifest.json")))
    t = man["tensors"][idx]
    rows, cols, gs = t["rows"], t["cols"], t["group_size"]
    q8 = np.fromfile(os.path.join(GOLD, "ct_dequant", t["q_file"]), np.int8).reshape(rows, cols)
    f32 = np.fromfile(os.path.join(GOLD, "ct_dequant", t["deq_file"]), np.float32).reshape(rows, cols)
    G = cols // gs
    zp = np.empty((rows, G), np.uint8)
    s = np.empty((rows, G), np.uint16)
    for o in range(rows):
        for g in range(G):
            sol = _solve_group(q8[o, g * gs:(g + 1) * gs], f32[o, g * gs:(g + 1) * gs], orc)
            assert sol is not None, (o, g)
            assert t["zp_min"] <= sol[0] <= t["zp_max"]
            zp[o, g] = sol[0] + 8
            s[o, g] = sol[1]
    q = (q8.astype(np.int16) + 8).astype(np.uint8)
    packed, scale, zpw = orc.pack_ct(q, zp, s, gs)
    q2, zp2, s2 = orc.unpack_ct(packed, scale, zpw, rows, cols, gs)
    assert np.array_equal(q2.astype(np.int16) - 8, q8.astype(np.int16))   # int4 values
    w = orc.dequant_f32(q2, zp2, s2, gs)
    assert np.array_equal(w.view(np.uint32), f32.view(np.uint32))          # |diff| == 0
    # signed accessors restate w4_q / w4_zp
    lib = orc.lib()
    for (o, i) in [(0, 0), (5, 77), (63, 511), (17, 300)]:
        assert lib.or_ct_q(packed, cols, o, i) == q8[o, i]
        assert lib.or_ct_zp(zpw, G, o, i // gs) == int(zp[o, i // gs]) - 8


def test_ct_unpack_matches_reference_header(orc):
    """oracle/_ref is the reference's src/loader/w4a16_unpack.h compiled as is."""
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(7)
    N, K, G = 24, 256, 2
    packed = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32)
    zpw = rng.integers(0, 2**32, size=(N // 8, G), dtype=np.uint64).astype(np.uint32)
    lib = orc.lib()
    for o in range(N):
        for i in range(K):
            assert lib.or_ct_q(packed, K, o, i) == ref.ref_w4_q(packed, K, o, i)
        for g in range(G):
            assert lib.or_ct_zp(zpw, G, o, g) == ref.ref_w4_zp(zpw, G, o, g)


# ----------------------------------------------------------- AWQ layouts
def test_pack_known_answers(orc):
    # one row, elements k = 0..7 valued k (8 rows so N % 8 == 0; other rows zero)
    N, K = 8, 128
    q = np.zeros((N, K), np.uint8)
    q[0, :8] = np.arange(8)
    zp = np.zeros((N, 1), np.uint8)
    zp[:, 0] = np.arange(8)
    s = np.full((N, 1), 0x3F80, np.uint16)
    p0, _, z0 = orc.pack_ct(q, zp, s)
    assert p0[0, 0] == 0x76543210 and z0[0, 0] == 0x76543210
    p1, s1, z1 = orc.pack_awq_k(q, zp, s)
    # AutoAWQ order {0,2,4,6,1,3,5,7}: slot i holds element AWQ_ORDER[i]
    assert p1[0, 0] == 0x75316420 and z1[0, 0] == 0x75316420
    assert s1.shape == (1, N)
    q2 = np.zeros((N, K), np.uint8)
    q2[:, 0] = np.arange(8)       # column k=0 across rows n = 0..7
    p2, _, _ = orc.pack_awq_n(q2, zp, s)
    assert p2.shape == (K, 1) and p2[0, 0] == 0x75316420


@pytest.mark.parametrize("N,K", [(64, 256), (40, 512)])
def test_layout_round_trips_agree(orc, N, K):
    q, zp, s = orc.gen_weights(N, K, seed=3, tensor=1)
    L0 = orc.unpack_ct(*orc.pack_ct(q, zp, s), N, K)
    L1 = orc.unpack_awq_k(*orc.pack_awq_k(q, zp, s), N, K)
    L2 = orc.unpack_awq_n(*orc.pack_awq_n(q, zp, s), N, K)
    for L in (L0, L1, L2):
        for a, b in zip(L, (q, zp, s)):
            assert np.array_equal(a, b)


# ----------------------------------------------------------- matmul forms
def _np_dequant(q, zp, s, group=128):
    z = np.repeat(zp.astype(np.float64), group, axis=1)
    sc = np.repeat(s.astype(np.uint32) << 16, group, axis=1).astype(np.uint32).view(np.float32)
    return (q.astype(np.float64) - z) * sc.astype(np.float64)


def test_matmul_brute_force_tiny(orc):
    N, K, M = 16, 256, 3
    q, zp, s = orc.gen_weights(N, K, seed=11)
    x = orc.gen_x(M, K, seed=11)
    want = orc.bf16_to_f32(x).astype(np.float64) @ _np_dequant(q, zp, s).T
    got = orc.matmul_f64(x, q, zp, s)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_matmul_closed_forms(orc):
    N, K = 8, 256
    q, zp, s = orc.gen_weights(N, K, seed=2)
    # s = 1, zp = 0, x = e_k picks column k of q
    one = np.full_like(s, 0x3F80)
    zero = np.zeros_like(zp)
    for k in (0, 37, 255):
        x = np.zeros((1, K), np.uint16)
        x[0, k] = 0x3F80
        assert np.array_equal(orc.matmul_f64(x, q, zero, one)[0], q[:, k].astype(np.float64))
    # q == zp everywhere -> zero output
    qz = np.repeat(zp, 128, axis=1)
    x = orc.gen_x(2, K, seed=4)
    assert not np.any(orc.matmul_f64(x, qz, zp, s))
    # constant x = 1 -> sum_g s * (sum_k q - 128 zp)
    x1 = np.full((1, K), 0x3F80, np.uint16)
    sf = orc.bf16_to_f32(s).astype(np.float64)
    want = (sf * (q.reshape(N, 2, 128).sum(-1) - 128.0 * zp)).sum(-1)
    np.testing.assert_allclose(orc.matmul_f64(x1, q, zp, s)[0], want, rtol=1e-13)


def test_cpu_baseline_agrees(orc):
    N, K, M = 64, 512, 2
    q, zp, s = orc.gen_weights(N, K, seed=5)
    x = orc.gen_x(M, K, seed=5)
    y, used = orc.cpu_w4a16_matmul(x, *orc.pack_ct(q, zp, s), N, K, threads=2)
    assert used == 2
    m = orc.parity_metrics(y, orc.matmul_f64(x, q, zp, s))
    assert m["max_rel"] < 1e-2 and m["mean_abs_vs_bf16_ref"] < 1e-3


def test_dequant_bf16_rounds_fp32_product(orc):
    q, zp, s = orc.gen_weights(8, 256, seed=9)
    wf = orc.dequant_f32(q, zp, s)
    wb = orc.dequant_bf16(q, zp, s)
    assert np.array_equal(wb, orc.f32_to_bf16(wf))
    np.testing.assert_array_equal(wf, _np_dequant(q, zp, s).astype(np.float32))


# ------------------------------------------------------------------ argmax
def test_argmax_lowest_index_on_ties(orc):
    rng = np.random.default_rng(1)
    v = rng.standard_normal((5, 1000))
    v[2, 10] = v[2, 900] = 50.0
    v[3, :] = 1.0
    idx, margin = orc.argmax_rows_f64(v)
    assert list(idx) == list(np.argmax(v, axis=1))
    assert idx[2] == 10 and idx[3] == 0 and margin[2] == 0 and margin[3] == 0
    assert np.all(margin[[0, 1, 4]] > 0)
    f = v.astype(np.float32)
    assert list(orc.argmax_rows_f32(f)) == list(np.argmax(f, axis=1))
    b = orc.f32_to_bf16(f)
    assert list(orc.argmax_rows_bf16(b)) == list(np.argmax(orc.bf16_to_f32(b), axis=1))


# ------------------------------------------------------------------ W8A16
def test_w8_quantize_recovers_power_of_two_grids(orc):
    """Rows that are integer multiples k*c of a power of two c with max |k| =
    127 quantize exactly: s = c and q = k (inv = 1/c is exact, so any sign,
    index or rounding slip shows)."""
    rng = np.random.default_rng(0)
    N, K = 16, 512
    k = rng.integers(-127, 128, (N, K))
    c = 2.0 ** rng.integers(-12, 3, (N, K // 128))
    k[:, ::128] = np.where(rng.random((N, K // 128)) < 0.5, 127, -127)   # pin the max
    w = (k * np.repeat(c, 128, axis=1)).astype(np.float32)
    q, s = orc.w8_quantize(orc.f32_to_bf16(w))
    assert np.array_equal(q, k.astype(np.int8))
    assert np.array_equal(orc.bf16_to_f32(s), c.astype(np.float32))


def test_w8_quantize_properties(orc):
    """Random bf16 rows: the group max maps to +-127, |q| <= 127, symmetric in
    sign, zero groups give s = q = 0, and the reconstruction error is at most
    half a step of the unrounded scale plus the bf16 rounding of the scale."""
    rng = np.random.default_rng(1)
    N, K = 32, 384
    w = orc.f32_to_bf16(rng.standard_normal((N, K)).astype(np.float32) * 0.05)
    w[3, 128:256] = 0                        # one all-zero group
    q, s = orc.w8_quantize(w)
    qn, sn = orc.w8_quantize(w ^ np.uint16(0x8000))   # negated source
    assert np.array_equal(qn, -q) and np.array_equal(sn, s)
    assert np.abs(q.astype(int)).max() <= 127
    wf = orc.bf16_to_f32(w).reshape(N, 3, 128)
    qg = q.reshape(N, 3, 128).astype(int)
    for n in range(N):
        for g in range(3):
            mx = np.abs(wf[n, g]).max()
            if mx == 0:
                assert s[n, g] == 0 and not qg[n, g].any()
                continue
            assert np.abs(qg[n, g])[np.abs(wf[n, g]) == mx].min() == 127
            step = mx / 127.0
            err = np.abs(wf[n, g] - qg[n, g] * orc.bf16_to_f32(s[n, g]))
            assert err.max() <= 0.5 * step * (1 + 1e-6) + 127 * abs(orc.bf16_to_f32(s[n, g]) - step)


def test_w8_quantize_rounds_half_to_even(orc):
    """w = (j + 1/2) * c for a power of two c with 127 c as the group max:
    rint sends the halves to the even neighbour (the reference's __float2int_rn)."""
    K = 128
    c = 2.0 ** -6
    row = np.zeros(K, np.float32)
    row[0] = 127 * c
    halves = np.arange(-60, 60) + 0.5
    row[1:1 + halves.size] = halves * c
    q, s = orc.w8_quantize(orc.f32_to_bf16(row[None, :]))
    assert q[0, 0] == 127 and orc.bf16_to_f32(s[0, 0]) == c
    want = np.rint(halves).astype(int)      # numpy rint: round half to even
    assert np.array_equal(q[0, 1:1 + halves.size].astype(int), want)
    assert all(v % 2 == 0 for v in want)


def test_w8_matmul_closed_forms(orc):
    """Column pick (x = e_k) returns q[:, k] * s; a constant x returns the row
    sums; brute force in numpy float64 on a tiny shape."""
    rng = np.random.default_rng(2)
    N, K = 24, 256
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = orc.f32_to_bf16(np.abs(rng.standard_normal((N, 2)).astype(np.float32)) * 0.01)
    sf = np.repeat(orc.bf16_to_f32(s).astype(np.float64), 128, axis=1)
    x = np.zeros((1, K), np.uint16)
    x[0, 77] = 0x3F80                                      # 1.0
    assert np.array_equal(orc.w8_matmul_f64(x, q, s)[0], q[:, 77] * sf[:, 77])
    ones = np.full((1, K), 0x3F80, np.uint16)
    assert np.allclose(orc.w8_matmul_f64(ones, q, s)[0], (q * sf).sum(1), rtol=0, atol=1e-12)
    xr = orc.f32_to_bf16(rng.standard_normal((3, K)).astype(np.float32))
    ref = orc.bf16_to_f32(xr).astype(np.float64) @ (q * sf).T
    assert np.allclose(orc.w8_matmul_f64(xr, q, s), ref, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------ INT4 quantizer
def _i4_unpack(orc, packed, scale, zp, N, K):
    q, z, s = orc.unpack_ct(packed, scale, zp, N, K)
    return q.astype(int), z.astype(int), orc.bf16_to_f32(s)


def test_quant_i4_recovers_even_grids(orc):
    """Groups of 16 evenly spaced values (i - z0) d, d a power of two, all 16
    present: s = 15 d / 15 = d exactly, z = z0, q = i, and the dequantized
    (q - z) s is the source exactly (k_quant_i4, model.cu:140-172)."""
    rng = np.random.default_rng(3)
    N, K = 16, 512
    G = K // 128
    z0 = rng.integers(0, 16, (N, G))
    d = 2.0 ** rng.integers(-10, 0, (N, G))
    idx = rng.integers(0, 16, (N, K))
    for g in range(G):
        idx[:, g * 128:g * 128 + 16] = np.arange(16)   # every level present
    w = (idx - np.repeat(z0, 128, axis=1)) * np.repeat(d, 128, axis=1)
    packed, scale, zp = orc.quant_i4(orc.f32_to_bf16(w.astype(np.float32)))
    q, z, s = _i4_unpack(orc, packed, scale, zp, N, K)
    assert np.array_equal(q, idx)
    assert np.array_equal(z, z0)
    assert np.array_equal(s, d.astype(np.float32))
    assert np.array_equal((q - np.repeat(z, 128, axis=1)) * np.repeat(s, 128, axis=1), w)


def test_quant_i4_constant_groups(orc):
    """max == min: s = 1e-8 (stored bf16(1e-8)); a positive constant gives z = 0
    and q = 15 (both clamped), a negative one z = 15 and q = 0, zero z = q = 0."""
    N, K = 8, 384
    w = np.zeros((N, K), np.float32)
    w[:, :128], w[:, 128:256] = 0.75, -2.5
    packed, scale, zp = orc.quant_i4(orc.f32_to_bf16(w))
    q, z, s = _i4_unpack(orc, packed, scale, zp, N, K)
    assert np.all(s == orc.bf16_to_f32(orc.f32_to_bf16(np.float32(1e-8))))
    assert np.all(z[:, 0] == 0) and np.all(q[:, :128] == 15)
    assert np.all(z[:, 1] == 15) and np.all(q[:, 128:256] == 0)
    assert np.all(z[:, 2] == 0) and np.all(q[:, 256:] == 0)


def test_quant_i4_rounds_half_to_even(orc):
    """lo = 0, hi = 15 d with d a power of two: s = d, 1/s exact, so the values
    (j + 1/2) d sit exactly on halves and rint sends them to the even
    neighbour (the reference's __float2int_rn)."""
    d = 2.0 ** -5
    row = np.zeros(128, np.float32)
    row[1] = 15 * d
    halves = np.arange(0, 14) + 0.5
    row[2:2 + halves.size] = halves * d
    packed, scale, zp = orc.quant_i4(orc.f32_to_bf16(np.tile(row, (8, 1))))
    q, z, s = _i4_unpack(orc, packed, scale, zp, 8, 128)
    assert s[0, 0] == d and z[0, 0] == 0 and q[0, 1] == 15
    want = np.rint(halves).astype(int)
    assert np.array_equal(q[0, 2:2 + halves.size], want) and all(v % 2 == 0 for v in want)


def test_quant_i4_brute_force_and_error_bound(orc):
    """Random bf16 rows against an independent float32 numpy restatement of
    the same steps (min / max, IEEE division, rint), and the reconstruction
    error within one step of the unrounded scale plus the scale's bf16
    rounding over 15 steps."""
    rng = np.random.default_rng(4)
    N, K = 24, 640
    w = orc.f32_to_bf16((rng.standard_normal((N, K)) * 0.03).astype(np.float32))
    packed, scale, zp = orc.quant_i4(w)
    q, z, s = _i4_unpack(orc, packed, scale, zp, N, K)
    f = orc.bf16_to_f32(w).reshape(N, K // 128, 128)
    lo, hi = f.min(axis=2), f.max(axis=2)
    sf = (hi - lo) / np.float32(15)
    sf = np.where(sf > 0, sf, np.float32(1e-8)).astype(np.float32)
    zf = np.clip(np.rint(-lo / sf), 0, 15).astype(int)
    inv = (np.float32(1) / sf).astype(np.float32)
    qf = np.clip(np.rint(f * inv[..., None]).astype(int) + zf[..., None], 0, 15)
    assert np.array_equal(z, zf)
    assert np.array_equal(q, qf.reshape(N, K))
    assert np.array_equal(orc.f32_to_bf16(sf), orc.f32_to_bf16(s))
    rec = (q.reshape(N, K // 128, 128) - z[..., None]) * s[..., None]
    bound = sf[..., None] * 1.0 + 15 * np.abs(s - sf)[..., None] + 1e-12
    assert np.all(np.abs(rec - f) <= bound)
