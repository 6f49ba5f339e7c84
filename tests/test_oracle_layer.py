"""CPU pins of the oracle's restatements of the reference's elementwise layer
steps (src/kernels/elementwise.cu:8-49): rmsnorm, swiglu, residual_add.

Each is checked against a library routine that computes the same
mathematics independently (torch.nn.functional.rms_norm / silu, torch bf16
addition) and against invariants a wrong term, sign or operand would break."""
import numpy as np
import pytest
import torch

import oracle as orc


def _t(bits):
    return torch.from_numpy(orc.bf16_to_f32(bits).astype(np.float32))


def _bits(t):
    return orc.f32_to_bf16(t.to(torch.float32).numpy())


@pytest.mark.parametrize("rows,dim", [(1, 5120), (9, 4096), (3, 136)])
def test_rmsnorm_matches_torch_rms_norm(rows, dim):
    x = orc.gen_x(rows, dim, seed=rows)
    w = orc.gen_bf16(dim, seed=7, stream=dim, kind=1)  # small positive weights
    eps = 1e-6
    got = orc.bf16_to_f32(orc.rmsnorm_bf16(x, w, eps)).astype(np.float64)
    # F.rms_norm with the reference's (1 + w) weight, fp32, then bf16
    ref = torch.nn.functional.rms_norm(_t(x), (dim,), weight=1.0 + _t(w), eps=eps)
    refb = orc.bf16_to_f32(_bits(ref)).astype(np.float64)
    # identical up to rare 1-ulp bf16 flips from the fp32 sum order
    ulp = np.abs(refb) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - refb) <= ulp)
    assert np.mean(got != refb) < 0.01


def test_rmsnorm_invariants():
    dim = 512
    x = orc.gen_x(1, dim, seed=3)
    zero_w = np.zeros(dim, np.uint16)                 # bf16 0.0: weight factor 1
    y = orc.bf16_to_f32(orc.rmsnorm_bf16(x, zero_w, 0.0)).astype(np.float64)
    # unit root-mean-square output (to bf16 precision)
    assert abs(np.sqrt(np.mean(y ** 2)) - 1.0) < 1e-2
    # scale invariance: rmsnorm(4x) == rmsnorm(x) exactly (power-of-two scale)
    x4 = orc.f32_to_bf16(orc.bf16_to_f32(x) * 4.0)
    assert np.array_equal(orc.rmsnorm_bf16(x4, zero_w, 0.0), orc.rmsnorm_bf16(x, zero_w, 0.0))
    # the weight enters as (1 + w): w = 1.0 doubles every output exactly
    one_w = np.full(dim, 0x3F80, np.uint16)
    y2 = orc.bf16_to_f32(orc.rmsnorm_bf16(x, one_w, 0.0)).astype(np.float64)
    assert np.array_equal(y2, 2.0 * y)
    # a constant row c normalizes to sign(c) (eps = 0)
    c = np.full((1, dim), 0xC0A0, np.uint16)          # -5.0
    assert np.all(orc.bf16_to_f32(orc.rmsnorm_bf16(c, zero_w, 0.0)) == -1.0)


@pytest.mark.parametrize("rows,inter", [(1, 17408), (12, 256)])
def test_swiglu_matches_torch_silu(rows, inter):
    fused = orc.gen_x(rows, 2 * inter, seed=inter)
    got = orc.swiglu_bf16(fused, inter)
    f = _t(fused)
    ref = _bits(torch.nn.functional.silu(f[:, :inter]) * f[:, inter:])
    gf, rf = orc.bf16_to_f32(got).astype(np.float64), orc.bf16_to_f32(ref).astype(np.float64)
    assert np.all(np.abs(gf - rf) <= np.abs(rf) * 2.0 ** -7 + 1e-30)
    assert np.mean(got != ref) < 0.01


def test_swiglu_invariants():
    inter = 64
    g = orc.gen_x(1, inter, seed=5)
    one = np.full((1, inter), 0x3F80, np.uint16)
    # up = 1: silu(g); gate = 0: 0 whatever up; large gate: ~ gate * up
    s1 = orc.bf16_to_f32(orc.swiglu_bf16(np.concatenate([g, one], 1), inter))
    gf = orc.bf16_to_f32(g).astype(np.float64)
    np.testing.assert_allclose(s1, gf / (1 + np.exp(-gf)), rtol=2 ** -7)
    zero = np.zeros((1, inter), np.uint16)
    assert np.all(orc.bf16_to_f32(orc.swiglu_bf16(np.concatenate([zero, g], 1), inter)) == 0.0)
    big = np.full((1, inter), 0x4220, np.uint16)      # 40.0
    assert np.array_equal(orc.swiglu_bf16(np.concatenate([big, g], 1), inter),
                          orc.f32_to_bf16(40.0 * orc.bf16_to_f32(g)))


def test_residual_add_matches_torch_bf16_add():
    a, b = orc.gen_x(4, 1000, seed=1), orc.gen_x(4, 1000, seed=2)
    ref = (_t(a).to(torch.bfloat16) + _t(b).to(torch.bfloat16)).to(torch.float32)
    assert np.array_equal(orc.residual_add_bf16(a, b), _bits(ref))
    assert np.array_equal(orc.residual_add_bf16(a, np.zeros_like(a)), a)
