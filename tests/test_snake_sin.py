"""The snake activation's sin^2 (thinksound-native_amd/csrc/snake.h): Cody-Waite reduction by pi in
three f32 parts and the odd Taylor series of sin through r^13. The device function runs the steps
below in f32 with fused multiply-adds; here each fma is evaluated exactly in float64 and rounded
once to float32, so the restatement reproduces the device rounding step by step. It is checked
against float64 sin(x)^2, the mathematics the kernels replace, over the argument ranges the VAE's
snakes see (max error 2.3e-7), and against planted mistakes (the r^11 term dropped, pi in one
f32 part), each of which must fail the bound. The decoder's GPU parity tests cover the device code itself."""
import numpy as np

F = np.float32
PI_PARTS = (float.fromhex("0x1.921fb6p+1"), float.fromhex("-0x1.777a5cp-24"), float.fromhex("-0x1.ee59dap-49"))
INV_PI = float.fromhex("0x1.45f306p-2")
COEF = (float.fromhex("0x1.612462p-33"), float.fromhex("-0x1.ae6456p-26"), float.fromhex("0x1.71de3ap-19"),
        float.fromhex("-0x1.a01a02p-13"), float.fromhex("0x1.111112p-7"), float.fromhex("-0x1.555556p-3"))


def fma32(a, b, c):
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(F)


def sin2_f32(x, parts=PI_PARTS, coef=COEF):
    x = np.asarray(x, F)
    k = np.rint((x * F(INV_PI)).astype(F)).astype(F)
    r = x
    for p in parts:
        r = fma32(-k, F(p), r)
    r2 = (r * r).astype(F)
    p = F(coef[0])
    for c in coef[1:]:
        p = fma32(p, r2, F(c))
    s = fma32((r * r2).astype(F), p, r)
    return (s * s).astype(F)


def _args():
    rng = np.random.default_rng(7)
    return np.concatenate([rng.uniform(-4, 4, 200000), rng.uniform(-60, 60, 200000),
                           rng.uniform(-2000, 2000, 100000), np.linspace(-1e-3, 1e-3, 2001)]).astype(F)


def _err(f):
    x = _args()
    ref = np.sin(x.astype(np.float64)) ** 2
    return np.max(np.abs(f(x).astype(np.float64) - ref))


def test_sin2_error_bound():
    # a few f32 ulps of 1: the reduction error grows with |k| (|x| up to 2000 here)
    assert _err(sin2_f32) < 4e-7


def test_sin2_small_arguments_relative():
    x = np.logspace(-6, 0, 2000).astype(F)
    ref = np.sin(x.astype(np.float64)) ** 2
    assert np.max(np.abs(sin2_f32(x) / ref - 1)) < 1e-6


def test_planted_mistakes_fail():
    # the r^11 term dropped (the r^13 term itself sits at the f32 rounding level, about 1e-7)
    assert _err(lambda x: sin2_f32(x, coef=(COEF[0],) + COEF[2:])) > 1e-6
    assert _err(lambda x: sin2_f32(x, parts=PI_PARTS[:1])) > 1e-6       # pi in one f32 part
