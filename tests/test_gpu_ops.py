"""GPU parity of every launcher of the net.h surface (libtsn C ABI) against the CPU oracle.

Tolerances: MFMA launchers take f16 operands, so each is checked twice — against the oracle in
f32 (bound set by f16 operand rounding, rel-L2 <= 2e-3) and against a float64 product of the
same f16-rounded operands (bound set by f32 accumulation order, rel-L2 <= 2e-5). f32 launchers
(LN, gate_add, rms_head, rope, elementwise, f32 linear) are held to rel-L2 <= 1e-5.
"""
import numpy as np
import pytest

from conftest import f16r, rel_l2, rng

pytestmark = pytest.mark.gpu

F32, F16, BF16 = 0, 1, 2


def _gemm_case(tsn, rt, orc, M, N, K, xdt, ydt, bias=True, ldx=0, ldw=0, ldy=0, seed=0):
    r = rng(seed)
    lx, lw, ly = ldx or K, ldw or K, ldy or N
    X = r.standard_normal((M, lx)).astype(np.float32)
    W = (r.standard_normal((N, lw)) * 0.03).astype(np.float32)
    b = r.standard_normal(N).astype(np.float32) if bias else None
    Wd = rt.array(W.astype(np.float16))
    Xd = rt.array(X.astype(np.float16) if xdt == F16 else X)
    ynp = np.float16 if ydt == F16 else np.float32
    Yd = rt.array(np.full((M, ly), np.nan, ynp))
    bd = rt.array(b) if bias else None
    rt.gemm(F16, Wd, Xd, xdt, Yd, ydt, bd, M, N, K, ldx, ldw, ldy)
    rt.sync()
    Y = Yd.numpy().astype(np.float32)
    if ly > N:
        assert np.isnan(Y[:, N:]).all(), "gemm wrote outside the N columns of a strided output"
    Y = Y[:, :N]
    Xr, Wr = f16r(X[:, :K]), f16r(W[:, :K])
    ref64 = Xr.astype(np.float64) @ Wr.T.astype(np.float64) + (b if bias else 0)
    ref_orc = orc.gemm(W[:, :K], X[:, :K], b)
    return Y, ref64, ref_orc


@pytest.mark.parametrize("M,N,K", [(512, 3072, 1024), (282, 1024, 4096), (794, 4096, 1024), (43, 1024, 3072),
                                   (1, 64, 64), (130, 200, 72), (77, 5120, 2048)])
def test_gemm_f32_io(tsn, rt, orc, M, N, K):
    Y, ref64, ref_orc = _gemm_case(tsn, rt, orc, M, N, K, F32, F32)
    assert not np.isnan(Y).any()
    assert rel_l2(Y, ref64) < 2e-5
    assert rel_l2(Y, ref_orc) < 2e-3


def test_gemm_f16_io_strided(tsn, rt, orc):
    Y, ref64, ref_orc = _gemm_case(tsn, rt, orc, 390, 1152, 1152, F16, F16, ldx=1160, ldw=1160, ldy=1280, seed=3)
    assert rel_l2(Y, ref64) < 1e-3   # f16 output rounding
    assert rel_l2(Y, ref_orc) < 2e-3


def test_gemm_f32_weights(tsn, rt, orc):
    r = rng(5)
    M, N, K = 77, 1024, 1024
    X = r.standard_normal((M, K)).astype(np.float32)
    W = (r.standard_normal((N, K)) * 0.03).astype(np.float32)
    b = r.standard_normal(N).astype(np.float32)
    Y = rt.empty((M, N))
    rt.gemm(F32, rt.array(W), rt.array(X), F32, Y, F32, rt.array(b), M, N, K)
    rt.sync()
    assert rel_l2(Y.numpy(), orc.gemm(W, X, b)) < 1e-5


def test_gemm_rejects_bad_shape(tsn, rt):
    Wd, Xd, Yd = rt.empty((64, 12), np.float16), rt.empty((4, 12)), rt.empty((4, 64))
    with pytest.raises(tsn.TsnError) as e:
        rt.gemm(F16, Wd, Xd, F32, Yd, F32, None, 4, 64, 12)   # K % 8 != 0
    assert e.value.code == 1


@pytest.mark.parametrize("T,IC,OC,K,pad", [(256, 1024, 4096, 3, 1), (256, 4096, 1024, 3, 1), (172, 1024, 64, 7, 3),
                                           (100, 64, 1024, 3, 1), (37, 128, 256, 1, 0), (1, 64, 128, 3, 1)])
def test_conv1d(tsn, rt, orc, T, IC, OC, K, pad):
    r = rng(T + IC + OC + K)
    x = r.standard_normal((T, IC)).astype(np.float32)
    W = (r.standard_normal((OC, IC, K)) * 0.03).astype(np.float32)
    b = r.standard_normal(OC).astype(np.float32)
    Wd = rt.array(W.astype(np.float16))
    Wp = rt.empty((OC, K, IC), np.float16)
    rt.conv1d_prepare(Wd, False, Wp, OC, IC, K)
    OL = T + 2 * pad - K + 1
    y = rt.empty((OL, OC))
    rt.conv1d(Wp, rt.array(b), rt.array(x), y, T, OL, IC, OC, K, 1, pad, 1)
    rt.sync()
    out = y.numpy()
    ref_m = orc.conv1d(f16r(W), b, f16r(x), pad, direct=True)
    ref = orc.conv1d(W, b, x, pad)
    assert rel_l2(out, ref_m) < 2e-5
    assert rel_l2(out, ref) < 2e-3


def test_conv1d_weight_prepare_layout(tsn, rt):
    r = rng(9)
    OC, IC, K = 8, 64, 3
    W = r.standard_normal((OC, IC, K)).astype(np.float16)
    Wp = rt.empty((OC, K, IC), np.float16)
    rt.conv1d_prepare(rt.array(W), False, Wp, OC, IC, K)
    rt.sync()
    assert np.array_equal(Wp.numpy(), np.transpose(W, (0, 2, 1)))


def test_conv1d_rejects_stride(tsn, rt):
    Wp, x, y = rt.empty((64, 3, 64), np.float16), rt.empty((16, 64)), rt.empty((8, 64))
    with pytest.raises(tsn.TsnError) as e:
        rt.conv1d(Wp, None, x, y, 16, 8, 64, 64, 3, 2, 1, 1)
    assert e.value.code == 3


@pytest.mark.parametrize("wdt", [BF16, F16, F32])
def test_gemv(tsn, rt, orc, wdt):
    r = rng(11 + wdt)
    N, K = 6144, 1024
    W = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    if wdt == BF16:
        Wh = tsn.synth_normal_bf16(7, 0, 0.0, 0.02, (N, K))
        W = tsn.bf16_to_f32(Wh)
    elif wdt == F16:
        Wh = W.astype(np.float16)
        W = Wh.astype(np.float32)
    else:
        Wh = W
    x = r.standard_normal(K).astype(np.float32)
    b = r.standard_normal(N).astype(np.float32)
    y = rt.empty((N,))
    rt.gemv(rt.array(Wh), wdt, rt.array(x), y, rt.array(b), N, K)
    rt.sync()
    assert rel_l2(y.numpy(), orc.gemv(W, x, b)) < 1e-5


@pytest.mark.parametrize("per_row,chunks,base,ydt", [(0, 6, 0, F32), (0, 6, 3 * 1024, F32), (1, 2, 0, F32),
                                                     (0, 6, 0, F16)])
def test_adaln_ln(tsn, rt, orc, per_row, chunks, base, ydt):
    r = rng(21 + per_row + base)
    rows, H = 397, 1024
    x = (r.standard_normal((rows, H)) * 3 + 1).astype(np.float32)
    mod = r.standard_normal((rows if per_row else 1, chunks * H)).astype(np.float32) * 0.5
    y = rt.empty((rows, H), np.float16 if ydt == F16 else np.float32)
    rt.adaln_ln(rt.array(x), rt.array(mod), y, ydt, rows, H, per_row, chunks, base, 1e-5)
    rt.sync()
    ref = orc.adaln_ln(x, mod, per_row, chunks, base)
    assert rel_l2(y.numpy().astype(np.float32), ref) < (1e-3 if ydt == F16 else 1e-5)


def test_gate_add(tsn, rt, orc):
    r = rng(31)
    rows, H = 141, 1024
    x, f = r.standard_normal((rows, H)).astype(np.float32), r.standard_normal((rows, H)).astype(np.float32)
    mod = r.standard_normal((rows, 6 * H)).astype(np.float32)
    for per_row in (0, 1):
        y = rt.empty((rows, H))
        rt.gate_add(rt.array(x), rt.array(f), rt.array(mod), y, rows, H, per_row, 6, 2)
        rt.sync()
        assert rel_l2(y.numpy(), orc.gate_add(x, f, mod, per_row, 6, 2)) < 1e-6


def test_rms_head_and_rope(tsn, rt, orc):
    r = rng(41)
    S, H, nh, hd = 397, 1024, 16, 64
    qkv = r.standard_normal((S, 3 * H)).astype(np.float32)
    w = (1 + 0.02 * r.standard_normal(hd)).astype(np.float32)
    d = rt.array(qkv)
    rt.rms_head(d, rt.array(w), 256, nh, 3 * H, hd, H, 10, 1e-6)
    rt.sync()
    ref = orc.rms_head(qkv, w, 256, nh, 3 * H, hd, H, 10, 1e-6)
    assert rel_l2(d.numpy(), ref) < 1e-6
    pos = np.arange(256, dtype=np.int32)[::-1].copy()
    rt.rope_pairs(d, rt.array(pos), 256, nh, 3 * H, hd, 0, 5, 0.5, 10000.0)
    rt.sync()
    ref = orc.rope_pairs(ref, pos, 256, nh, 3 * H, hd, 0, 5, 0.5, 10000.0)
    assert rel_l2(d.numpy(), ref) < 1e-5


def test_elementwise(tsn, rt, orc):
    r = rng(51)
    n = 256 * 64 + 7
    a, b, c = (r.standard_normal(n).astype(np.float32) for _ in range(3))
    da, db, dc = rt.array(a), rt.array(b), rt.array(c)
    y = rt.empty((n,))
    rt.swiglu(da, db, y, n); rt.sync()
    assert rel_l2(y.numpy(), orc.swiglu(a, b)) < 1e-6
    rt.add_(da, db, y, n); rt.sync()
    assert np.array_equal(y.numpy(), orc.add(a, b))
    rt.copy(da, y, n); rt.sync()
    assert np.array_equal(y.numpy(), a)
    rt.silu(y, n); rt.sync()
    assert rel_l2(y.numpy(), orc.silu(a)) < 1e-6
    x2 = rt.array(c)
    rt.cfg_euler(da, db, x2, n, 5.0, -1.0 / 24); rt.sync()
    assert rel_l2(x2.numpy(), orc.cfg_euler(a, b, c, 5.0, -1.0 / 24)) < 1e-6
    S, H = 64, 256
    X = r.standard_normal((S, H)).astype(np.float32)
    v = r.standard_normal(H).astype(np.float32)
    yy = rt.empty((S, H))
    rt.add_bcast_col(rt.array(X), rt.array(v), yy, S, H); rt.sync()
    assert np.array_equal(yy.numpy(), orc.add_bcast_col(X, v))


@pytest.mark.parametrize("S", [397, 1101, 1, 64, 65])
def test_attention(tsn, rt, orc, S):
    r = rng(61 + S)
    H, nh, hd = 1024, 16, 64
    qkv = r.standard_normal((S, 3 * H)).astype(np.float32)
    qkv[:, :2 * H] *= 1.5     # sharper softmax than N(0,1) logits/8
    out = rt.array(np.full((S, H), np.nan, np.float32))
    rt.attention(rt.array(qkv), out, S, nh, hd, 3 * H, H, 0, H, 2 * H, 0, 0.125)
    rt.sync()
    o = out.numpy()
    assert not np.isnan(o).any()
    ref_m = orc.attention(f16r(qkv), S, nh, hd, 3 * H, H, 0, H, 2 * H, 0, 0.125)
    ref = orc.attention(qkv, S, nh, hd, 3 * H, H, 0, H, 2 * H, 0, 0.125)
    assert rel_l2(o, ref_m) < 2e-3
    assert rel_l2(o, ref) < 3e-3
