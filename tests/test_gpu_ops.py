"""GPU parity of every launcher of the net.h surface (libtsn C ABI) against the CPU oracle.

Tolerances: GEMM and conv launchers with f32 activations keep the reference's f32-activation
contract (the activation is an f16 hi|lo pair on MFMA), so they are held to rel-L2 <= 2e-5 against a
float64 product of the unrounded activation and the f16 weight, and to <= 2e-3 against the oracle
on the unrounded weight (bound set by the f16 weight). f32 weights (three-part products) are held
to <= 2e-5 against the oracle. The opt-in f16-activation GEMM is checked against f16-rounded
operands. f32 launchers (norms, gate_add, rms_head, rope, elementwise, f32 linear) are held to
rel-L2 <= 1e-5.
"""
import numpy as np
import pytest

from conftest import f16r, rel_l2, rng

pytestmark = pytest.mark.gpu

F32, F16, BF16 = 0, 1, 2


def _gemm_case(tsn, rt, orc, M, N, K, xdt, ydt, bias=True, ldx=0, ldw=0, ldy=0, seed=0, oracle=True):
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
    Xr = f16r(X[:, :K]) if xdt == F16 else X[:, :K]
    ref64 = Xr.astype(np.float64) @ f16r(W[:, :K]).T.astype(np.float64) + (b if bias else 0)
    ref_orc = orc.gemm(W[:, :K], X[:, :K], b) if oracle else None
    return Y, ref64, ref_orc


@pytest.mark.parametrize("M,N,K", [(512, 3072, 1024), (282, 1024, 4096), (794, 4096, 1024), (43, 1024, 3072),
                                   (1, 64, 64), (130, 200, 72), (77, 5120, 2048), (172, 1000, 1024)])
def test_gemm_f32_io(tsn, rt, orc, M, N, K):
    """f32 X keeps f32 accuracy: MFMA over the hi|lo split (K % 64 == 0, N % 8 == 0) or the exact
    SIMT path (K = 72, N = 1000 here)"""
    Y, ref64, ref_orc = _gemm_case(tsn, rt, orc, M, N, K, F32, F32)
    assert not np.isnan(Y).any()
    assert rel_l2(Y, ref64) < 2e-5
    assert rel_l2(Y, ref_orc) < 2e-3


def test_gemm_f32_x_is_not_rounded(tsn, rt, orc):
    """the product sees X itself, not f16(X): an f16-rounded X would sit about 3e-4 away"""
    M, N, K = 256, 512, 1024
    Y, ref64, _ = _gemm_case(tsn, rt, orc, M, N, K, F32, F32, seed=8)
    r = rng(8)
    X = r.standard_normal((M, K)).astype(np.float32)
    W = (r.standard_normal((N, K)) * 0.03).astype(np.float32)
    b = r.standard_normal(N).astype(np.float32)
    rounded = f16r(X).astype(np.float64) @ f16r(W).T.astype(np.float64) + b
    assert rel_l2(Y, ref64) < 2e-6 < rel_l2(rounded, ref64) / 10


def test_gemm_f32_x_f16_y_strided(tsn, rt, orc):
    Y, ref64, ref_orc = _gemm_case(tsn, rt, orc, 390, 1152, 1152, F32, F16, ldx=1160, ldw=1160, ldy=1280, seed=4)
    assert rel_l2(Y, ref64) < 1e-3   # f16 output rounding
    assert rel_l2(Y, ref_orc) < 2e-3


def test_gemm_f16_io_strided(tsn, rt, orc):
    Y, ref64, ref_orc = _gemm_case(tsn, rt, orc, 390, 1152, 1152, F16, F16, ldx=1160, ldw=1160, ldy=1280, seed=3)
    assert rel_l2(Y, ref64) < 1e-3   # f16 output rounding
    assert rel_l2(Y, ref_orc) < 2e-3


@pytest.mark.parametrize("M,N,K,ydt", [(4133, 4096, 1024, F16), (4096, 3200, 192, F32), (3900, 4160, 64, F32),
                                        (6352, 4096, 1024, F16), (2048, 8192, 2048, F32), (4133, 4096, 2048, F16),
                                        (4100, 4160, 2112, F32)])
def test_gemm_f16_large_grids(tsn, rt, orc, M, N, K, ydt):
    """f16 X at batch-16-sized shapes, grids of several rounds. K >= 2048 with a round of 256x256
    tiles takes the wide kernel: 2048 x 8192 x 2048 (256 tiles), 4133 x 4096 x 2048 (272 tiles, a
    37-row M tail), 4100 x 4160 x 2112 (289 tiles, tails in M and N, 66 K tiles); the rest the
    two-stage 128x128 kernel with two workgroups per CU: a ragged M tail (4133 = 32*128 + 37), N
    not a multiple of 256 (3200, 4160), K of 3 and 1 K tiles, the batch-16 FFN1 (6352 x 4096 x
    1024). Held against the float64 product of the same f16 operands (the oracle's GEMM is the same
    product and would take tens of seconds at this size)"""
    Y, ref64, _ = _gemm_case(tsn, rt, orc, M, N, K, F16, ydt, seed=11, oracle=False)
    assert not np.isnan(Y).any()
    assert rel_l2(Y, ref64) < (1e-3 if ydt == F16 else 1e-5)


@pytest.mark.parametrize("M,N,K,xdt,ydt", [(794, 1024, 4096, F16, F16), (794, 1024, 4096, F16, F32),
                                            (130, 512, 3072, F16, F32), (1600, 1024, 1024, F16, F16),
                                            (100, 200, 192, F16, F32), (282, 1024, 4096, F32, F16),
                                            (282, 1024, 4096, F32, F32), (794, 1024, 4096, F32, F32)])
def test_gemm_few_tiles(tsn, rt, orc, M, N, K, xdt, ydt):
    """grids under one round of 128x128 tiles. f16 X: 64x64 tiles over the full K (two wave groups
    on alternate K tiles for 208 and 16 tiles with K a multiple of 128; four waves for 400 tiles and
    for K = 192 with ragged M and N = 200). f32 X (the hi|lo route, whose half-width W the 64x64
    kernel does not take): a long K over 24 or 56 tiles is split into the runtime's workspace and
    summed in split order by the reduce, which applies bias and the output type. The result does not
    change from call to call"""
    Y, ref64, _ = _gemm_case(tsn, rt, orc, M, N, K, xdt, ydt, seed=17, oracle=False)
    assert not np.isnan(Y).any()
    assert rel_l2(Y, ref64) < (1e-3 if ydt == F16 else (2e-5 if xdt == F32 else 1e-5))
    Y2, _, _ = _gemm_case(tsn, rt, orc, M, N, K, xdt, ydt, seed=17, oracle=False)
    assert np.array_equal(Y, Y2)


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


def _bf16(x):
    """round-to-nearest-even f32 -> bf16 bits, and the f32 value those bits hold"""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return b, (b.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("M,N,K", [(794, 4096, 1024), (1100, 4096, 256), (130, 200, 128), (1, 64, 64)])
def test_gemm_bf16_operands(tsn, rt, M, N, K):
    """bf16 X and W on MFMA (1100 x 4096: more than one round of tiles, the two-stage kernel): each
    bf16 x bf16 product is exact in f32, so against the float64
    product of the same bf16 values only the f32 accumulation differs (rel-L2 <= 1e-5); the bias
    is added in f32"""
    r = rng(11)
    X = r.standard_normal((M, K)).astype(np.float32)
    W = (r.standard_normal((N, K)) * 0.03).astype(np.float32)
    b = r.standard_normal(N).astype(np.float32)
    xb, xv = _bf16(X)
    wb, wv = _bf16(W)
    Y = rt.array(np.full((M, N), np.nan, np.float32))
    rt.gemm(BF16, rt.array(wb), rt.array(xb), BF16, Y, F32, rt.array(b), M, N, K)
    rt.sync()
    ref = xv.astype(np.float64) @ wv.T.astype(np.float64) + b
    y = Y.numpy()
    assert not np.isnan(y).any()
    assert rel_l2(y, ref) < 1e-5
    # and it is a bf16 product, not a wider one: the product of the unrounded operands sits well
    # above that (bias left out, it would mask the product at small K)
    exact = X.astype(np.float64) @ W.T.astype(np.float64)
    assert rel_l2(y - b, exact) > 1e-3


def test_gemm_bf16_rejects_untiled_shape(tsn, rt):
    """bf16 operands run only on the MFMA tiling: K % 64 != 0 is refused, not computed elsewhere"""
    Wd, Xd, Yd = rt.empty((64, 72), np.uint16), rt.empty((4, 72), np.uint16), rt.empty((4, 64))
    with pytest.raises(tsn.TsnError) as e:
        rt.gemm(BF16, Wd, Xd, BF16, Yd, F32, None, 4, 64, 72)
    assert e.value.code == 3
    with pytest.raises(tsn.TsnError) as e:   # bf16 operands give f32 Y
        rt.gemm(BF16, rt.empty((64, 64), np.uint16), rt.empty((4, 64), np.uint16), BF16, rt.empty((4, 64), np.float16),
                F16, None, 4, 64, 64)
    assert e.value.code == 1


def test_gemm_rejects_bad_shape(tsn, rt):
    Wd, Xd, Yd = rt.empty((64, 12), np.float16), rt.empty((4, 12), np.float16), rt.empty((4, 64))
    with pytest.raises(tsn.TsnError) as e:
        rt.gemm(F16, Wd, Xd, F16, Yd, F32, None, 4, 64, 12)   # f16 X: K % 8 != 0
    assert e.value.code == 1
    Yh = rt.empty((4, 64), np.float16)
    with pytest.raises(tsn.TsnError) as e:
        rt.gemm(F16, Wd, rt.empty((4, 12)), F32, Yh, F16, None, 4, 64, 12)   # f32 X, f16 Y, K % 64 != 0
    assert e.value.code == 3


def _conv_ref(orc, W, b, x, stride, pad, dil, convt, OL):
    if convt:
        y = orc.conv1d_t(W, b, x, stride, pad)
        assert y.shape[0] == OL
        return y
    y = orc.conv1d(W, b, x, pad, stride, dil)
    assert y.shape[0] == OL
    return y


# (T, IC, OC, K, stride, pad, dil, convt, weight dtype): the DiT's own convs (implicit GEMM), dilated and
# strided convs, transposed convs (the VAE's upsamplers), channel counts that are not a multiple of
# 64 (gathered operand), outputs too narrow for a GEMM tile (direct conv), and f32 / bf16 weights
CONV_CASES = [
    (256, 1024, 4096, 3, 1, 1, 1, 0, F16), (256, 4096, 1024, 3, 1, 1, 1, 0, F16), (172, 1024, 64, 7, 1, 3, 1, 0, F16),
    (100, 64, 1024, 3, 1, 1, 1, 0, F16), (37, 128, 256, 1, 1, 0, 1, 0, F16), (1, 64, 128, 3, 1, 1, 1, 0, F16),
    (40, 128, 64, 7, 1, 9, 3, 0, F32), (60, 64, 128, 7, 1, 27, 9, 0, F16), (33, 64, 32, 4, 2, 1, 1, 0, F16),
    (20, 128, 64, 16, 8, 11, 1, 1, F32), (24, 256, 128, 8, 4, 5, 1, 1, F16), (50, 72, 48, 3, 1, 1, 1, 0, BF16),
    (100, 128, 2, 7, 1, 3, 1, 0, F32), (64, 128, 256, 3, 1, 1, 1, 0, F32), (9, 3, 16, 5, 1, 2, 1, 0, F32),
]


@pytest.mark.parametrize("T,IC,OC,K,stride,pad,dil,convt,wdt", CONV_CASES)
def test_conv1d(tsn, rt, orc, T, IC, OC, K, stride, pad, dil, convt, wdt):
    r = rng(T + IC + OC + K + stride + dil)
    x = r.standard_normal((T, IC)).astype(np.float32)
    W = (r.standard_normal((OC, IC, K)) / np.sqrt(IC * K)).astype(np.float32)
    b = r.standard_normal(OC).astype(np.float32)
    if wdt == F16:
        Wh = W.astype(np.float16)
        Wexact = f16r(W)
    elif wdt == BF16:
        Wh = tsn.synth_normal_bf16(T, IC, 0.0, 1.0 / np.sqrt(IC * K), (OC, IC, K))
        Wexact = tsn.bf16_to_f32(Wh)
        W = Wexact
    else:
        Wh = W
        Wexact = W
    Wp = rt.empty((rt.conv1d_prepared_bytes(wdt, OC, IC, K),), np.uint8)
    rt.conv1d_prepare(rt.array(Wh), wdt, Wp, OC, IC, K)
    OL = T * stride if convt else (T + 2 * pad - dil * (K - 1) - 1) // stride + 1
    y = rt.array(np.full((OL, OC), np.nan, np.float32))
    rt.conv1d(wdt, Wp, rt.array(b), rt.array(x), y, T, OL, IC, OC, K, stride, pad, dil, convt)
    rt.sync()
    out = y.numpy()
    assert not np.isnan(out).any()
    ref_exact = _conv_ref(orc, Wexact, b, x, stride, pad, dil, convt, OL)
    assert rel_l2(out, ref_exact) < 2e-5
    if wdt == F16:
        assert rel_l2(out, _conv_ref(orc, W, b, x, stride, pad, dil, convt, OL)) < 2e-3


def test_conv1d_weight_prepare_layout(tsn, rt):
    r = rng(9)
    OC, IC, K = 8, 64, 3
    W = r.standard_normal((OC, IC, K)).astype(np.float16)
    assert rt.conv1d_prepared_bytes(F16, OC, IC, K) == OC * K * IC * 2
    Wp = rt.empty((OC, K, IC), np.float16)
    rt.conv1d_prepare(rt.array(W), F16, Wp, OC, IC, K)
    rt.sync()
    assert np.array_equal(Wp.numpy(), np.transpose(W, (0, 2, 1)))
    # f32 weights: [hi | hi | lo] per tap, rows zero-padded to a multiple of 64 columns
    IC, K = 3, 5
    Wf = r.standard_normal((OC, IC, K)).astype(np.float32)
    cols = rt.conv1d_prepared_bytes(F32, OC, IC, K) // (2 * OC)
    assert cols == 64
    Wp = rt.empty((OC, cols), np.float16)
    rt.conv1d_prepare(rt.array(Wf), F32, Wp, OC, IC, K)
    rt.sync()
    got = Wp.numpy()
    hi = Wf.astype(np.float16)
    lo = (Wf - hi.astype(np.float32)).astype(np.float16)
    for k in range(K):
        blk = got[:, k * 3 * IC:(k + 1) * 3 * IC]
        assert np.array_equal(blk[:, :IC], hi[:, :, k]) and np.array_equal(blk[:, IC:2 * IC], hi[:, :, k])
        assert np.array_equal(blk[:, 2 * IC:], lo[:, :, k])
    assert (got[:, 3 * IC * K:] == 0).all()


def test_conv1d_rejects_bad_arguments(tsn, rt):
    Wp, x, y = rt.empty((64, 3, 64), np.float16), rt.empty((16, 64)), rt.empty((8, 64))
    with pytest.raises(tsn.TsnError) as e:
        rt.conv1d(F16, Wp, None, x, y, 16, 8, 64, 64, 3, 0, 1, 1)   # stride 0
    assert e.value.code == 1
    with pytest.raises(tsn.TsnError) as e:
        rt.conv1d(7, Wp, None, x, y, 16, 8, 64, 64, 3, 1, 1, 1)     # unknown weight dtype
    assert e.value.code == 1


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


# routes (16 heads, one sample): S <= 512 the all-resident eight-wave kernel; 512 < S with at most
# 256 query-tile workgroups (S = 600: 160, S = 1024: 256) the two-stage eight-wave kernel; more than
# 256 workgroups (S = 1101: 288) the four-wave kernel
@pytest.mark.parametrize("S", [397, 1101, 1, 64, 65, 100, 500, 512, 600, 1024])
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


@pytest.mark.parametrize("S", [910, 1024])
def test_attention_two_group_route(tsn, rt, orc, S):
    """64 heads: at least 512 workgroups of 128 queries, the route of the batch-16 workload (the
    four-wave kernel with two 16-query groups per wave). S = 910 leaves a last tile of 14 queries,
    so three of its four waves hold no query and only take their share of the key-block loads."""
    r = rng(83 + S)
    nh, hd = 64, 64
    H = nh * hd
    qkv = r.standard_normal((S, 3 * H)).astype(np.float32)
    qkv[:, :2 * H] *= 1.5
    out = rt.array(np.full((S, H), np.nan, np.float32))
    rt.attention(rt.array(qkv), out, S, nh, hd, 3 * H, H, 0, H, 2 * H, 0, 0.125)
    rt.sync()
    o = out.numpy()
    assert not np.isnan(o).any()
    ref_m = orc.attention(f16r(qkv), S, nh, hd, 3 * H, H, 0, H, 2 * H, 0, 0.125)
    assert rel_l2(o, ref_m) < 2e-3


@pytest.mark.parametrize("S,nh,sign", [(397, 16, 1), (397, 16, -1), (600, 16, 1), (1101, 16, 1), (1101, 16, -1),
                                       (910, 64, 1), (910, 64, -1), (910, 128, 1), (397, 256, -1)])
def test_attention_moving_reference(tsn, rt, S, nh, sign):
    """Scores that rise along the keys by about 12 log2 units per 64-key block (sign 1), so every
    block moves the running reference and rescales O and the row sum, or fall (sign -1), so later
    blocks underflow against the first block's reference; on every route (397: eight-wave
    resident, 600: eight-wave two-stage, 1101: four-wave, 910 with 64 heads: two query groups per
    wave (512 workgroups of 128 queries; 910 with 128 heads and 397 with 256 heads, the batch-16
    shape, 1024 workgroups in more than one round)). Held against a float64 softmax of the operands
    as the kernel holds them: q rounded to f16 after the softmax scale and log2(e) are folded in, k
    and v rounded to f16."""
    r = rng(97 + S)
    H = nh * 64
    qkv = (r.standard_normal((S, 3 * H)) * 0.3).astype(np.float32)
    ramp = ((np.arange(S) - S / 2) / 64.0 * 8.4 * sign).astype(np.float32)   # natural-log units
    for h in range(nh):
        qkv[:, h * 64] = 4.0                   # q . k gains 4 * 2 * ramp, times the scale 1/8
        qkv[:, H + h * 64] = 2.0 * ramp
    out = rt.array(np.full((S, H), np.nan, np.float32))
    rt.attention(rt.array(qkv), out, S, nh, 64, 3 * H, H, 0, H, 2 * H, 0, 0.125)
    rt.sync()
    o = out.numpy()
    assert not np.isnan(o).any()
    c = np.float32(0.125 * 1.4426950408889634)
    q = (qkv[:, :H] * c).astype(np.float16).astype(np.float64)
    k = qkv[:, H:2 * H].astype(np.float16).astype(np.float64)
    v = qkv[:, 2 * H:].astype(np.float16).astype(np.float64)
    ref = np.zeros((S, H))
    for h in range(nh):
        sl = slice(h * 64, (h + 1) * 64)
        s2 = q[:, sl] @ k[:, sl].T                        # log2 units
        p = np.exp2(s2 - s2.max(1, keepdims=True))
        ref[:, sl] = (p @ v[:, sl]) / p.sum(1, keepdims=True)
    assert rel_l2(o, ref) < 3e-3


def test_launcher_surface_rest(tsn, rt, orc):
    """geglu, gelu_quick, ln_plain, ln_wb, rms_w, mean_cols and qkv_split3 against the oracle"""
    r = rng(71)
    n = 5 * 1024 + 3
    a, b = (3 * r.standard_normal(n)).astype(np.float32), r.standard_normal(n).astype(np.float32)
    y = rt.empty((n,))
    rt.geglu(rt.array(a), rt.array(b), y, n); rt.sync()
    assert rel_l2(y.numpy(), orc.geglu(a, b)) < 1e-6
    xa = rt.array(a)
    rt.gelu_quick(xa, n); rt.sync()
    assert rel_l2(xa.numpy(), orc.gelu_quick(a)) < 1e-6
    S, H = 77, 1024
    x = (1.5 + 2 * r.standard_normal((S, H))).astype(np.float32)
    w, bb = (1 + 0.1 * r.standard_normal(H)).astype(np.float32), r.standard_normal(H).astype(np.float32)
    xd, yd = rt.array(x), rt.empty((S, H))
    rt.ln_plain(xd, yd, S, H, 1e-5); rt.sync()
    assert rel_l2(yd.numpy(), orc.ln_plain(x, 1e-5)) < 1e-5
    rt.ln_wb(xd, yd, rt.array(w), rt.array(bb), S, H, 1e-5); rt.sync()
    assert rel_l2(yd.numpy(), orc.ln_wb(x, w, bb, 1e-5)) < 1e-5
    rt.rms_w(xd, yd, rt.array(w), S, H, 1e-6); rt.sync()
    assert rel_l2(yd.numpy(), orc.rms_w(x, w, 1e-6)) < 1e-5
    m = rt.empty((H,))
    rt.mean_cols(xd, m, S, H); rt.sync()
    assert rel_l2(m.numpy(), orc.mean_cols(x)) < 1e-6
    rows, Hq, off = 141, 1024, 64
    src = r.standard_normal((rows, 3 * Hq)).astype(np.float32)
    dst0 = np.full((rows + off, 3 * Hq), -7.0, np.float32)
    dd = rt.array(dst0)
    rt.qkv_split3(rt.array(src), dd, rows, Hq, off); rt.sync()
    assert np.array_equal(dd.numpy(), orc.qkv_split3(src, dst0, off))
