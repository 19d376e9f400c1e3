"""tsn_gemm_noalloc: the allocation-free variant of tsn_gemm (the f32-X hi|lo split in a fixed
per-GPU device array instead of the runtime's grow-on-demand scratch) gives tsn_gemm's results bit
for bit, on two calls in a row with the second one smaller, and refuses shapes beyond its array
with an argument error before touching the GPU."""
import numpy as np
import pytest

from conftest import f16r, rel_l2, rng

pytestmark = pytest.mark.gpu

F32, F16 = 0, 1


def _case(rt, r, M, N, K, ydt):
    X = r.standard_normal((M, K)).astype(np.float32)
    W = (r.standard_normal((N, K)) * 0.03).astype(np.float16)
    b = r.standard_normal(N).astype(np.float32)
    return X, W, b


def test_gemm_noalloc_matches_gemm(tsn, rt):
    r = rng(123)
    # second call smaller than the first: the array keeps the first call's contents beyond the
    # second's operand, which the second must not read
    # (282, 1024, 4096): a long K over 24 tiles, split into the runtime's fixed workspace
    for (M, N, K, ydt) in [(794, 4096, 1024, F32), (130, 1024, 512, F32), (256, 3072, 1024, F16),
                           (282, 1024, 4096, F32)]:
        X, W, b = _case(rt, r, M, N, K, ydt)
        Xd, Wd, bd = rt.array(X), rt.array(W), rt.array(b)
        ynp = np.float16 if ydt == F16 else np.float32
        Y0 = rt.array(np.full((M, N), np.nan, ynp))
        Y1 = rt.array(np.full((M, N), np.nan, ynp))
        rt.gemm(F16, Wd, Xd, F32, Y0, ydt, bd, M, N, K)
        rt.gemm_noalloc(F16, Wd, Xd, F32, Y1, ydt, bd, M, N, K)
        rt.sync()
        y0, y1 = Y0.numpy(), Y1.numpy()
        assert np.array_equal(y0.view(np.uint16 if ydt == F16 else np.uint32), y1.view(np.uint16 if ydt == F16 else np.uint32))
        ref = X.astype(np.float64) @ W.astype(np.float64).T + b
        assert rel_l2(y1.astype(np.float32), ref) < (1e-3 if ydt == F16 else 2e-5)


def test_gemm_noalloc_other_routes_and_limit(tsn, rt):
    r = rng(7)
    # f16 X (plain f16 product) and a shape outside the MFMA tiling (K % 64 != 0: exact SIMT path)
    for (M, N, K, xdt) in [(100, 256, 256, F16), (33, 200, 72, F32)]:
        X, W, b = _case(rt, r, M, N, K, F32)
        Xd = rt.array(X.astype(np.float16) if xdt == F16 else X)
        Wd, bd = rt.array(W), rt.array(b)
        Y0, Y1 = rt.empty((M, N)), rt.empty((M, N))
        rt.gemm(F16, Wd, Xd, xdt, Y0, F32, bd, M, N, K)
        rt.gemm_noalloc(F16, Wd, Xd, xdt, Y1, F32, bd, M, N, K)
        rt.sync()
        assert np.array_equal(Y0.numpy().view(np.uint32), Y1.numpy().view(np.uint32))
        Xr = f16r(X) if xdt == F16 else X
        assert rel_l2(Y1.numpy(), Xr.astype(np.float64) @ W.astype(np.float64).T + b) < 2e-5
    # beyond the array: an argument error, checked on the host before any launch
    cap = rt.gemm_noalloc_max_elems()
    assert cap == (32 << 20) // 4
    M, K = 4096, 4096                      # M*K = 16 Mi elements > 8 Mi
    assert M * K > cap
    Wd, Xd, Yd = rt.empty((64, K), np.float16), rt.empty((M, K)), rt.empty((M, 64))
    with pytest.raises(tsn.TsnError) as e:
        rt.gemm_noalloc(F16, Wd, Xd, F32, Yd, F32, None, M, 64, K)
    assert e.value.code == 1 and "static scratch" in str(e.value)


def test_gemm_noalloc_allocates_nothing_on_a_fresh_runtime(tsn):
    """On a runtime that has never run tsn_gemm (so its grow-on-demand scratch does not exist), the
    hi|lo route of tsn_gemm_noalloc leaves the runtime's allocations exactly as they were; a later
    tsn_gemm of the same shape grows the scratch (so the accessor does see it) and gives the same
    bits."""
    r = rng(321)
    M, N, K = 512, 1024, 1024
    X, W, b = _case(None, r, M, N, K, F32)
    with tsn.Runtime(0) as rt2:
        Xd, Wd, bd = rt2.array(X), rt2.array(W), rt2.array(b)
        Y1, Y0 = rt2.empty((M, N)), rt2.empty((M, N))
        before = rt2.alloc_stats()
        rt2.gemm_noalloc(F16, Wd, Xd, F32, Y1, F32, bd, M, N, K)
        rt2.sync()
        assert rt2.alloc_stats() == before
        rt2.gemm(F16, Wd, Xd, F32, Y0, F32, bd, M, N, K)
        rt2.sync()
        cnt, nbytes = rt2.alloc_stats()
        assert cnt == before[0] + 1 and nbytes >= before[1] + 4 * M * K
        assert np.array_equal(Y0.numpy().view(np.uint32), Y1.numpy().view(np.uint32))
        ref = X.astype(np.float64) @ W.astype(np.float64).T + b
        assert rel_l2(Y1.numpy(), ref) < 2e-5
        for a in (Xd, Wd, bd, Y1, Y0):
            a.free()


def test_gemm_noalloc_two_runtimes_in_a_row(tsn, rt):
    """Two runtimes (two streams) share the per-GPU array: back-to-back calls from both, with no
    host synchronisation between them, are ordered on the device and each matches tsn_gemm."""
    r = rng(99)
    shapes = [(794, 3072, 1024), (600, 1024, 2048)]
    with tsn.Runtime(0) as rt2:
        runs = []
        for (M, N, K), R in zip(shapes, (rt, rt2)):
            X, W, b = _case(None, r, M, N, K, F32)
            runs.append((R, M, N, K, R.array(X), R.array(W), R.array(b), R.empty((M, N)), R.empty((M, N))))
        for R, M, N, K, Xd, Wd, bd, Y0, Y1 in runs:
            R.gemm(F16, Wd, Xd, F32, Y0, F32, bd, M, N, K)
        rt.sync()
        rt2.sync()
        for _ in range(3):
            for R, M, N, K, Xd, Wd, bd, Y0, Y1 in runs:
                R.gemm_noalloc(F16, Wd, Xd, F32, Y1, F32, bd, M, N, K)
        rt.sync()
        rt2.sync()
        for R, M, N, K, Xd, Wd, bd, Y0, Y1 in runs:
            assert np.array_equal(Y0.numpy().view(np.uint32), Y1.numpy().view(np.uint32))
            for a in (Xd, Wd, bd, Y0, Y1):
                a.free()
