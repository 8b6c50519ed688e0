"""GPU parity of the 2:4 sparse-MFMA GEMMs.

int8: int32 accumulators and requantised int8 are bit-exact against the
oracle (quantized_matmul + quantize_tensor) and the golden vectors written
by the compiled reference; at the full 11008 x 4096 x 512 size every row and
every column is pinned by exact integer sum identities, and a sample of rows
by the oracle.  bf16: operands rounded by the oracle's from_float (its
sign quirk included); fp32 outputs within 1e-4 of sum |w| |x| of the
float64 product of those operands (products of bf16 values are exact in
fp32; the MFMA sums in a different order, so bit equality is not
expected), infinities and NaN exactly where it has them.
"""
import sys

import numpy as np
import pytest

from oracle import oracle as O
from pyflamert_amd import _lib, workloads

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    from pyflamert_amd import rocm

    c = rocm.Context(0)
    yield c
    c.close()


def rand_24_int8(rng, M, K, zero_frac=0.0):
    w = rng.standard_normal((M, K)).astype(np.float32)
    w = O.orc_apply_mask(w, O.orc_nm_mask(w.ravel(), 2, 4).reshape(M, K))
    if zero_frac:
        w[rng.random(w.shape) < zero_frac] = 0.0
    s, _ = O.orc_dynamic_params_per_channel(w.reshape(1, M, K))
    q = O.orc_quantize(w, s, np.zeros(M, np.int32), O.I8, (1, M, K))
    return q, s


# (1600, 512, 4096) and (1600, 300, 4000): a grid of more than one
# workgroup per CU (row-major X and transposed X)
@pytest.mark.parametrize("M,K,N", [(16, 128, 16), (200, 300, 70), (128, 4096, 512), (33, 257, 1),
                                   (1600, 512, 4096), (1600, 300, 4000)])
def test_i8_accumulators_exact(ctx, M, K, N):
    rng = np.random.default_rng(M * 7 + K)
    K4 = (K + 3) // 4 * 4
    q, s = rand_24_int8(rng, M, K4, zero_frac=0.1)
    q = np.ascontiguousarray(q[:, :K])
    X = rng.integers(-128, 128, (K, N)).astype(np.int8)
    say(f"sp24 i8 acc M={M} K={K} N={N}")
    W = ctx.sp24_pack(q, s)
    Y = W.gemm_i8(X, out="i32")
    assert np.array_equal(Y, O.orc_int8_matmul_acc(q, X))


def test_i8_register_streamed_forms(ctx):
    """K = 4096 with N a multiple of 128 and a row-major X runs the kernel
    that streams the weight into registers (32 k steps): ragged M, every
    output form (int32 accumulators, float, requantised int8 with a zero
    point) and a uint8 activation with a zero point, against the oracle and
    exact int64 products."""
    rng = np.random.default_rng(21)
    M, K, N = 700, 4096, 256
    q, s = rand_24_int8(rng, M, K, zero_frac=0.1)
    X = rng.integers(-128, 128, (K, N)).astype(np.int8)
    say(f"sp24 i8 register-streamed M={M} K={K} N={N}")
    W = ctx.sp24_pack(q, s)
    assert np.array_equal(W.gemm_i8(X, out="i32"), O.orc_int8_matmul_acc(q, X))
    F = W.gemm_i8(X, x_scale=0.05, out="f32")
    R = O.orc_quantized_matmul_rowscale(q, X, s, 0.05)
    assert np.array_equal(F.view(np.uint32), R.view(np.uint32))
    os_, oz = O.orc_dynamic_params(R)
    Q = W.gemm_i8(X, x_scale=0.05, out="i8", out_scale=float(os_), out_zp=int(oz))
    assert np.array_equal(Q, O.orc_quantize(R, [os_], [oz], O.I8))
    Xu = rng.integers(0, 256, (K, N)).astype(np.uint8)
    Yu = W.gemm_q(Xu, 1.0, 131, out="i32")
    assert np.array_equal(Yu.astype(np.int64), q.astype(np.int64) @ (Xu.astype(np.int64) - 131))


def test_i8_register_streamed_strided_outputs(ctx):
    """The register-streamed kernel (K = 4096, N a multiple of 128) with an
    output row stride that is not a multiple of 16 elements, so its
    epilogues store element by element: int32, float and requantised int8
    into the first N columns of wider rows, the padding left untouched."""
    import torch

    rng = np.random.default_rng(23)
    M, K, N, pad = 300, 4096, 128, 3
    q, s = rand_24_int8(rng, M, K, zero_frac=0.1)
    X = rng.integers(-128, 128, (K, N)).astype(np.int8)
    say(f"sp24 i8 register-streamed strided outputs M={M} N={N} ldy={N + pad}")
    W = ctx.sp24_pack(q, s)
    dX = torch.from_numpy(X).cuda()
    acc = O.orc_int8_matmul_acc(q, X)
    R = O.orc_quantized_matmul_rowscale(q, X, s, 0.05)
    os_, oz = O.orc_dynamic_params(R)
    want = {"i32": acc, "f32": R, "i8": O.orc_quantize(R, [os_], [oz], O.I8)}
    for out, dt, fill in (("i32", torch.int32, 7), ("f32", torch.float32, 7.0), ("i8", torch.int8, 7)):
        dY = torch.full((M, N + pad), fill, dtype=dt, device="cuda")
        torch.cuda.synchronize()
        W.gemm_i8_dev(dX.data_ptr(), N, dY.data_ptr(), x_scale=0.05, out=out, out_scale=float(os_),
                      out_zp=int(oz), ldy=N + pad)
        torch.cuda.synchronize()
        Y = dY.cpu().numpy()
        got, w = Y[:, :N], want[out]
        if out == "f32":
            assert np.array_equal(got.view(np.uint32), w.view(np.uint32)), out
        else:
            assert np.array_equal(got, w), out
        assert (Y[:, N:] == fill).all(), out


def test_i8_rowscale_float_and_requant(ctx):
    rng = np.random.default_rng(11)
    M, K, N = 96, 512, 80
    q, s = rand_24_int8(rng, M, K)
    X = O.orc_quantize(rng.standard_normal((K, N)).astype(np.float32), [0.05], [0], O.I8)
    say("sp24 i8 per-row scales: float and requant outputs")
    W = ctx.sp24_pack(q, s)
    F = W.gemm_i8(X, x_scale=0.05, out="f32")
    R = O.orc_quantized_matmul_rowscale(q, X, s, 0.05)
    assert np.array_equal(F.view(np.uint32), R.view(np.uint32))
    os_, oz = O.orc_dynamic_params(R)
    for zp in (0, 3, -5):
        Q = W.gemm_i8(X, x_scale=0.05, out="i8", out_scale=float(os_), out_zp=zp)
        assert np.array_equal(Q, O.orc_quantize(R, [os_], [zp], O.I8)), zp
    # scale small enough that outputs saturate and round half away at .5
    Q = W.gemm_i8(X, x_scale=0.05, out="i8", out_scale=float(os_) / 7.0, out_zp=0)
    assert np.array_equal(Q, O.orc_quantize(R, [np.float32(os_) / np.float32(7.0)], [0], O.I8))


def test_i8_requant_extreme_scales(ctx):
    """Requantisation at output scales that push RN(RN((float)acc * s) * (1 /
    out_scale)) past the int32 range or to infinity: quantize_tensor's x86
    cast gives INT32_MIN there, so -128 after the clamp, whatever the sign
    (quant_ops.cpp:42-47); and at a scale where it stays in range.  Both
    requant forms of the kernel (the bounded one and the one with the range
    select) against the oracle."""
    rng = np.random.default_rng(13)
    M, K, N = 300, 1024, 128
    q, s = rand_24_int8(rng, M, K)
    X = O.orc_quantize(rng.standard_normal((K, N)).astype(np.float32), [0.05], [0], O.I8)
    W = ctx.sp24_pack(q, s)
    R = O.orc_quantized_matmul_rowscale(q, X, s, 0.05)
    for os_ in (1e-30, 1e-12, 2e-9, 3e-6, 0.05, 7.0):
        say(f"sp24 i8 requant out_scale={os_}")
        Q = W.gemm_i8(X, x_scale=0.05, out="i8", out_scale=os_, out_zp=0)
        assert np.array_equal(Q, O.orc_quantize(R, [np.float32(os_)], [0], O.I8)), os_


def test_i8_golden(ctx, golden):
    """quantized_matmul with a per-tensor 2:4 weight and its requant, exactly
    as the compiled reference produced them."""
    g = golden("qmatmul.npz")
    say("sp24 golden qmatmul")
    W = ctx.sp24_pack(g["sp_wq"], [g["sp_ws"]])
    F = W.gemm_i8(g["sp_xq"], x_scale=0.05, out="f32")
    assert np.array_equal(F.view(np.uint32), g["sp_yf"].view(np.uint32))
    ys, yz = g["sp_y_params"]
    Q = W.gemm_i8(g["sp_xq"], x_scale=0.05, out="i8", out_scale=float(ys), out_zp=int(yz))
    assert np.array_equal(Q, g["sp_yq"])


def test_i8_full_size_properties(ctx):
    """W 11008 x 4096 (2:4, per-row int8), X 4096 x 512 int8 (scale 0.05):
    every int32 accumulator against the exact product (a float64 BLAS product
    of the int8 operands is exact here: every partial sum is below
    4096 * 128^2 < 2^53), the float output of every row, (float)acc *
    RN(s_row * 0.05) as quantized_matmul computes it (quant_ops.cpp:435,
    :456-466), and every requantised int8 output against orc_quantize
    (quant_ops.cpp:15-127); plus the exact row and column sums and 192 rows
    against the oracle's own loops."""
    M, K, N = 11008, 4096, 512
    say("sp24 full size: generating")
    q, s = workloads.sp24_int8_weight(M, K, seed=3)
    X = workloads.quantize_per_tensor(workloads.dense_normal((K, N), 1.0, seed=4), 0.05)
    W = ctx.sp24_pack(q, s)
    say("sp24 full size: int32")
    Y = W.gemm_i8(X, out="i32")
    q64, x64 = q.astype(np.int64), X.astype(np.int64)
    assert np.array_equal(Y.astype(np.int64).sum(axis=1), q64 @ x64.sum(axis=1))
    assert np.array_equal(Y.astype(np.int64).sum(axis=0), q64.sum(axis=0) @ x64)
    rows = np.random.default_rng(5).choice(M, 192, replace=False)
    rows.sort()
    acc = O.orc_int8_matmul_acc(q[rows], X)
    assert np.array_equal(Y[rows], acc)
    say("sp24 full size: every accumulator against the float64 product")
    exact = q.astype(np.float64) @ X.astype(np.float64)
    assert np.array_equal(Y.astype(np.float64), exact)
    del exact
    say("sp24 full size: float output, every row")
    F_ref = (Y.astype(np.float32) * (s * np.float32(0.05)).astype(np.float32)[:, None]).astype(np.float32)
    assert np.array_equal(O.orc_quantized_matmul_rowscale(q[rows], X, s[rows], 0.05).view(np.uint32),
                          F_ref[rows].view(np.uint32))
    Fg = W.gemm_i8(X, x_scale=0.05, out="f32")
    assert np.array_equal(Fg.view(np.uint32), F_ref.view(np.uint32))
    say("sp24 full size: requantised int8, every row")
    os_, _ = O.orc_dynamic_params(F_ref)
    Q = W.gemm_i8(X, x_scale=0.05, out="i8", out_scale=float(os_), out_zp=0)
    assert np.array_equal(Q, O.orc_quantize(F_ref, [os_], [0], O.I8))


NEG_CARRY = np.float32(np.array([0xBF80C000], np.uint32).view(np.float32)[0])  # bf16 from_float: -inf
NEG_DOWN = np.float32(np.array([0xBF803FFF], np.uint32).view(np.float32)[0])   # rounds down to -1


def round_down_negatives(a):
    """Negative values with bit 15 cleared: their bf16 rounding never carries
    out of the low half, where from_float's sign quirk would make them -inf
    (half of all negative floats); positive values keep their RNE carries."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).copy()
    u[(u >> 31) == 1] &= np.uint32(0xFFFF7FFF)
    return u.view(np.float32)


def bf16_operands(rng, M, K, N, quirk):
    """A 2:4 weight and an activation rounded by the reference's
    BFloat16::from_float (half_types.cpp:132-174, the oracle's
    orc_f32_to_bf16): positive values round to nearest even (carries
    included), negative ones round down; with quirk, three kept weights are
    negatives whose rounding carries, which from_float makes -inf, and some
    activations are the round-down case next to it."""
    w = round_down_negatives(rng.standard_normal((M, K)).astype(np.float32))
    w = O.orc_apply_mask(w, O.orc_nm_mask(w.ravel(), 2, 4).reshape(M, K))
    x = round_down_negatives(rng.standard_normal((K, N)).astype(np.float32))
    if quirk:
        kept = np.argwhere(w != 0)
        for r, k in kept[rng.choice(len(kept), 3, replace=False)]:
            w[r, k] = NEG_CARRY
        x[rng.random(x.shape) < 0.01] = NEG_DOWN
    wb = O.orc_f32_to_bf16(w.ravel()).reshape(M, K)
    xb = O.orc_f32_to_bf16(x.ravel()).reshape(K, N)
    if quirk:
        assert (wb == 0xFF80).sum() == 3
    return wb, xb


def check_bf16(Y, wb, xb, rows=None):
    """Y against the float64 product of the bf16 operands (products of bf16
    values are exact in fp32, so only the fp32 sums differ): infinities and
    NaN where it has them, finite outputs within 1e-4 of sum |w| |x|."""
    wf = O.orc_bf16_to_f32(wb).astype(np.float64)
    xf = O.orc_bf16_to_f32(xb).astype(np.float64)
    if rows is not None:
        wf, Y = wf[rows], Y[rows]
    with np.errstate(invalid="ignore", over="ignore"):
        R = wf @ xf
        S = np.abs(wf) @ np.abs(xf)
    assert np.array_equal(np.isnan(Y), np.isnan(R))
    inf = np.isinf(R)
    assert np.array_equal(Y[inf], R[inf])
    ok = np.isfinite(R)
    assert (np.abs(Y[ok] - R[ok]) <= 1e-4 * S[ok] + 1e-30).all(), np.abs(Y[ok] - R[ok]).max()
    return R


# K % 256 == 0 with N % 128 == 0 reads X rows directly (ds_read_b64_tr_b16);
# the others go through the transposed copy
@pytest.mark.parametrize("M,K,N,quirk", [(64, 128, 64, False), (200, 512, 96, True), (33, 300, 70, True),
                                         (1024, 2048, 256, False), (300, 1028, 129, True), (256, 512, 128, True)])
def test_bf16_within_tolerance(ctx, M, K, N, quirk):
    import torch

    rng = np.random.default_rng(M + K + N)
    wb, xb = bf16_operands(rng, M, K, N, quirk)
    say(f"sp24 bf16 M={M} K={K} N={N} quirk={quirk}")
    W = ctx.sp24_pack(wb)
    Y = W.gemm_bf16(xb)
    R = check_bf16(Y, wb, xb)
    # device pointers, X rows 8 elements longer than N and Y rows 3 longer
    dX = torch.from_numpy(np.concatenate([xb, np.zeros((K, 8), np.uint16)], 1).view(np.int16)).cuda()
    dY = torch.zeros((M, N + 3), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    W.gemm_bf16_dev(dX.data_ptr(), N, dY.data_ptr(), ldx=N + 8, ldy=N + 3)
    ctx.synchronize()
    Yd = dY.cpu().numpy()
    assert np.array_equal(Yd[:, :N].view(np.uint32), Y.view(np.uint32)) and not Yd[:, N:].any()
    # and the composition with the reference's dense cpu_gemm on those operands
    F32 = O.orc_gemm(O.orc_bf16_to_f32(wb), O.orc_bf16_to_f32(xb))
    assert np.array_equal(np.isnan(F32), np.isnan(R)) and np.array_equal(F32[np.isinf(R)], R[np.isinf(R)])
    W.free()


def test_bf16_full_size(ctx):
    """11008 x 4096 x 512 (the 2:4 benchmark shape) with the from_float
    quirk in the weight: every output against the float64 product."""
    rng = np.random.default_rng(3)
    M, K, N = 11008, 4096, 512
    wb, xb = bf16_operands(rng, M, K, N, True)
    say("sp24 bf16 full size 11008 x 4096 x 512")
    W = ctx.sp24_pack(wb)
    Y = W.gemm_bf16(xb)
    check_bf16(Y, wb, xb)
    W.free()


def test_rejects_non_24(ctx):
    say("sp24 argument errors")
    w = np.zeros((16, 8), np.int8)
    w[3, 4:7] = 1  # three nonzeros in one group
    with pytest.raises(_lib.InvalidArgument, match="not 2:4 sparse: row 3, k 4..7"):
        ctx.sp24_pack(w, [1.0])
    with pytest.raises(_lib.InvalidArgument, match="scales"):
        ctx.sp24_pack(np.zeros((16, 8), np.int8), np.ones(3, np.float32))
    W = ctx.sp24_pack(np.zeros((16, 8), np.int8), [1.0])
    with pytest.raises(ValueError, match="inner dimensions"):
        W.gemm_i8(np.zeros((9, 4), np.int8))
    with pytest.raises(_lib.InvalidArgument, match="output scale"):
        W.gemm_i8(np.zeros((8, 4), np.int8), x_scale=1.0, out="i8", out_scale=0.0)
