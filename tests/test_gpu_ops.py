"""GPU parity of every per-op entry point against the oracle, through the
C ABI, on seeded inputs. Integer/byte work is checked bit-exact; floating
point to the tolerance stated in each test."""
import numpy as np
import pytest

import mxenc
from mxenc import from_bf16_bits, to_bf16_bits
from orc import P

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = mxenc.Context(0)
    yield c
    c.close()


def test_device_is_mi355x(ctx):
    assert ctx.props.arch.decode().startswith("gfx950")
    assert ctx.props.compute_units >= 256


# ---- narrow_f32_bf16: bit-exact with the host's to_bf16 ----------------------

def test_narrow_f32_bf16_bit_exact(ctx, orc):
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x4000, 0xC000], np.uint32)
    rng = np.random.default_rng(0)
    bits = np.concatenate([(hi[:, None] | lows[None, :]).reshape(-1),
                           rng.integers(0, 1 << 32, 1 << 22, dtype=np.uint64).astype(np.uint32)])
    x = bits.view(np.float32)
    want = np.empty(x.size, np.uint16)
    orc.orc_bf16_fill(P(want), P(bits), x.size)
    dx = ctx.put(bits)
    out = ctx.empty(x.shape, np.uint16)
    mxenc.narrow_f32_bf16(ctx, dx, out)
    got = out.host()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"bits {bits[bad[0]]:#x}: {got[bad[0]]:#x} != {want[bad[0]]:#x}"


def test_narrow_f32_bf16_tails_and_misaligned(ctx, orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 1 << 32, 1031, dtype=np.uint64).astype(np.uint32)
    want = np.empty(bits.size, np.uint16)
    orc.orc_bf16_fill(P(want), P(bits), bits.size)
    dx = ctx.put(bits)
    out = ctx.empty((bits.size,), np.uint16)
    # odd length: vector body + scalar tail
    mxenc.check(mxenc.lib().mx_narrow_f32_bf16(ctx.stream, dx.p, out.p, bits.size))
    assert np.array_equal(out.host(), want)
    # one element in: misaligned pointers take the scalar kernel
    mxenc.check(mxenc.lib().mx_narrow_f32_bf16(ctx.stream, dx.offset(1), out.offset(1),
                                               bits.size - 1))
    assert np.array_equal(out.host()[1:], want[1:])


def test_narrow_i32_bf16_single_rounding(ctx, orc):
    rng = np.random.default_rng(2)
    v = np.concatenate([rng.integers(-2**31, 2**31, 1 << 20, dtype=np.int64),
                        rng.integers(-5000, 5000, 4096),
                        [0, 1, -1, 255, 256, 257, 2**24 + 1, 2**24 + 2**16 + 2**15 + 1,
                         2**31 - 1, -2**31]]).astype(np.int32)
    want = np.empty(v.size, np.uint16)
    orc.orc_narrow_i32_bf16(P(v), P(want), v.size)
    dv = ctx.put(v)
    out = ctx.empty(v.shape, np.uint16)
    mxenc.narrow_i32_bf16(ctx, dv, out)
    assert np.array_equal(out.host(), want)


# ---- GELU ----------------------------------------------------------------------

def test_gelu_poly_fp32_bit_exact(ctx, orc):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(1 << 20).astype(np.float32) * 3,
                        np.array([0, -0.0, 4, -4, 3.9999, 1e30, -1e30, np.inf], np.float32)])
    want = x.copy()
    orc.orc_gelu_poly_inplace(P(want), want.size)
    dx = ctx.put(x)
    mxenc.gelu(ctx, dx, dx, mxenc.MX_GELU_POLY)  # in place
    assert np.array_equal(dx.host().view(np.uint32), want.view(np.uint32))


def test_gelu_erf_fp32(ctx, orc):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(1 << 18) * 4).astype(np.float32)
    want = x.copy()
    orc.orc_gelu_erf_inplace(P(want), want.size)
    dx = ctx.put(x)
    dy = ctx.empty(x.shape, np.float32)
    mxenc.gelu(ctx, dx, dy, mxenc.MX_GELU_ERF)
    got = dy.host()
    # fp32 erff against the host's double erf rounded once: a few ulp
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-30)) < 1e-5 or \
        np.max(np.abs(got - want)) < 1e-6


def test_gelu_erf_as_bf16_matches_aie_restatement(ctx, orc):
    x = np.linspace(-12, 12, 1 << 16, dtype=np.float32)
    xb = to_bf16_bits(x)
    want = np.empty_like(xb)
    orc.orc_aie_gelu_erf_bf16(P(xb), P(want), xb.size)
    dx = ctx.put(xb)
    dy = ctx.empty(xb.shape, np.uint16)
    mxenc.gelu(ctx, dx, dy, mxenc.MX_GELU_ERF_AS)
    assert np.array_equal(dy.host(), want)


def test_gelu_poly_bf16_vs_aie_kernel(ctx, orc):
    """bf16 in/out: the fused-FMA polynomial against gelu_poly_rne.cc's
    multiply-then-add. Where the output is not small they are at most one bf16
    ulp apart. Near |x| = 4 the polynomial cancels to ~3e-4 from terms of size
    ~0.5 and each Horner step's rounding is amplified by u^(8-k) ~ 4^7, so the
    two evaluation orders differ by up to ~4e-6 absolute there (two bf16 ulps
    of a 3e-4 output); 1e-5 absolute bounds that."""
    x = np.linspace(-9, 9, 1 << 16, dtype=np.float32)
    xb = to_bf16_bits(x)
    want = np.empty_like(xb)
    orc.orc_aie_gelu_poly_bf16(P(xb), P(want), xb.size)
    dx = ctx.put(xb)
    dy = ctx.empty(xb.shape, np.uint16)
    mxenc.gelu(ctx, dx, dy, mxenc.MX_GELU_POLY)
    got = dy.host()
    wf, gf = from_bf16_bits(want), from_bf16_bits(got)
    big = np.abs(wf) >= 1e-2
    assert np.max(np.abs(got[big].astype(np.int32) - want[big].astype(np.int32))) <= 1
    assert np.max(np.abs(gf[~big] - wf[~big])) <= 1e-5
    # and the fp32-then-narrow result is the host gelu_cpu's, narrowed, bit for bit
    f = from_bf16_bits(xb).copy()
    orc.orc_gelu_poly_inplace(P(f), f.size)
    assert np.array_equal(got, to_bf16_bits(f))


# ---- LayerNorm -----------------------------------------------------------------

@pytest.mark.parametrize("cols", [384, 768, 1024, 1280, 200])
def test_layernorm_residual_fused(ctx, orc, cols):
    rng = np.random.default_rng(cols)
    rows = 1000
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    y = (rng.standard_normal((rows, cols)) * 0.5).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cols)).astype(np.float32)
    want = np.empty_like(x)
    orc.orc_add_into(P(want), P(y), P(x), x.size)
    if cols % 8 == 0:
        orc.orc_layer_norm_rows(P(want), rows, cols, P(g), P(b), 1e-12)
    else:
        orc.orc_layernorm_rows_f64(P(want), rows, cols, P(g), P(b), 1e-12)
    dx, dy, dg, db = ctx.put(x), ctx.put(y), ctx.put(g), ctx.put(b)
    of = ctx.empty(x.shape, np.float32)
    ob = ctx.empty(x.shape, np.uint16)
    mxenc.layernorm(ctx, dx, dy, dg, db, 1e-12, rows, cols, out_f32=of, out_bf16=ob)
    got = of.host()
    assert np.max(np.abs(got - want)) < 2e-5
    # the bf16 copy is the fp32 result narrowed by to_bf16, bit for bit
    assert np.array_equal(ob.host(), to_bf16_bits(got))
    # in place over the residual stream, with the bf16 copy as the stack writes
    # it (the form whose accesses stream, nontemporal): the same bits
    ob2 = ctx.empty(x.shape, np.uint16)
    mxenc.layernorm(ctx, dx, dy, dg, db, 1e-12, rows, cols, out_f32=dx, out_bf16=ob2)
    assert np.array_equal(dx.host(), got)
    assert np.array_equal(ob2.host(), ob.host())


def test_layernorm_bf16_input(ctx, orc):
    rng = np.random.default_rng(9)
    rows, cols = 257, 768
    x = to_bf16_bits(rng.standard_normal((rows, cols)).astype(np.float32))
    g = np.ones(cols, np.float32)
    b = np.zeros(cols, np.float32)
    want = from_bf16_bits(x).copy()
    orc.orc_layernorm_rows_f64(P(want), rows, cols, P(g), P(b), 1e-5)
    dx, dg, db = ctx.put(x), ctx.put(g), ctx.put(b)
    of = ctx.empty((rows, cols), np.float32)
    mxenc.layernorm(ctx, dx, None, dg, db, 1e-5, rows, cols, out_f32=of)
    assert np.max(np.abs(of.host() - want)) < 2e-5


# ---- softmax -------------------------------------------------------------------

def test_softmax_poly_masked(ctx, orc):
    rng = np.random.default_rng(10)
    B, H, S = 3, 4, 128
    x = (rng.standard_normal((B * H * S, S)) * 3).astype(np.float32)
    mask = np.zeros((B, S), np.float32)
    mask[1, 70:] = -1e30
    mask[2, 5:] = -1e30
    want = x.copy()
    orc.orc_softmax_rows_poly(P(want), B * H * S, S, P(mask), H * S)
    dx, dm = ctx.put(x), ctx.put(mask)
    mxenc.softmax_rows(ctx, dx, B * H * S, S, S, dm, H * S, mxenc.MX_SOFTMAX_POLY)
    got = dx.host()
    assert np.max(np.abs(got - want)) < 1e-6
    assert np.all(got[H * S:2 * H * S, 70:] < 1e-30)


@pytest.mark.parametrize("bf", [False, True], ids=["fp32", "bf16"])
@pytest.mark.parametrize("variant", ["poly", "exact"])
@pytest.mark.parametrize("rows,cols", [(33, 8), (250, 136), (4099, 512), (18, 384), (7, 264),
                                       (1030, 1024)])
def test_softmax_16_byte_paths_against_the_host(ctx, orc, rows, cols, variant, bf):
    """The 16-byte softmax paths (sixteen lanes per row up to 512 columns, a
    wave per row group beyond) over ragged widths and row counts, masked
    tails, a fully masked row (-1e30 everywhere: uniform, as the host) and a
    row with a logit spread past the host's -120 clamp, against the host
    softmax on the same (bf16-rounded) inputs, plus one bf16 rounding for a
    bf16 output."""
    rng = np.random.default_rng(rows * 7 + cols)
    H, S = 1, cols
    B = rows
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    x[0, : cols // 2] += 150.0  # probabilities of the other half below 2^-120
    mask = np.zeros((B, S), np.float32)
    mask[min(1, B - 1), cols // 3:] = -1e30
    mask[min(2, B - 1), :] = -1e30
    if bf:
        x = from_bf16_bits(to_bf16_bits(x))
    want = x.copy()
    fn = orc.orc_softmax_rows_poly if variant == "poly" else orc.orc_softmax_rows_exact
    fn(P(want), rows, cols, P(mask), 1)
    code = mxenc.MX_SOFTMAX_POLY if variant == "poly" else mxenc.MX_SOFTMAX_EXACT
    dx, dm = ctx.put(to_bf16_bits(x) if bf else x), ctx.put(mask)
    mxenc.softmax_rows(ctx, dx, rows, cols, cols, dm, 1, code)
    got = from_bf16_bits(dx.host()) if bf else dx.host()
    # the poly variant within 1e-6 of the host; the exact one (fp32 expf
    # against the host's std::exp, another sum order) within 1e-5 relative
    # (1e-12 absolute for the tiny probabilities), as the wide-row test states
    base = 1e-6 if variant == "poly" else np.abs(want) * 1e-5 + 1e-12
    tol = base + (np.abs(want) * 2.0 ** -8 if bf else 0.0)
    assert np.all(np.abs(got - want) <= tol), np.max(np.abs(got - want) - tol)
    if rows > 2:
        assert np.allclose(got[2], 1.0 / cols, rtol=1e-2)  # fully masked: uniform
    assert np.all(got[0, cols // 2:] < 1e-30)


@pytest.mark.parametrize("cols", [197, 1500])
def test_softmax_exact_wide_rows(ctx, orc, cols):
    rng = np.random.default_rng(cols)
    rows = 300
    x = (rng.standard_normal((rows, cols)) * 4).astype(np.float32)
    want = x.copy()
    orc.orc_softmax_rows_exact(P(want), rows, cols, None, 1)
    dx = ctx.put(x)
    mxenc.softmax_rows(ctx, dx, rows, cols, cols, None, 1, mxenc.MX_SOFTMAX_EXACT)
    got = dx.host()
    # The host sums the exponentials left to right, the kernel as a tree, and
    # the two exps may differ by an ulp: relative gap ~ (cols**0.5) * 2^-24,
    # bounded here by 1e-5 (1e-12 absolute for the tiny probabilities).
    assert np.max(np.abs(got - want) / (want + 1e-7)) < 1e-5
    # and both sit within the same bound of the fp64 closed form
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(1, keepdims=True))
    exact = e / e.sum(1, keepdims=True)
    assert np.max(np.abs(got - exact) / (exact + 1e-7)) < 1e-5


def test_softmax_aie_bf16(ctx, orc):
    rng = np.random.default_rng(11)
    rows, cols = 512, 64
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    x[7, 30:] = -1e30
    xb = to_bf16_bits(x)
    want = np.empty_like(xb)
    orc.orc_aie_softmax_bf16(P(xb), P(want), rows, cols)
    dx = ctx.put(xb)
    mxenc.softmax_rows(ctx, dx, rows, cols, cols, None, 1, mxenc.MX_SOFTMAX_AIE)
    got = dx.host()
    # the same exponentials summed in the same 16-lane order: bit for bit
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows,cols", [(1, 16), (7, 48), (300, 768), (64, 4096), (17455, 64),
                                       (33, 200)])
def test_softmax_aie_bf16_shapes(ctx, orc, rows, cols):
    """The accelerator softmax at ragged and full row widths, masked tails and
    a row whose every entry is at the clamp: bit for bit."""
    rng = np.random.default_rng(rows * 31 + cols)
    x = (rng.standard_normal((rows, cols)) * 4).astype(np.float32)
    if rows > 3:
        x[1, cols // 2:] = -1e30
        x[2, :] = -3e38
    xb = to_bf16_bits(x)
    want = np.empty_like(xb)
    orc.orc_aie_softmax_bf16(P(xb), P(want), rows, cols)
    dx = ctx.put(xb)
    mxenc.softmax_rows(ctx, dx, rows, cols, cols, None, 1, mxenc.MX_SOFTMAX_AIE)
    assert np.array_equal(dx.host(), want)


LN_AIE_SHAPES = [(1, 16), (5, 384), (4096, 768), (17455, 768), (3, 1024), (9, 4096), (6, 48)]


@pytest.mark.parametrize("rows,cols", LN_AIE_SHAPES)
def test_layernorm_aie_bit_exact(ctx, orc, rows, cols):
    """mx_layernorm_aie (the K2r kernel's arithmetic) against the oracle's
    restatement, bit for bit: row scales over four decades, a constant row
    (variance 0: fast_invsqrt of eps), random gamma and beta; in place too."""
    rng = np.random.default_rng(rows + 7 * cols)
    sc = np.exp(rng.uniform(np.log(1e-2), np.log(1e2), rows)).astype(np.float32)
    x = (rng.standard_normal((rows, cols)).astype(np.float32) + 0.3) * sc[:, None]
    if rows > 2:
        x[2, :] = 1.5
    g = (1 + 0.2 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.2 * rng.standard_normal(cols)).astype(np.float32)
    xb = to_bf16_bits(x)
    for eps in (1e-12, 1e-5):
        want = np.empty_like(xb)
        orc.orc_aie_layernorm_bf16(P(xb), P(want), rows, cols, P(g), P(b), eps)
        dx, dg, db = ctx.put(xb), ctx.put(g), ctx.put(b)
        out = ctx.empty(xb.shape, np.uint16)
        mxenc.layernorm_aie(ctx, dx, dg, db, eps, rows, cols, out)
        assert np.array_equal(out.host(), want), (rows, cols, eps)
        mxenc.layernorm_aie(ctx, dx, dg, db, eps, rows, cols, dx)  # in place
        assert np.array_equal(dx.host(), want)


def test_layernorm_aie_refusals(ctx):
    x = ctx.empty((4, 40), np.uint16)
    g = ctx.empty((40,), np.float32)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        mxenc.layernorm_aie(ctx, x, g, g, 1e-5, 4, 40, x)
    y = ctx.empty((2, 8192), np.uint16)
    g2 = ctx.empty((8192,), np.float32)
    with pytest.raises(RuntimeError, match="up to 4096"):
        mxenc.layernorm_aie(ctx, y, g2, g2, 1e-5, 2, 8192, y)
    with pytest.raises(RuntimeError, match="bad eps"):
        mxenc.layernorm_aie(ctx, x, g, g, -1.0, 4, 32, x)


# ---- GEMM ------------------------------------------------------------------------

GEMM_SHAPES = [
    (77, 136, 200),      # every tail: M, N and K not multiples of the tiles
    (256, 768, 2304),    # bge-base QKV shape at small M
    (4096, 384, 1152),   # MiniLM QKV
    (512, 3072, 768),    # bge-base FFN-down
    (256, 768, 1000),    # ViT head-like N
    (1000, 1280, 3840),  # Whisper QKV, ragged M
]


@pytest.mark.parametrize("M,K,N", GEMM_SHAPES)
def test_gemm_vs_oracle(ctx, orc, M, K, N):
    rng = np.random.default_rng(M * 7 + N)
    A = to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    W = to_bf16_bits((rng.standard_normal((K, N)) * 0.05).astype(np.float32))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    Af, Wf = from_bf16_bits(A), from_bf16_bits(W)
    want = np.empty((M, N), np.float32)
    orc.orc_gemm_nt(P(np.ascontiguousarray(Af)), M, P(np.ascontiguousarray(Wf)), K, N, P(bias),
                    P(want))
    dA = ctx.put(A)
    dW = ctx.put(np.ascontiguousarray(W.T))  # [N, K] panel
    db = ctx.put(bias)
    C = ctx.empty((M, N), np.float32)
    mxenc.gemm_wt(ctx, dA, M, K, K, dW, N, db, mxenc.MX_EPI_NONE, None, C, N)
    got = C.host()
    scale = np.max(np.abs(want))
    assert np.max(np.abs(got - want)) / scale < 1e-5
    # bf16 C: the same sums narrowed once
    Cb = ctx.empty((M, N), np.uint16)
    mxenc.gemm_wt(ctx, dA, M, K, K, dW, N, db, mxenc.MX_EPI_NONE, None, Cb, N)
    gb = from_bf16_bits(Cb.host())
    rel = np.abs(gb - want) / (np.abs(want) + 1e-3 * scale)
    assert np.max(rel) < 1e-2  # the per-op GEMM bar: max relative error <= 1e-2
    assert np.array_equal(Cb.host(), to_bf16_bits(got)) or \
        np.mean(Cb.host() != to_bf16_bits(got)) < 1e-3


def test_gemm_epilogues_and_residual(ctx, orc):
    M, K, N = 300, 384, 1536
    rng = np.random.default_rng(12)
    A = to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    W = to_bf16_bits((rng.standard_normal((K, N)) * 0.05).astype(np.float32))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    base = np.empty((M, N), np.float32)
    Af, Wf = from_bf16_bits(A), from_bf16_bits(W)  # kept alive across the call
    orc.orc_gemm_nt(P(Af), M, P(Wf), K, N, P(bias), P(base))
    dA, dW, db = ctx.put(A), ctx.put(np.ascontiguousarray(W.T)), ctx.put(bias)
    C = ctx.empty((M, N), np.float32)
    for epi, fn in ((mxenc.MX_EPI_GELU_POLY, orc.orc_gelu_poly_inplace),
                    (mxenc.MX_EPI_GELU_ERF, orc.orc_gelu_erf_inplace)):
        want = base.copy()
        fn(P(want), want.size)
        mxenc.gemm_wt(ctx, dA, M, K, K, dW, N, db, epi, None, C, N)
        assert np.max(np.abs(C.host() - want)) < 1e-4
    R = (rng.standard_normal((M, N))).astype(np.float32)
    dR = ctx.put(R)
    mxenc.gemm_wt(ctx, dA, M, K, K, dW, N, db, mxenc.MX_EPI_NONE, dR, dR, N)  # in place
    assert np.max(np.abs(dR.host() - (R + base))) < 1e-4


GEMM_PATHS = [
    # M, K, N, epilogue, C dtype, residual, expected kernel
    (16384, 768, 2304, mxenc.MX_EPI_NONE, np.uint16, False, "lds_256x192"),     # QKV at M = 16384
    (16384, 768, 3072, mxenc.MX_EPI_GELU_POLY, np.uint16, False, "lds_256x256"),  # FFN-up
    (16384, 3072, 768, mxenc.MX_EPI_NONE, np.float32, False, "lds_256x192"),    # FFN-down
    (16384, 768, 768, mxenc.MX_EPI_NONE, np.float32, True, "lds_256x192"),      # x += proj
    (16000, 768, 1532, mxenc.MX_EPI_GELU_ERF, np.float32, True, "lds_256x192"),  # ragged M, N
    (4096, 384, 1536, mxenc.MX_EPI_GELU_POLY, np.uint16, False, "lds_128x256"),  # MiniLM FFN-up
    (1000, 1280, 3840, mxenc.MX_EPI_GELU_ERF, np.float32, True, "lds_128x128"),  # ragged M
    # bf16 C rows of 1004 are not 16-byte multiples: the register-staged kernel
    (777, 512, 1004, mxenc.MX_EPI_GELU_ERF, np.uint16, False, "staged_"),      # ragged M, N
    (777, 512, 1000, mxenc.MX_EPI_GELU_ERF, np.uint16, False, "lds_128x128"),   # ragged M, N
    # the 256 x 256 tile on 128-byte slabs (bf16 C, no residual, K % 64 == 0)
    (17455, 768, 2304, mxenc.MX_EPI_NONE, np.uint16, False, "lds_256x256x64"),  # packed QKV
    (17455, 3072, 768, mxenc.MX_EPI_NONE, np.uint16, False, "lds_256x256x64"),  # FFN-down
    (8000, 1024, 2000, mxenc.MX_EPI_GELU_ERF, np.uint16, False, "lds_256x256x64"),  # ragged
    (8000, 192, 2048, mxenc.MX_EPI_GELU_POLY, np.uint16, False, "lds_256x256x64"),  # 3 slabs
    # ... and an fp32 C with a residual (the pre-LN stacks; half-block staging)
    (50432, 768, 768, mxenc.MX_EPI_NONE, np.float32, True, "lds_256x256x64"),  # ViT attn-out
    (12000, 5120, 1280, mxenc.MX_EPI_NONE, np.float32, True, "lds_256x256x64"),  # Whisper down
    (8000, 1024, 2000, mxenc.MX_EPI_GELU_POLY, np.float32, True, "lds_256x256x64"),  # ragged
]


@pytest.mark.parametrize("M,K,N,epi,cdt,res,plan", GEMM_PATHS)
def test_gemm_kernel_paths(ctx, orc, M, K, N, epi, cdt, res, plan):
    """Each GEMM kernel configuration at a size that selects it, checked on a
    subset of rows (rows are independent) against the oracle's gemm_nt with
    the same epilogue: the first and last 128 rows and 128 random ones."""
    cdtype = mxenc.MX_BF16 if cdt == np.uint16 else mxenc.MX_F32
    assert mxenc.lib().mx_gemm_plan_for(M, N, K, cdtype, int(res), 0).decode().startswith(plan)
    rng = np.random.default_rng(M + K + N)
    A = to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    W = to_bf16_bits((rng.standard_normal((K, N)) * 0.05).astype(np.float32))
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32)
    R = rng.standard_normal((M, N)).astype(np.float32) if res else None
    dA, dW, db = ctx.put(A), ctx.put(np.ascontiguousarray(W.T)), ctx.put(bias)
    if res:
        dC = ctx.put(R)  # in place: C = epi(A W + b) + C
        mxenc.gemm_wt(ctx, dA, M, K, K, dW, N, db, epi, dC, dC, N)
    else:
        dC = ctx.empty((M, N), cdt)
        mxenc.gemm_wt(ctx, dA, M, K, K, dW, N, db, epi, None, dC, N)
    got = dC.host()
    rows = np.unique(np.concatenate([np.arange(128), np.arange(M - 128, M),
                                     rng.integers(0, M, 128)]))
    Af = np.ascontiguousarray(from_bf16_bits(A[rows]))
    Wf = np.ascontiguousarray(from_bf16_bits(W))
    want = np.empty((rows.size, N), np.float32)
    orc.orc_gemm_nt(P(Af), rows.size, P(Wf), K, N, P(bias), P(want))
    if epi == mxenc.MX_EPI_GELU_POLY:
        orc.orc_gelu_poly_inplace(P(want), want.size)
    elif epi == mxenc.MX_EPI_GELU_ERF:
        orc.orc_gelu_erf_inplace(P(want), want.size)
    if res:
        want += R[rows]
    g = got[rows]
    scale = np.max(np.abs(want))
    if cdt == np.uint16:
        g = from_bf16_bits(g)
        # one bf16 rounding of an fp32 result: half a bf16 ulp relative
        assert np.max(np.abs(g - want) / (np.abs(want) + 1e-3 * scale)) < 1e-2
    else:
        assert np.max(np.abs(g - want)) / scale < 1e-5


def test_gemm_refusals(ctx):
    A = ctx.empty((8, 12), np.uint16)
    W = ctx.empty((8, 12), np.uint16)
    C = ctx.empty((8, 8), np.float32)
    with pytest.raises(mxenc.MxError, match="multiples of 8"):
        mxenc.gemm_wt(ctx, A, 8, 12, 12, W, 8, None, 0, None, C, 8)


# ---- attention -------------------------------------------------------------------

def _attn_ref(orc, qkv_bits, B, S, H, hd, mask, scale=1.0):
    d = H * hd
    q = from_bf16_bits(qkv_bits).reshape(B * S, 3 * d).copy()
    out = np.empty((B * S, d), np.float32)
    if mask is None and scale != 1.0 or S % 8:
        for b in range(B):
            base = np.ascontiguousarray(q[b * S:(b + 1) * S])
            import ctypes
            o = np.empty((S, d), np.float32)
            orc.orc_whisper_attention(P(base), 3 * d, ctypes.c_void_p(base.ctypes.data + d * 4),
                                      3 * d, S, S, d, H, hd, scale, P(o))
            out[b * S:(b + 1) * S] = o
        return out
    sc = np.empty((B * H * S, S), np.float32)
    orc.orc_qk(P(q), B, S, H, hd, P(sc))
    orc.orc_softmax_rows_poly(P(sc), B * H * S, S, P(mask) if mask is not None else None, H * S)
    orc.orc_av(P(sc), P(q), B, S, H, hd, P(out))
    return out


# The attention bar, of the output's scale: the kernel writes a bf16 context
# (half an ulp: 2^-9 of a value) from bf16 probabilities into the PV product
# (each p within 2^-9, errors averaging over the keys) with the hardware exp2
# (~1e-7); the host keeps fp32 throughout. Together about 3e-3 of the largest
# output at worst; the mean error is the bf16 rounding's, ~1e-3 of the scale.
ATT_TOL = 5e-3
ATT_MEAN_TOL = 1e-3


@pytest.mark.parametrize("B,S,H,hd", [(4, 128, 3, 32), (3, 512, 2, 64), (2, 64, 12, 64)])
def test_attention_masked_vs_oracle(ctx, orc, B, S, H, hd):
    rng = np.random.default_rng(S + hd)
    d = H * hd
    qkv = to_bf16_bits((rng.standard_normal((B * S, 3 * d))).astype(np.float32))
    lens = rng.integers(1, S + 1, size=B)
    lens[0] = S
    mask = np.zeros((B, S), np.float32)
    for b, n in enumerate(lens):
        mask[b, n:] = -1e30
    kv = lens.astype(np.int32)
    want = _attn_ref(orc, qkv, B, S, H, hd, mask)
    dq, dm, dk = ctx.put(qkv), ctx.put(mask), ctx.put(kv)
    out = ctx.empty((B * S, d), np.uint16)
    for kvl in (None, dk):  # skipping masked tiles changes nothing the tolerance sees
        mxenc.attention(ctx, dq, 3 * d, B, S, H, hd, 1.0, dm, kvl, out, d)
        got = from_bf16_bits(out.host())
        err = np.abs(got - want)
        print(f"attention B{B} S{S} H{H} hd{hd}: max err / scale "
              f"{np.max(err) / np.max(np.abs(want)):.2e}, mean {np.mean(err):.2e}")
        assert np.max(err) < ATT_TOL * np.max(np.abs(want)), np.max(err)
        assert np.mean(err) < ATT_MEAN_TOL * np.max(np.abs(want))


@pytest.mark.parametrize("B,S,H,scale", [(2, 197, 3, 0.125), (1, 1500, 2, 1.0)])
def test_attention_unmasked_odd_lengths(ctx, orc, B, S, H, scale):
    hd = 64
    rng = np.random.default_rng(S)
    d = H * hd
    qkv = to_bf16_bits(rng.standard_normal((B * S, 3 * d)).astype(np.float32))
    want = _attn_ref(orc, qkv, B, S, H, hd, None, scale)
    dq = ctx.put(qkv)
    out = ctx.empty((B * S, d), np.uint16)
    mxenc.attention(ctx, dq, 3 * d, B, S, H, hd, scale, None, None, out, d)
    got = from_bf16_bits(out.host())
    err = np.abs(got - want)
    print(f"attention B{B} S{S} H{H}: max err / scale {np.max(err) / np.max(np.abs(want)):.2e}")
    assert np.max(err) < ATT_TOL * np.max(np.abs(want))


@pytest.mark.parametrize("with_mask", [False, True])
def test_attention_kvlen_holes_and_additive_mask(ctx, orc, with_mask):
    """kv_len cutting mid-tile with and without a mask row; with a mask, holes
    (-1e30) inside the sequence and finite additive values (-3, +0.5), which
    send every tile through the logits path."""
    B, S, H, hd = 3, 320, 4, 64  # S % 8 == 0: the oracle's masked qk/softmax/av form
    rng = np.random.default_rng(31 + with_mask)
    d = H * hd
    qkv = to_bf16_bits(rng.standard_normal((B * S, 3 * d)).astype(np.float32))
    lens = np.array([300, 77, 129], np.int32)
    mask = np.zeros((B, S), np.float32)
    for b, n in enumerate(lens):
        mask[b, n:] = -1e30
    if with_mask:
        mask[0, 5:9] = -1e30
        mask[1, 64] = -3.0
        mask[2, 1:100:7] = 0.5
    want = _attn_ref(orc, qkv, B, S, H, hd, mask)
    dq, dk = ctx.put(qkv), ctx.put(lens)
    out = ctx.empty((B * S, d), np.uint16)
    mxenc.attention(ctx, dq, 3 * d, B, S, H, hd, 1.0, ctx.put(mask) if with_mask else None, dk,
                    out, d)
    got = from_bf16_bits(out.host())
    err = np.abs(got - want)
    print(f"attention holes mask={with_mask}: max err / scale "
          f"{np.max(err) / np.max(np.abs(want)):.2e}")
    assert np.max(err) < ATT_TOL * np.max(np.abs(want)), np.max(err)
    assert np.mean(err) < ATT_MEAN_TOL * np.max(np.abs(want))


@pytest.mark.parametrize("hd", [64, 32])
def test_attention_key_tile_edge_lengths(ctx, orc, hd):
    """Sequence lengths on either side of the key-tile edges (32-key tiles at
    head_dim 64, 64-key tiles at 32) and -1e30 / finite mask entries inside
    middle tiles, with kv_len, against the oracle."""
    lens = np.array([1, 2, 31, 32, 33, 63, 64, 65, 95, 96, 97, 128], np.int32)
    B, S, H = len(lens), 128, 2
    d = H * hd
    rng = np.random.default_rng(101 + hd)
    qkv = to_bf16_bits(rng.standard_normal((B * S, 3 * d)).astype(np.float32))
    mask = np.zeros((B, S), np.float32)
    for b, n in enumerate(lens):
        mask[b, n:] = -1e30
    mask[8, 40] = -1e30   # a hole in the second 32-key tile
    mask[10, 70] = -2.0   # a finite entry in the third
    mask[11, 33:37] = 0.5
    want = _attn_ref(orc, qkv, B, S, H, hd, mask)
    dq, dm, dk = ctx.put(qkv), ctx.put(mask), ctx.put(lens)
    out = ctx.empty((B * S, d), np.uint16)
    mxenc.attention(ctx, dq, 3 * d, B, S, H, hd, 1.0, dm, dk, out, d)
    got = from_bf16_bits(out.host())
    scale = np.max(np.abs(want))
    for b, n in enumerate(lens):  # only the rows before kv_len are the attention's
        rows = slice(b * S, b * S + n)
        err = np.abs(got[rows] - want[rows])
        assert np.max(err) < ATT_TOL * scale, (b, n, np.max(err) / scale)


def test_attention_row_strides_bit_exact(ctx):
    """QKV rows wider than 3*d (a row stride of 3*d + 8) and a ctx stride of
    d + 4 give the same bits as the dense layout (head_dim 64 and 32)."""
    for hd in (64, 32):
        B, S, H = 2, 200, 3
        d = H * hd
        rng = np.random.default_rng(hd)
        qkv = to_bf16_bits(rng.standard_normal((B * S, 3 * d)).astype(np.float32))
        wide = np.zeros((B * S, 3 * d + 8), np.uint16)
        wide[:, :3 * d] = qkv
        lens = np.array([200, 61], np.int32)
        dk = ctx.put(lens)
        out = ctx.empty((B * S, d), np.uint16)
        mxenc.attention(ctx, ctx.put(qkv), 3 * d, B, S, H, hd, 0.125, None, dk, out, d)
        out2 = ctx.empty((B * S, d + 4), np.uint16)
        mxenc.attention(ctx, ctx.put(wide), 3 * d + 8, B, S, H, hd, 0.125, None, dk, out2, d + 4)
        assert np.array_equal(out.host(), out2.host()[:, :d])


def test_attention_fully_masked_row_is_uniform(ctx):
    """All keys masked with -1e30: the host softmax gives every key the same
    weight; so does the kernel (kv_len = S, finite mask)."""
    B, S, H, hd = 1, 64, 1, 64
    rng = np.random.default_rng(5)
    qkv = to_bf16_bits(rng.standard_normal((S, 3 * hd)).astype(np.float32))
    mask = np.full((B, S), -1e30, np.float32)
    dq, dm = ctx.put(qkv), ctx.put(mask)
    out = ctx.empty((S, hd), np.uint16)
    mxenc.attention(ctx, dq, 3 * hd, B, S, H, hd, 1.0, dm, None, out, hd)
    v = from_bf16_bits(qkv)[:, 2 * hd:]
    want = np.repeat(v.mean(0, keepdims=True), S, axis=0)
    assert np.max(np.abs(from_bf16_bits(out.host()) - want)) < ATT_TOL * np.max(np.abs(want))


# ---- embedding sum, mask, pooling ------------------------------------------------

def test_embed_sum_mask_kvlen_bit_exact(ctx, orc, golden_dir):
    z = np.load(golden_dir / "minilm_s64_pool.npz")
    ids = np.ascontiguousarray(z["input_ids"])
    am = np.ascontiguousarray(z["attention_mask"])
    B, S = ids.shape
    d = 384
    rng = np.random.default_rng(13)
    word = (rng.standard_normal((30522, d)) * 0.02).astype(np.float32)
    pos = (rng.standard_normal((512, d)) * 0.02).astype(np.float32)
    typ = (rng.standard_normal((2, d)) * 0.02).astype(np.float32)
    want = np.empty((B * S, d), np.float32)
    wmask = np.empty((B, S), np.float32)
    orc.orc_embed_sum(P(ids), P(am), B, S, d, P(word), P(pos), P(typ), P(want), P(wmask))
    L = mxenc.lib()
    d_ids, d_am, d_w, d_p, d_t = ctx.put(ids), ctx.put(am), ctx.put(word), ctx.put(pos), ctx.put(typ)
    emb = ctx.empty((B * S, d), np.float32)
    msk = ctx.empty((B, S), np.float32)
    kvl = ctx.empty((B,), np.int32)
    mxenc.check(L.mx_embed_sum(ctx.stream, d_ids.p, d_am.p, B, S, d, d_w.p, 30522, d_p.p, d_t.p,
                               emb.p, msk.p, kvl.p))
    assert np.array_equal(emb.host(), want)
    assert np.array_equal(msk.host(), wmask)
    assert np.array_equal(kvl.host(), am.sum(1).astype(np.int32))  # prefix masks: 8,22,17,33
    bad = ids.copy()
    bad[1, 3] = 30522
    d_bad = ctx.put(bad)
    with pytest.raises(mxenc.MxError, match="outside"):
        mxenc.check(L.mx_embed_sum(ctx.stream, d_bad.p, d_am.p, B, S, d, d_w.p, 30522, d_p.p,
                                   d_t.p, emb.p, None, None))


@pytest.mark.parametrize("B,S,d", [(5, 77, 1100), (3, 130, 100), (64, 512, 768)])
def test_pool_rows_mean_bit_exact_random(ctx, orc, B, S, d):
    """Mean pooling in double, in row order, over values spread across 2^-20 ..
    2^20 (so a reordered sum would differ), a weighted mask with holes, a
    sequence with no kept row (denominator 1e-9), S and d not multiples of the
    kernel's read-ahead, and d beyond one column per thread."""
    rng = np.random.default_rng(S)
    h = (rng.standard_normal((B, S, d)) *
         np.exp2(rng.integers(-20, 20, (B, S, d)))).astype(np.float32)
    am = ((rng.random((B, S)) < 0.7) *
          rng.choice([1.0, 0.5, 3.0], (B, S))).astype(np.float32)
    am[0] = 0
    L = mxenc.lib()
    dh, dam = ctx.put(h), ctx.put(am)
    out = ctx.empty((B, d), np.float32)
    for l2 in (0, 1):
        want = np.empty((B, d), np.float32)
        assert orc.orc_pool_rows(P(h), P(am), B, S, d, 0, l2, P(want)) == 0
        mxenc.check(L.mx_pool_rows(ctx.stream, dh.p, dam.p, B, S, d, 0, l2, out.p))
        assert np.array_equal(out.host().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("cls", [0, 1])
def test_pool_rows_bit_exact_on_reference_goldens(ctx, orc, golden_dir, cls):
    if cls:
        z = np.load(golden_dir / "bge_base_s64_cls.npz")
        head = z["last_hidden_state_head"]
        B, _, d = head.shape
        S = z["attention_mask"].shape[1]
        h = np.full((B, S, d), np.nan, np.float32)
        h[:, :4] = head
    else:
        z = np.load(golden_dir / "minilm_s64_pool.npz")
        h = np.ascontiguousarray(z["last_hidden_state"])
        B, S, d = h.shape
    am = np.ascontiguousarray(z["attention_mask"])
    L = mxenc.lib()
    dh, dam = ctx.put(h), ctx.put(am)
    out = ctx.empty((B, d), np.float32)
    for l2 in (0, 1):
        want = np.empty((B, d), np.float32)
        assert orc.orc_pool_rows(P(h), P(am), B, S, d, cls, l2, P(want)) == 0
        mxenc.check(L.mx_pool_rows(ctx.stream, dh.p, dam.p, B, S, d, cls, l2, out.p))
        assert np.array_equal(out.host().view(np.uint32), want.view(np.uint32))
    # and against the reference's own golden embedding
    assert np.max(np.abs(out.host() - z["embedding"])) < 1e-7
    if cls:
        am2 = am.copy()
        am2[1, 0] = 0
        dam2 = ctx.put(am2)
        with pytest.raises(mxenc.MxError, match="first token is masked"):
            mxenc.check(L.mx_pool_rows(ctx.stream, dh.p, dam2.p, B, S, d, 1, 1, out.p))
