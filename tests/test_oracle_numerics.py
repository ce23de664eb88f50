"""The oracle's per-op restatements, pinned against the reference's own compiled
host kernels (oracle/_ref), the reference's golden files (tests/golden) and
closed forms. CPU only."""
import ctypes
import math

import numpy as np
import pytest

from orc import P, bf16_round


def test_to_bf16_known_answers(orc):
    cases = {
        0x3F808000: 0x3F80,  # tie, even mantissa stays
        0x3F818000: 0x3F82,  # tie, odd mantissa rounds up
        0x3F807FFF: 0x3F80,
        0x3F808001: 0x3F81,
        0x7F800001: 0x7F80,  # the formula turns this NaN into +Inf
        0xFFFFFFFF: 0x0000,  # ... and this NaN into +0.0
        0x7FFFFFFF: 0x8000,
        0x7F7FFFFF: 0x7F80,  # FLT_MAX rounds to +Inf
        0x00000000: 0x0000,
        0x80000000: 0x8000,
    }
    bits = np.array(list(cases), np.uint32)  # bit patterns, so NaNs keep their payload
    got = np.empty(bits.size, np.uint16)
    orc.orc_bf16_fill(P(got), P(bits), bits.size)
    for b, g in zip(bits, got):
        assert g == cases[int(b)], hex(int(b))


def test_to_bf16_exhaustive_vs_reference(orc, ref):
    """Every one of the 2^32 fp32 bit patterns, against the reference's own
    AVX2 bf16_fill (host_kernels.hpp:179-199)."""
    chunk = 1 << 24
    want = np.empty(chunk, np.uint16)
    got = np.empty(chunk, np.uint16)
    for c in range(1 << 8):
        lo = c * chunk
        bits = np.arange(lo, lo + chunk, dtype=np.uint64).astype(np.uint32)
        ref.ref_bf16_fill_bits(lo, chunk, P(want))
        orc.orc_bf16_fill(P(got), P(bits), chunk)
        if not np.array_equal(got, want):
            bad = np.nonzero(got != want)[0][0]
            raise AssertionError(f"bits {lo + bad:#x}: {got[bad]:#x} != {want[bad]:#x}")


def _specials():
    return np.array([0.0, -0.0, 1.0, -1.0, 3.999, 4.0, 4.001, -4.0, 1e-30, -1e-30, 80.0,
                     -80.0, 1e30, -1e30, np.inf, -np.inf], np.float32)


def test_gelu8_vs_reference(orc, ref):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(1 << 16).astype(np.float32) * 3, _specials()])
    y_avx = np.empty_like(x)
    ref.ref_gelu8_avx2(P(x), P(y_avx), x.size)
    y = np.array([orc.orc_gelu8(float(v)) for v in x], np.float32)
    # the AVX2 branch is the one gelu_cpu runs on all but the last n % 8
    assert np.array_equal(y.view(np.uint32)[: x.size // 8 * 8],
                          y_avx.view(np.uint32)[: x.size // 8 * 8])
    ys = np.array([ref.ref_gelu8_scalar(float(v)) for v in x[:4096]], np.float32)
    assert np.array_equal(y[:4096].view(np.uint32), ys.view(np.uint32))


def test_gelu8_is_gelu(orc):
    """The degree-8 fit approximates 0.5x(1+erf(x/sqrt2)); a wrong coefficient
    or sign shows up far above the fit's error."""
    x = np.linspace(-8, 8, 20001, dtype=np.float32)
    y = np.array([orc.orc_gelu8(float(v)) for v in x], np.float64)
    exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    assert np.max(np.abs(y - exact)) < 2e-4


def test_gelu_erf_exact(orc):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(4096) * 4).astype(np.float32)
    y = x.copy()
    orc.orc_gelu_erf_inplace(P(y), y.size)
    exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    assert np.array_equal(y, exact.astype(np.float32))


def test_exp2_poly_vs_reference(orc, ref):
    x = np.concatenate([np.linspace(-120, 0, 100003, dtype=np.float32),
                        np.linspace(-3, 3, 1001, dtype=np.float32)])
    a = np.empty_like(x)
    b = np.empty_like(x)
    orc.orc_exp2_poly(P(x), P(a), x.size)
    ref.ref_exp2_avx2(P(x), P(b), x.size)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    exact = np.exp2(x.astype(np.float64))
    assert np.max(np.abs(a / exact - 1)) < 5e-7


def test_gemm_nt_vs_reference(orc, ref):
    rng = np.random.default_rng(3)
    for (M, K, N) in [(1, 8, 8), (17, 40, 24), (64, 96, 136), (9, 384, 33)]:
        A = rng.standard_normal((M, K)).astype(np.float32)
        B = bf16_round(rng.standard_normal((K, N)).astype(np.float32))
        bias = rng.standard_normal(N).astype(np.float32)
        c1 = np.empty((M, N), np.float32)
        c2 = np.empty((M, N), np.float32)
        orc.orc_gemm_nt(P(A), M, P(B), K, N, P(bias), P(c1))
        ref.ref_gemm_nt(P(A), M, P(B), K, N, P(bias), P(c2), 3)
        assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32)), (M, K, N)
        exact = A.astype(np.float64) @ B.astype(np.float64) + bias
        assert np.max(np.abs(c1 - exact)) / np.max(np.abs(exact)) < 1e-5


def _ln64(x, g, b, eps):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


@pytest.mark.parametrize("cols", [384, 768, 1024, 1280])
def test_layer_norm_rows(orc, cols):
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((37, cols)) * 3 + 0.5).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cols)).astype(np.float32)
    want = _ln64(x, g, b, 1e-12)
    y = x.copy()
    orc.orc_layer_norm_rows(P(y), 37, cols, P(g), P(b), 1e-12)
    assert np.max(np.abs(y - want)) < 2e-5
    y = x.copy()
    orc.orc_layernorm_rows_f64(P(y), 37, cols, P(g), P(b), 1e-5)
    assert np.max(np.abs(y - _ln64(x, g, b, 1e-5))) < 2e-5


def _softmax64(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def test_softmax_poly_and_mask_rows(orc):
    """softmax_cpu with the additive mask: mask row b applies to the H*S score
    rows of sequence b and to nothing else."""
    rng = np.random.default_rng(5)
    B, H, S = 3, 2, 16
    x = (rng.standard_normal((B * H * S, S)) * 4).astype(np.float32)
    mask = np.zeros((B, S), np.float32)
    mask[1, 5:] = -1e30
    mask[2, 11:] = -1e30
    y = x.copy()
    orc.orc_softmax_rows_poly(P(y), B * H * S, S, P(mask), H * S)
    want = _softmax64(x + np.repeat(mask, H * S, axis=0))
    assert np.max(np.abs(y - want)) < 1e-6
    r1 = y[H * S: 2 * H * S]
    assert np.all(r1[:, 5:] < 1e-30) and np.all(y[: H * S] > 0)
    y = x.copy()
    orc.orc_softmax_rows_exact(P(y), B * H * S, S, P(mask), H * S)
    assert np.max(np.abs(y - want)) < 1e-6


def _attn64(q, k, v, mask=None, scale=1.0):
    s = q @ k.T * scale
    if mask is not None:
        s = s + mask
    return _softmax64(s) @ v


def test_qk_av_brute_force(orc):
    rng = np.random.default_rng(6)
    for hd in (32, 64):
        B, S, H = 2, 24, 3
        d = H * hd
        qkv = rng.standard_normal((B * S, 3 * d)).astype(np.float32)
        mask = np.zeros((B, S), np.float32)
        mask[1, 17:] = -1e30
        sc = np.empty((B * H * S, S), np.float32)
        ctx = np.empty((B * S, d), np.float32)
        orc.orc_qk(P(qkv), B, S, H, hd, P(sc))
        orc.orc_softmax_rows_poly(P(sc), B * H * S, S, P(mask), H * S)
        orc.orc_av(P(sc), P(qkv), B, S, H, hd, P(ctx))
        q64 = qkv.astype(np.float64)
        for b in range(B):
            for h in range(H):
                rows = slice(b * S, (b + 1) * S)
                q = q64[rows, h * hd:(h + 1) * hd]
                k = q64[rows, d + h * hd: d + (h + 1) * hd]
                v = q64[rows, 2 * d + h * hd: 2 * d + (h + 1) * hd]
                want = _attn64(q, k, v, mask[b])
                got = ctx[rows, h * hd:(h + 1) * hd]
                assert np.max(np.abs(got - want)) < 2e-5, (hd, b, h)


def test_whisper_attention_brute_force(orc):
    rng = np.random.default_rng(7)
    n, H, hd = 21, 3, 64
    d = H * hd
    qkv = rng.standard_normal((n, 3 * d)).astype(np.float32)
    out = np.empty((n, d), np.float32)
    # K|V block starts d floats into each fused row
    orc.orc_whisper_attention(P(qkv), 3 * d, ctypes.c_void_p(qkv.ctypes.data + d * 4), 3 * d,
                              n, n, d, H, hd, 0.125, P(out))
    q64 = qkv.astype(np.float64)
    for h in range(H):
        q = q64[:, h * hd:(h + 1) * hd]
        k = q64[:, d + h * hd: d + (h + 1) * hd]
        v = q64[:, 2 * d + h * hd: 2 * d + (h + 1) * hd]
        assert np.max(np.abs(out[:, h * hd:(h + 1) * hd] - _attn64(q, k, v, None, 0.125))) < 2e-5


def test_pool_mean_vs_reference_golden(orc, golden_dir):
    z = np.load(golden_dir / "minilm_s64_pool.npz")
    h = np.ascontiguousarray(z["last_hidden_state"])
    m = np.ascontiguousarray(z["attention_mask"])
    B, S, d = h.shape
    out = np.empty((B, d), np.float32)
    assert orc.orc_pool_rows(P(h), P(m), B, S, d, 0, 0, P(out)) == 0
    assert np.max(np.abs(out - z["pool_mean"])) < 2e-7
    assert orc.orc_pool_rows(P(h), P(m), B, S, d, 0, 1, P(out)) == 0
    assert np.max(np.abs(out - z["embedding"])) < 1e-7


def test_pool_cls_vs_reference_golden(orc, golden_dir):
    z = np.load(golden_dir / "bge_base_s64_cls.npz")
    head = z["last_hidden_state_head"]
    B, _, d = head.shape
    S = z["attention_mask"].shape[1]
    h = np.full((B, S, d), np.nan, np.float32)  # CLS pooling must read row 0 only
    h[:, :4] = head
    m = np.ascontiguousarray(z["attention_mask"])
    out = np.empty((B, d), np.float32)
    assert orc.orc_pool_rows(P(h), P(m), B, S, d, 1, 1, P(out)) == 0
    assert np.max(np.abs(out - z["embedding"])) < 1e-7
    assert np.max(np.abs(out - z["st_embedding"])) < 5e-7
    m2 = m.copy()
    m2[2, 0] = 0
    assert orc.orc_pool_rows(P(h), P(m2), B, S, d, 1, 1, P(out)) == -1


def test_embed_sum_indexing(orc, golden_dir):
    """emb = word[id] + pos[s] + type[0]; cmask 0 / -1e30 -- on the
    reference's own input_ids/attention_mask."""
    z = np.load(golden_dir / "minilm_s64_pool.npz")
    ids = np.ascontiguousarray(z["input_ids"])
    m = np.ascontiguousarray(z["attention_mask"])
    B, S = ids.shape
    d = 16
    word = (np.arange(30522 * d, dtype=np.float32).reshape(30522, d) * 1e-3)
    pos = np.arange(S * d, dtype=np.float32).reshape(S, d) * 1e-1
    typ = np.arange(2 * d, dtype=np.float32).reshape(2, d) + 7
    emb = np.empty((B * S, d), np.float32)
    cm = np.empty((B, S), np.float32)
    orc.orc_embed_sum(P(ids), P(m), B, S, d, P(word), P(pos), P(typ), P(emb), P(cm))
    want = (word[ids.reshape(-1)] + np.tile(pos, (B, 1))) + typ[0]
    assert np.array_equal(emb, want.astype(np.float32))
    assert np.array_equal(cm, np.where(m > 0, 0.0, -1e30).astype(np.float32))


def test_aie_softmax_bf16(orc):
    rng = np.random.default_rng(8)
    rows, cols = 64, 64
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    x[3, 40:] = -1e30  # masked tail, as a padded score row carries
    xb = np.empty(x.shape, np.uint16)
    orc.orc_bf16_fill(P(xb), P(x), x.size)
    out = np.empty_like(xb)
    orc.orc_aie_softmax_bf16(P(xb), P(out), rows, cols)
    got = (out.astype(np.uint32) << 16).view(np.float32)
    want = _softmax64((xb.astype(np.uint32) << 16).view(np.float32))
    assert np.max(np.abs(got - want)) < 4e-3
    assert np.all(got[3, 40:] < 1e-30)


def test_aie_layernorm_bf16(orc):
    rng = np.random.default_rng(9)
    rows, cols = 16, 384
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cols)).astype(np.float32)
    xb = np.empty(x.shape, np.uint16)
    orc.orc_bf16_fill(P(xb), P(x), x.size)
    out = np.empty_like(xb)
    orc.orc_aie_layernorm_bf16(P(xb), P(out), rows, cols, P(g), P(b), 1e-12)
    got = (out.astype(np.uint32) << 16).view(np.float32)
    want = _ln64((xb.astype(np.uint32) << 16).view(np.float32), g, b, 1e-12)
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-2)) < 1e-2


def test_aie_gelu_bf16(orc):
    x = np.linspace(-10, 10, 4096, dtype=np.float32)
    xb = np.empty(x.shape, np.uint16)
    orc.orc_bf16_fill(P(xb), P(x), x.size)
    xw = (xb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xw])
    for fn in (orc.orc_aie_gelu_erf_bf16, orc.orc_aie_gelu_poly_bf16):
        out = np.empty_like(xb)
        fn(P(xb), P(out), x.size)
        got = (out.astype(np.uint32) << 16).view(np.float32)
        assert np.max(np.abs(got - exact) / (np.abs(exact) + 1e-2)) < 1.2e-2


def _i32_bf16_exact(v):
    """Nearest-even bf16 of an integer, by exact rational rounding."""
    if v == 0:
        return 0
    s = 0x8000 if v < 0 else 0
    a = abs(v)
    e = a.bit_length() - 1
    if e <= 7:
        mant = a << (7 - e)
    else:
        sh = e - 7
        mant, rem = a >> sh, a & ((1 << sh) - 1)
        half = 1 << (sh - 1)
        if rem > half or (rem == half and mant & 1):
            mant += 1
        if mant == 256:
            mant, e = 128, e + 1
    return s | ((e + 127) << 7) | (mant & 0x7F)


def test_narrow_i32_single_rounding(orc):
    rng = np.random.default_rng(10)
    v = np.concatenate([
        rng.integers(-2**31, 2**31, 20000, dtype=np.int64),
        rng.integers(-70000, 70000, 20000),
        np.array([0, 1, -1, 127, 128, 255, 256, 257, 383, 384, 385, 2**24, 2**24 + 1,
                  2**24 + 2**16 + 2**15, 2**31 - 1, -2**31, 0x7FFF8000, -0x7FFF8000]),
    ]).astype(np.int32)
    out = np.empty(v.shape, np.uint16)
    orc.orc_narrow_i32_bf16(P(v), P(out), v.size)
    want = np.array([_i32_bf16_exact(int(a)) for a in v], np.uint16)
    assert np.array_equal(out, want)
    tw = np.empty_like(out)
    orc.orc_narrow_i32_bf16_twice(P(v), P(tw), v.size)
    small = np.abs(v.astype(np.int64)) <= 2**24
    assert np.array_equal(tw[small], out[small])
    # double rounding differs somewhere above 2^24 (e.g. 2^24 + 2^16 + 2^15 + 1)
    w = np.array([2**24 + 2**16 + 2**15 + 1, 0x01018001], np.int32)
    a, b = np.empty(2, np.uint16), np.empty(2, np.uint16)
    orc.orc_narrow_i32_bf16(P(w), P(a), 2)
    orc.orc_narrow_i32_bf16_twice(P(w), P(b), 2)
    assert np.array_equal(a, np.array([_i32_bf16_exact(int(x)) for x in w], np.uint16))


def test_narrow_f32_is_to_bf16(orc):
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2**32, 100000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    out = np.empty(x.shape, np.uint16)
    orc.orc_narrow_f32_bf16(P(x), P(out), x.size)
    want = ((bits.astype(np.uint64) + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(out, want)


# ---- pins of the accelerator-kernel restatements that catch seeded mistakes --
#
# Each pin compares a restatement's bf16 output with an fp64 evaluation of the
# reference kernel's stated arithmetic (exact mean, variance, 1/sqrt, exp2 and
# erf; the kernel's bf16 narrowing points kept), element by element, to half a
# bf16 ulp plus the fp32 evaluation error. The inputs are built so that each
# plausible mistake moves many results past that bound: rounding toward -inf
# instead of to nearest even (the accelerator's default mode; the _rne kernels
# set conv_even), one Newton step of fast_invsqrt instead of two, exponentials
# summed or stored without their bf16 narrowing. test_aie_pins_catch_each_
# seeded_mistake plants each mistake in a copy of the oracle and checks that
# its pin fails.

ROOT = __import__("os").path.dirname(__import__("os").path.dirname(
    __import__("os").path.abspath(__file__)))


def _as_f64(u16):
    return (np.asarray(u16, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _to_bf16_rne(v):
    """fp64 -> nearest-even bf16 bits, through the exact fp32 value when v is
    one (the models below form fp32-exact or fp64 values)."""
    f = np.asarray(v, np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def _bf16_ulp(v):
    a = np.maximum(np.abs(np.asarray(v, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def _aie_sigs(lib):
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.orc_aie_layernorm_bf16.argtypes = [vp, vp, i64, i64, vp, vp, ctypes.c_float]
    lib.orc_aie_layernorm_bf16.restype = None
    lib.orc_aie_softmax_bf16.argtypes = [vp, vp, i64, i64]
    lib.orc_aie_softmax_bf16.restype = None
    for n in ("orc_aie_gelu_erf_bf16", "orc_aie_gelu_poly_bf16"):
        getattr(lib, n).argtypes = [vp, vp, i64]
        getattr(lib, n).restype = None
    return lib


def _ln_pin_inputs():
    """96 rows of 768: row scales log-uniform over 1e-2 .. 1e2 (so var + eps
    runs through every mantissa, where fast_invsqrt's one-step error spans 0 ..
    1.75e-3), an offset of half a scale, random gamma and beta."""
    rng = np.random.default_rng(31)
    rows, cols = 96, 768
    sc = np.exp(rng.uniform(np.log(1e-2), np.log(1e2), rows))
    x = (rng.standard_normal((rows, cols)) + 0.5 * rng.standard_normal((rows, 1))) * sc[:, None]
    g = (1 + 0.25 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.25 * rng.standard_normal(cols)).astype(np.float32)
    return _to_bf16_rne(x), g, b


def pin_aie_layernorm(lib):
    """Fraction of layernorm_rne's outputs off the fp64 model by more than
    half a bf16 ulp plus the fp32 error (2e-5 of the normalised value: the
    16-way sums, two-step fast_invsqrt ~5e-6, three roundings)."""
    xb, g, b = _ln_pin_inputs()
    rows, cols = xb.shape
    out = np.empty_like(xb)
    eps = 1e-12
    lib.orc_aie_layernorm_bf16(P(xb), P(out), rows, cols, P(g), P(b), eps)
    x = _as_f64(xb)
    d = x - x.mean(1, keepdims=True)
    nrm = d / np.sqrt((d * d).mean(1, keepdims=True) + eps) * g
    y = nrm + b
    err = np.abs(_as_f64(out) - y)
    return float(np.mean(err > 0.5 * _bf16_ulp(y) + 2e-5 * np.abs(nrm) + 1e-7 * np.abs(b)))


def _sm_pin_inputs():
    """32 rows of 16 (a 0 and 15 values in [-1, -1/64) whose exp2(d * log2e)
    sits 0.30 .. 0.45 ulp above a bf16 grid point, so narrowing each
    exponential lowers it by that much and the narrowed sum is ~0.25 % under
    the unnarrowed one), then 16 rows of 64 normal values with a masked tail."""
    rng = np.random.default_rng(32)
    cand = -_as_f64(np.arange(0x3C80, 0x3F80, dtype=np.uint16))  # bf16 grid in (-1, -1/64]
    a = (cand.astype(np.float32) * np.float32(1.4426950408889634)).astype(np.float64)
    e = 2.0 ** a
    frac = e / _bf16_ulp(e) % 1.0
    pool = cand[(frac > 0.30) & (frac < 0.45)]
    assert pool.size > 40
    crafted = np.concatenate([np.zeros((32, 1)), rng.choice(pool, (32, 15))], 1)
    normal = rng.standard_normal((16, 64)) * 3
    normal[3, 40:] = -1e30
    return _to_bf16_rne(crafted), _to_bf16_rne(normal)


def _sm_model(xb):
    """softmax.cc:76-160 in fp64 with its bf16 narrowing points: inputs
    clamped at bf16(-1e30), the row max, d clamped at -100, a = d * log2e in
    fp32 clamped at -120, e = bf16(2^a), o = bf16(e / sum e)."""
    x = np.maximum(_as_f64(xb), _as_f64(_to_bf16_rne(-1e30)))
    m = np.maximum(x.max(1, keepdims=True), -1e30)
    d = np.maximum(x - m, -100.0).astype(np.float32)
    a = np.maximum((d * np.float32(1.4426950408889634)).astype(np.float64), -120.0)
    e = _as_f64(_to_bf16_rne(2.0 ** a))
    return e / e.sum(1, keepdims=True)


def pin_aie_softmax(lib):
    """Fraction of softmax_rne's outputs off the model by more than half a
    bf16 ulp plus 4e-6 relative (the fp32 sum and reciprocal)."""
    worst = 0.0
    for xb in _sm_pin_inputs():
        out = np.empty_like(xb)
        lib.orc_aie_softmax_bf16(P(xb), P(out), xb.shape[0], xb.shape[1])
        o = _sm_model(xb)
        err = np.abs(_as_f64(out) - o)
        live = o > 1e-30
        bad = err[live] > 0.5 * _bf16_ulp(o[live]) + 4e-6 * o[live]
        worst = max(worst, float(np.mean(bad)))
    return worst


def pin_aie_gelu(lib):
    """Fractions of gelu_erf's and gelu_poly's outputs off their fp64 models
    by more than half a bf16 ulp plus the evaluation error, over every bf16
    value with 1/16 <= |x| <= 6 (below that GELU is x/2 plus a term under the
    rounding, which no rounding mode changes): gelu_erf against the exact GELU
    (A&S 7.1.26 is within
    1.5e-7 of erf: 1e-6 |x| covers it); gelu_poly against its own degree-8
    polynomial evaluated in fp64 (the polynomial's fit to GELU is pinned by
    test_aie_gelu_bf16; this pins the narrowing)."""
    import scipy.special
    allb = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    finite = ((allb >> 7) & 0xFF) != 0xFF
    v = _as_f64(np.where(finite, allb, 0).astype(np.uint16))
    xb = np.ascontiguousarray(allb[finite & (np.abs(v) <= 6.0) & (np.abs(v) >= 1.0 / 16)])
    x = _as_f64(xb)
    fr = []
    out = np.empty_like(xb)
    lib.orc_aie_gelu_erf_bf16(P(xb), P(out), xb.size)
    y = 0.5 * x * (1.0 + scipy.special.erf(x / np.sqrt(2.0)))
    fr.append(np.mean(np.abs(_as_f64(out) - y) > 0.5 * _bf16_ulp(y) + 1e-6 * np.abs(x)))
    lib.orc_aie_gelu_poly_bf16(P(xb), P(out), xb.size)
    u = np.minimum(np.abs(x), 4.0)
    c = [-7.2340282171e-05, 1.8179518005e-03, -1.7707383379e-02, 8.4577147641e-02,
         -1.9228671834e-01, 9.8431124458e-02, 3.6137852062e-01, -4.9454128936e-01,
         -1.3007010117e-04]
    p = np.zeros_like(u)
    for k in c:
        p = p * u + np.float64(np.float32(k))
    y = np.maximum(x, 0.0) + p
    fr.append(np.mean(np.abs(_as_f64(out) - y) > 0.5 * _bf16_ulp(y) + 1e-6 * (np.abs(x) + 1)))
    return float(max(fr))


def test_aie_layernorm_pinned(orc):
    assert pin_aie_layernorm(orc) == 0.0


def test_aie_softmax_pinned(orc):
    assert pin_aie_softmax(orc) == 0.0


def test_aie_gelu_pinned(orc):
    assert pin_aie_gelu(orc) == 0.0


_FLOOR = ("{ uint32_t u_; memcpy(&u_, &{v}, 4); uint32_t t_ = u_ >> 16; "
          "if ((u_ & 0xFFFFu) && (u_ >> 31)) t_ += 1; {dst} = (uint16_t)t_; }")

# (pin, [(text in oracle/orc_numerics.c, replacement, count)])
SEEDED = {
    "layernorm rounds toward -inf": (pin_aie_layernorm, [
        ("      o[j] = orc_to_bf16(y);\n",
         "      " + _FLOOR.replace("{v}", "y").replace("{dst}", "o[j]") + "\n", 1)]),
    "fast_invsqrt with one Newton step": (pin_aie_layernorm, [
        ("  y = y * (1.5f - xhalf * y * y);\n  y = y * (1.5f - xhalf * y * y);\n",
         "  y = y * (1.5f - xhalf * y * y);\n", 1)]),
    "softmax rounds toward -inf": (pin_aie_softmax, [
        ("o[j] = orc_to_bf16(e[j] * inv);",
         "{ const float q_ = e[j] * inv; " +
         _FLOOR.replace("{v}", "q_").replace("{dst}", "o[j]") + " }", 1)]),
    "softmax exponentials not narrowed": (pin_aie_softmax, [
        ("e[j] = bf(aie_exp2(a));", "e[j] = aie_exp2(a);", 1)]),
    "softmax sum of unnarrowed exponentials": (pin_aie_softmax, [
        ("      e[j] = bf(aie_exp2(a));\n      acc[j % 16] += e[j];",
         "      e[j] = bf(aie_exp2(a));\n      acc[j % 16] += aie_exp2(a);", 1)]),
    "gelu_erf rounds toward -inf": (pin_aie_gelu, [
        ("    const float y = x * 0.5f + (fabsf(x) * 0.5f) * eabs;\n    out[i] = orc_to_bf16(y);",
         "    const float y = x * 0.5f + (fabsf(x) * 0.5f) * eabs;\n    " +
         _FLOOR.replace("{v}", "y").replace("{dst}", "out[i]"), 1)]),
    "gelu_poly rounds toward -inf": (pin_aie_gelu, [
        ("    out[i] = orc_to_bf16((x > 0.0f ? x : 0.0f) + p);",
         "    const float y_ = (x > 0.0f ? x : 0.0f) + p;\n    " +
         _FLOOR.replace("{v}", "y_").replace("{dst}", "out[i]"), 1)]),
}


@pytest.mark.parametrize("mistake", sorted(SEEDED))
def test_aie_pins_catch_each_seeded_mistake(mistake, tmp_path):
    """A copy of the oracle with one mistake planted (on the CPU) fails the
    pin of the function it changes."""
    import os
    import shutil
    import subprocess
    pin, edits = SEEDED[mistake]
    src = os.path.join(ROOT, "oracle")
    for f in os.listdir(src):
        if f.endswith((".c", ".h")):
            shutil.copy(os.path.join(src, f), tmp_path / f)
    path = tmp_path / "orc_numerics.c"
    text = path.read_text()
    for old, new, count in edits:
        assert text.count(old) == count, (mistake, old)
        text = text.replace(old, new)
    path.write_text(text)
    so = tmp_path / "liborc_seeded.so"
    srcs = [str(tmp_path / f) for f in ("orc_pool.c", "orc_numerics.c", "orc_ops.c",
                                        "orc_encoders.c")]
    r = subprocess.run(["gcc", "-std=gnu11", "-O2", "-march=x86-64-v3", "-ffp-contract=off",
                        "-fPIC", "-shared", "-o", str(so)] + srcs + ["-lm", "-lpthread"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    lib = _aie_sigs(ctypes.CDLL(str(so)))
    assert pin(lib) > 0.01, mistake
