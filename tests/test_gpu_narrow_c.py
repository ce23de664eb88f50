"""GPU parity of the narrowed C (MX_EPI_NARROW_C, mx_encoder_set_narrowed_c):
the array designs that round C to bf16 on the core (c_elem_bytes == 2, the
export default) and finish from that bf16 value on the host. Per op, bit for
bit against the oracle's restatements of BertEncoder::gemm's bf16-C branch,
dequant_act_bf16 and dequantise_c's 2-byte branch (each pinned against the
reference's own code in test_oracle_narrow_c.py), applied to the GPU's own
accumulator (read back through the plain epilogue, which adds nothing);
end to end against the oracle's stack in the same array arithmetic."""
import numpy as np
import pytest

import mxenc
from mxenc import synth
from orc import P, encoder_struct, OrcI8, array_arith, ORC_ARR_A_BF16, ORC_ARR_C_BF16, \
    ORC_ARR_ATTN_BF16

pytestmark = pytest.mark.gpu

NC = mxenc.MX_EPI_NARROW_C


@pytest.fixture(scope="module")
def ctx():
    c = mxenc.Context(0)
    yield c
    c.close()


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint32 if x.dtype == np.float32 else np.uint16)


def _gemm(ctx, A_bits, Wt_bits, bias, epi, c_dtype):
    M, K = A_bits.shape
    N = Wt_bits.shape[0]
    C = ctx.empty((M, N), np.float32 if c_dtype == mxenc.MX_F32 else np.uint16)
    mxenc.gemm_wt(ctx, ctx.put(A_bits), M, K, K, ctx.put(Wt_bits), N, ctx.put(bias), epi, None,
                  C, N)
    return C.host()


# (M, K, N): the 256 x 256 tile and the 128 x 128 tile of the narrowed-C launch,
# with rows and columns past the last whole tile
SHAPES = [(4100, 768, 2304), (300, 384, 1536), (1000, 1024, 1032)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemm_narrowed_c_bit_exact(ctx, orc, M, K, N):
    rng = np.random.default_rng(M + K + N)
    A = mxenc.to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    Wt = mxenc.to_bf16_bits((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    bias = rng.standard_normal(N).astype(np.float32)
    # the GPU's own fp32 accumulator: the plain epilogue over a zero bias
    acc = _gemm(ctx, A, Wt, np.zeros(N, np.float32), mxenc.MX_EPI_NONE, mxenc.MX_F32)
    c16 = mxenc.to_bf16_bits(acc)  # the core's narrowing (RNE)
    # fp32 C: from_bf16(c) + bias (bert_encoder.cpp:874-900)
    want = np.empty((M, N), np.float32)
    orc.orc_bias_c_bf16(P(c16), M, N, P(bias), P(want))
    got = _gemm(ctx, A, Wt, bias, NC | mxenc.MX_EPI_NONE, mxenc.MX_F32)
    assert np.array_equal(_bits(got), _bits(want))
    # the narrowing is there: the unnarrowed epilogue differs
    plain = _gemm(ctx, A, Wt, bias, mxenc.MX_EPI_NONE, mxenc.MX_F32)
    assert not np.array_equal(_bits(plain), _bits(want))
    # bf16 C: that value rounded once more (the next op's bf16 operand)
    got16 = _gemm(ctx, A, Wt, bias, NC | mxenc.MX_EPI_NONE, mxenc.MX_BF16)
    assert np.array_equal(got16, mxenc.to_bf16_bits(want))
    # bf16 C with gelu8: dequant_act_bf16 (bert_encoder.cpp:633-712)
    wact = np.empty((M, N), np.uint16)
    orc.orc_dequant_act_bf16(P(c16), M, N, 0, P(bias), P(wact))
    gact = _gemm(ctx, A, Wt, bias, NC | mxenc.MX_EPI_GELU_POLY, mxenc.MX_BF16)
    assert np.array_equal(gact, wact)


def test_gemm_narrowed_c_exact_erf_within_its_bound(ctx, orc):
    """The exact-erf GELU epilogue (A&S 7.1.26 form: within 2.3e-7 max(|x|,
    1e-3) of the double erf's GELU) after the narrowing: within that bound plus
    one bf16 rounding (half an ulp, 2^-9 relative) of the host's
    gelu_erf_exact on x = from_bf16(c) + bias, rounded to bf16."""
    rng = np.random.default_rng(9)
    M, K, N = 512, 768, 3072
    A = mxenc.to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    Wt = mxenc.to_bf16_bits((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    bias = rng.standard_normal(N).astype(np.float32)
    acc = _gemm(ctx, A, Wt, np.zeros(N, np.float32), mxenc.MX_EPI_NONE, mxenc.MX_F32)
    c16 = mxenc.to_bf16_bits(acc)  # kept alive across the call that reads it
    x = np.empty((M, N), np.float32)
    orc.orc_bias_c_bf16(P(c16), M, N, P(bias), P(x))
    v = x.copy()
    orc.orc_gelu_erf_inplace(P(v), v.size)
    got = mxenc.from_bf16_bits(
        _gemm(ctx, A, Wt, bias, NC | mxenc.MX_EPI_GELU_ERF, mxenc.MX_BF16))
    bound = 2.3e-7 * np.maximum(np.abs(x), 1e-3) + np.abs(v) * 2.0 ** -8
    assert np.all(np.abs(got.astype(np.float64) - v) <= bound)
    # and the narrowing happened first: the same epilogue on the unnarrowed
    # accumulator lands elsewhere
    plain = mxenc.from_bf16_bits(_gemm(ctx, A, Wt, bias, mxenc.MX_EPI_GELU_ERF, mxenc.MX_BF16))
    assert not np.array_equal(plain, got)


def _i8(rng, shape):
    return rng.integers(-127, 128, shape, dtype=np.int8)


@pytest.mark.parametrize("M,K,N", [(1000, 768, 2304), (4096, 3072, 768), (257, 512, 68)])
def test_gemm_i8_narrowed_c_bit_exact(ctx, orc, M, K, N):
    """int8: the exact int32 product rounded to bf16 once (narrow_i32_bf16),
    then dequantise_c's 2-byte branch; with gelu8 for FFN-up's fp32 value
    (dequant_act_quant's first half) and as a bf16 C."""
    rng = np.random.default_rng(M * 3 + N)
    A, W = _i8(rng, (M, K)), _i8(rng, (K, N))
    sa = rng.uniform(1e-4, 1e-1, M).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    slot = mxenc.stage_weight_i8(ctx, W, ws, np.ones(K, np.float32))
    dA, dsa, db = ctx.put(A), ctx.put(sa), ctx.put(b)
    raw = ctx.empty((M, N), np.int32)
    mxenc.gemm_i8(ctx, dA, None, M, K, K, slot, None, mxenc.MX_EPI_NONE, None, raw, N)
    c16 = np.empty((M, N), np.uint16)
    r = np.ascontiguousarray(raw.host())
    assert np.array_equal(r.astype(np.int64), A.astype(np.int64) @ W.astype(np.int64))
    orc.orc_narrow_i32_bf16(P(r), P(c16), M * N)
    want = np.empty((M, N), np.float32)
    orc.orc_dequantise_c_bf16(P(c16), M, N, P(sa), P(ws), P(b), P(want))
    C = ctx.empty((M, N), np.float32)
    mxenc.gemm_i8(ctx, dA, dsa, M, K, K, slot, db, NC | mxenc.MX_EPI_NONE, None, C, N)
    assert np.array_equal(_bits(C.host()), _bits(want))
    wg = want.copy()
    orc.orc_gelu_poly_inplace(P(wg), wg.size)
    mxenc.gemm_i8(ctx, dA, dsa, M, K, K, slot, db, NC | mxenc.MX_EPI_GELU_POLY, None, C, N)
    assert np.array_equal(_bits(C.host()), _bits(wg))
    if N % 8 == 0:  # a bf16 C keeps its rows 16-byte aligned
        C16 = ctx.empty((M, N), np.uint16)
        mxenc.gemm_i8(ctx, dA, dsa, M, K, K, slot, db, NC | mxenc.MX_EPI_NONE, None, C16, N)
        assert np.array_equal(C16.host(), mxenc.to_bf16_bits(want))
    mxenc.check(mxenc.lib().mx_release_weight(ctx.handle, slot))


def test_narrowed_c_refusals(ctx):
    L = mxenc.lib()
    M, K, N = 64, 256, 256
    A = ctx.put(np.zeros((M, K), np.uint16))
    Wt = ctx.put(np.zeros((N, K), np.uint16))
    bias = ctx.put(np.zeros(N, np.float32))
    C = ctx.empty((M, N), np.float32)

    def call(epi, resid=None, c_dtype=mxenc.MX_F32, k=K, lda=K):
        return L.mx_gemm_wt(ctx.stream, A.p, M, k, lda, Wt.p, N, bias.p, epi,
                            resid.p if resid else None, C.p, c_dtype, N)

    assert call(NC | mxenc.MX_EPI_NONE, resid=C) == mxenc.MX_E_UNSUPPORTED
    assert "residual" in L.mx_last_error().decode()
    assert call(NC | mxenc.MX_EPI_GELU_POLY) == mxenc.MX_E_UNSUPPORTED  # fp32 C, activation
    # K % 32 != 0: the register-staged kernel, which has no narrowed C
    assert call(NC | mxenc.MX_EPI_NONE, k=72, lda=K) == mxenc.MX_E_UNSUPPORTED
    assert "direct-to-LDS" in L.mx_last_error().decode()
    assert call(64 | mxenc.MX_EPI_NONE) == mxenc.MX_E_INVALID  # an unknown flag
    assert call(NC | mxenc.MX_EPI_NONE) == mxenc.MX_OK
    ctx.sync()
    # int8: not the raw product, no residual
    Wq = np.zeros((K, N), np.int8)
    slot = mxenc.stage_weight_i8(ctx, Wq, np.ones(N, np.float32), np.ones(K, np.float32))
    Aq = ctx.put(np.zeros((M, K), np.int8))
    raw = ctx.empty((M, N), np.int32)
    assert L.mx_gemm_i8(ctx.stream, Aq.p, None, M, K, K, slot, None, NC, None, raw.p,
                        mxenc.MX_I32, N) == mxenc.MX_E_UNSUPPORTED
    mxenc.check(L.mx_release_weight(ctx.handle, slot))
    # the encoder switch: BERT stacks only
    vm = synth.make_model("vit_base", layers=1)
    venc = mxenc.Encoder(ctx, vm)
    assert L.mx_encoder_set_narrowed_c(venc.handle, 1) == mxenc.MX_E_UNSUPPORTED
    assert L.mx_encoder_set_narrowed_c(venc.handle, 0) == mxenc.MX_OK
    venc.close()


# ---- the encoder stack ---------------------------------------------------------

def _cos(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return np.sum(a * b, -1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1))


def _oracle(orc, m, ids, am, flags, q8=None):
    B, S = ids.shape
    d = m["hidden"]
    emb = np.empty((B * S, d), np.float32)
    cm = np.empty((B, S), np.float32)
    orc.orc_embed_sum(P(ids), P(am), B, S, d, P(m["word"]), P(m["pos"]), P(m["type"]), P(emb),
                      P(cm))
    keep = []
    with array_arith(flags):
        if q8 is None:
            orc.orc_bert_run(encoder_struct(m, keep), P(emb), P(cm), B, S, -1)
        else:
            ops = OrcI8()
            for i, (q, ws, sm) in enumerate(q8):
                ias = np.ascontiguousarray((np.float32(1.0) / sm).astype(np.float32))
                keep += [q, ws, ias]
                ops.wq[i], ops.wscale[i], ops.ias[i] = (q.ctypes.data, ws.ctypes.data,
                                                        ias.ctypes.data)
            orc.orc_bert_run_i8(encoder_struct(m, keep), ops, P(emb), P(cm), B, S, -1)
    out = np.empty((B, d), np.float32)
    assert orc.orc_pool_rows(P(emb), P(am), B, S, d, int(m["cls_pool"]), 1, P(out)) == 0
    return out


def _embed(ctx, enc, ids, am):
    B, S = ids.shape
    out = ctx.empty((B, enc.desc.hidden), np.float32)
    enc.embed(ctx.put(ids), ctx.put(am), B, S, out)
    return out.host()


ARRAY = ORC_ARR_A_BF16 | ORC_ARR_C_BF16 | ORC_ARR_ATTN_BF16

CASES = {
    "minilm": lambda: (synth.make_model("minilm", layers=3, ln_random=True), None),
    "bge_int8": lambda: (lambda m: (m, synth.quantise_model(m)))(
        synth.make_model("bge_base", layers=2, hidden=256, heads=4, head_dim=64, ffn=1024,
                         ln_random=True)),
    "nomic": lambda: (synth.make_model("nomic", layers=2, hidden=256, heads=4, head_dim=64,
                                       ffn=512, ln_random=True), None),
    "gte": lambda: (synth.make_model("gte", layers=2, hidden=256, heads=4, head_dim=64,
                                     ffn=512, ln_random=True), None),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_encoder_narrowed_c_matches_the_array_oracle(ctx, orc, name):
    """The stack with every GEMM's C narrowed, against the oracle's stack in the
    array arithmetic (bf16 A, narrowed C, bf16 attention operands): cosine >=
    0.9999 per sequence; the switch changes the GPU result (it is applied);
    token packing stays bit-identical to the padded computation under it."""
    m, q8 = CASES[name]()
    ids, am, _ = synth.make_text_inputs(m, batch=8, seq=96)
    enc = mxenc.Encoder(ctx, m, int8=q8) if q8 else mxenc.Encoder(ctx, m)
    plain = _embed(ctx, enc, ids, am)
    enc.set_narrowed_c(True)
    got = _embed(ctx, enc, ids, am)
    enc.set_packing(False)
    padded = _embed(ctx, enc, ids, am)
    enc.close()
    assert np.array_equal(got.view(np.uint32), padded.view(np.uint32))
    assert not np.array_equal(got.view(np.uint32), plain.view(np.uint32))
    want = _oracle(orc, m, ids, am, ARRAY, q8)
    cos = _cos(got, want)
    print(f"{name}: 1-cos gpu~array oracle {1 - cos.min():.3e}, "
          f"gpu plain~array oracle {1 - _cos(plain, want).min():.3e}")
    assert cos.min() >= 0.9999, cos.min()
