"""GPU parity of the int8 (W8A8) datapath through the C ABI: quantise_a_int8,
the exact int8 GEMM, dequantise_c fused into its epilogue, and add_norm_quant,
against the oracle (itself pinned bit-exact to the reference's own
quantise_a_int8/dequantise_c and to a 64-bit integer product). Integer work
and the quantisation are checked bit for bit."""
import numpy as np
import pytest

import mxenc
from orc import P, quantise_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = mxenc.Context(0)
    yield c
    c.close()


def _rows(rng, M, K):
    a = (rng.standard_normal((M, K)) * rng.uniform(0.01, 30, size=(M, 1))).astype(np.float32)
    a[1] = 0.0                        # an all-zero row: scale 1, all zeros
    a[2, 5] = 1e30                    # one huge element
    a[3] = np.float32(0.5) * np.arange(K, dtype=np.float32) - 7.0  # exact halves
    return a


def _oracle_quantise(orc, a, ias):
    M, K = a.shape
    q, s = np.zeros((M, K), np.int8), np.zeros(M, np.float32)
    orc.orc_quantise_a_int8(P(np.ascontiguousarray(a)), M, K, P(ias), P(q), P(s))
    return q, s


@pytest.mark.parametrize("M,K", [(64, 384), (33, 1536), (8, 64), (517, 768), (5, 5120),
                                 (6, 8192), (4, 260)])
def test_quantise_bit_exact(ctx, orc, M, K):
    rng = np.random.default_rng(M * K)
    a = _rows(rng, M, K)
    ias = (1.0 / rng.uniform(0.5, 2.0, K)).astype(np.float32)
    want_q, want_s = _oracle_quantise(orc, a, ias)
    q, s = ctx.empty((M, K), np.int8), ctx.empty((M,), np.float32)
    mxenc.quantise_a_int8(ctx, ctx.put(a), M, K, ctx.put(ias), q, s)
    assert np.array_equal(s.host().view(np.uint32), want_s.view(np.uint32))
    got = q.host()
    bad = np.argwhere(got != want_q)
    assert bad.size == 0, f"first mismatch at {bad[0]}: {got[tuple(bad[0])]} != " \
                          f"{want_q[tuple(bad[0])]}"


def test_quantise_bf16_input(ctx, orc):
    rng = np.random.default_rng(11)
    M, K = 129, 3072
    a = mxenc.from_bf16_bits(mxenc.to_bf16_bits(_rows(rng, M, K)))
    ias = (1.0 / rng.uniform(0.5, 2.0, K)).astype(np.float32)
    want_q, want_s = _oracle_quantise(orc, a, ias)
    q, s = ctx.empty((M, K), np.int8), ctx.empty((M,), np.float32)
    mxenc.quantise_a_int8(ctx, ctx.put(mxenc.to_bf16_bits(a)), M, K, ctx.put(ias), q, s)
    assert np.array_equal(q.host(), want_q)
    assert np.array_equal(s.host().view(np.uint32), want_s.view(np.uint32))


def _i8(rng, shape):
    return rng.integers(-127, 128, shape, dtype=np.int8)


@pytest.mark.parametrize("M,K,N", [(300, 768, 2304), (4096, 3072, 768), (77, 256, 100),
                                   (1030, 1024, 1028), (2048, 384, 1536)])
def test_gemm_i8_raw_is_the_exact_integer_product(ctx, M, K, N):
    rng = np.random.default_rng(M + K + N)
    A, W = _i8(rng, (M, K)), _i8(rng, (K, N))
    A[0] = 127
    W[:, 0] = 127                      # the largest accumulation of the shape
    A[1] = -127
    ws = np.ones(N, np.float32)
    sm = np.ones(K, np.float32)
    slot = mxenc.stage_weight_i8(ctx, W, ws, sm)
    C = ctx.empty((M, N), np.int32)
    mxenc.gemm_i8(ctx, ctx.put(A), None, M, K, K, slot, None, mxenc.MX_EPI_NONE, None, C, N)
    got = C.host().astype(np.int64)
    want = A.astype(np.int64) @ W.astype(np.int64)
    assert np.array_equal(got, want)
    assert got[0, 0] == K * 127 * 127 and got[1, 0] == -K * 127 * 127
    mxenc.check(mxenc.lib().mx_release_weight(ctx.handle, slot))


@pytest.mark.parametrize("M,K,N", [(32768, 768, 768), (20000, 768, 2304)])
def test_gemm_i8_raw_multi_tile_per_block(ctx, M, K, N):
    """More tiles than CUs: each persistent block runs several tiles, and the
    slab waits after an epilogue leave its stores in flight -- any slab read
    before its loads landed would show as a wrong integer."""
    rng = np.random.default_rng(M + N)
    A, W = _i8(rng, (M, K)), _i8(rng, (K, N))
    slot = mxenc.stage_weight_i8(ctx, W, np.ones(N, np.float32), np.ones(K, np.float32))
    C = ctx.empty((M, N), np.int32)
    mxenc.gemm_i8(ctx, ctx.put(A), None, M, K, K, slot, None, mxenc.MX_EPI_NONE, None, C, N)
    got = C.host()
    want = A.astype(np.float64) @ W.astype(np.float64)  # exact: |sum| < 2^31
    assert np.array_equal(got, want.astype(np.int32))
    mxenc.check(mxenc.lib().mx_release_weight(ctx.handle, slot))


@pytest.mark.parametrize("M,K,N,bias", [(1000, 768, 2304, True), (4096, 3072, 768, True),
                                        (257, 512, 68, False)])
def test_gemm_i8_dequant_bit_exact(ctx, orc, M, K, N, bias):
    """fp32 C: dequantise_c fused, bit-identical to the host's int32-C form."""
    rng = np.random.default_rng(K + N)
    A = _i8(rng, (M, K))
    W = _i8(rng, (K, N))
    sa = rng.uniform(1e-4, 1e-1, M).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if bias else np.zeros(N, np.float32)
    c32 = np.zeros((M, N), np.int32)
    orc.orc_gemm_i8(P(A), M, K, P(W), N, P(c32))
    want = np.zeros((M, N), np.float32)
    orc.orc_dequantise_c(P(c32), M, N, P(sa), P(ws), P(b), P(want))
    slot = mxenc.stage_weight_i8(ctx, W, ws, np.ones(K, np.float32))
    C = ctx.empty((M, N), np.float32)
    mxenc.gemm_i8(ctx, ctx.put(A), ctx.put(sa), M, K, K, slot, ctx.put(b) if bias else None,
                  mxenc.MX_EPI_NONE, None, C, N)
    got = C.host()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # bf16 C is the same value narrowed once (round to nearest even); its rows
    # are stored 16 bytes at a time, so N % 8 != 0 is refused by name
    Cb = ctx.empty((M, N), np.uint16)
    if N % 8:
        with pytest.raises(mxenc.MxError, match="16-byte aligned"):
            mxenc.gemm_i8(ctx, ctx.put(A), ctx.put(sa), M, K, K, slot, None,
                          mxenc.MX_EPI_NONE, None, Cb, N)
    else:
        mxenc.gemm_i8(ctx, ctx.put(A), ctx.put(sa), M, K, K, slot, ctx.put(b) if bias else None,
                      mxenc.MX_EPI_NONE, None, Cb, N)
        assert np.array_equal(Cb.host(), mxenc.to_bf16_bits(want))
    mxenc.check(mxenc.lib().mx_release_weight(ctx.handle, slot))


@pytest.mark.parametrize("K,epi", [(1024, mxenc.MX_EPI_NONE), (384, mxenc.MX_EPI_GELU_POLY)])
def test_gemm_i8_deep_tile_bit_exact(ctx, orc, K, epi):
    """The 256 x 256 tile on 128-byte slabs (bf16 C, no residual, K % 128 ==
    0; K = 384 is an odd number of slabs): dequantise_c (and the activation)
    fused, bit-identical to the host forms, on a subset of rows (rows are
    independent): the first and last 256 and 256 random ones."""
    M, N = 8000, 2048
    assert mxenc.lib().mx_gemm_plan_for(M, N, K, mxenc.MX_BF16, 0, 1).decode().startswith(
        "lds_256x256x128")
    rng = np.random.default_rng(K)
    A, W = _i8(rng, (M, K)), _i8(rng, (K, N))
    sa = rng.uniform(1e-4, 1e-2, M).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    slot = mxenc.stage_weight_i8(ctx, W, ws, np.ones(K, np.float32))
    C = ctx.empty((M, N), np.uint16)
    mxenc.gemm_i8(ctx, ctx.put(A), ctx.put(sa), M, K, K, slot, ctx.put(b), epi, None, C, N)
    got = C.host()
    rows = np.unique(np.concatenate([np.arange(256), np.arange(M - 256, M),
                                     rng.integers(0, M, 256)]))
    Ar = np.ascontiguousarray(A[rows])
    c32 = np.zeros((rows.size, N), np.int32)
    orc.orc_gemm_i8(P(Ar), rows.size, K, P(W), N, P(c32))
    want = np.zeros((rows.size, N), np.float32)
    sar = np.ascontiguousarray(sa[rows])
    orc.orc_dequantise_c(P(c32), rows.size, N, P(sar), P(ws), P(b), P(want))
    if epi == mxenc.MX_EPI_GELU_POLY:
        orc.orc_gelu_poly_inplace(P(want), want.size)
    assert np.array_equal(got[rows], mxenc.to_bf16_bits(want))
    mxenc.check(mxenc.lib().mx_release_weight(ctx.handle, slot))


def test_gemm_i8_gelu_epilogue_is_dequant_act(ctx, orc):
    """FFN up on the int8 design: dequantise, bias, then the host's gelu8 --
    the first half of dequant_act_quant (host_kernels.hpp:405-500), bit for bit."""
    rng = np.random.default_rng(5)
    M, K, N = 512, 768, 3072
    A, W = _i8(rng, (M, K)), _i8(rng, (K, N))
    sa = rng.uniform(1e-3, 3e-2, M).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-3, N).astype(np.float32)
    b = (rng.standard_normal(N) * 0.5).astype(np.float32)
    c32 = np.zeros((M, N), np.int32)
    orc.orc_gemm_i8(P(A), M, K, P(W), N, P(c32))
    want = np.zeros((M, N), np.float32)
    orc.orc_dequantise_c(P(c32), M, N, P(sa), P(ws), P(b), P(want))
    orc.orc_gelu_poly_inplace(P(want), want.size)
    C = ctx.empty((M, N), np.float32)
    Wt = ctx.put(np.ascontiguousarray(W.T))
    mxenc.gemm_i8_wt(ctx, ctx.put(A), ctx.put(sa), M, K, K, Wt, ctx.put(ws), N, ctx.put(b),
                     mxenc.MX_EPI_GELU_POLY, None, C, N)
    assert np.array_equal(C.host().view(np.uint32), want.view(np.uint32))


def test_gemm_i8_end_to_end_tracks_fp32(ctx, orc):
    """quantise -> int8 GEMM -> dequantise on the packer's operand scheme equals
    the oracle's gemm_i8_dequant bit for bit, and stays within int8 noise of
    the fp32 product of the unquantised operands."""
    rng = np.random.default_rng(9)
    M, K, N = 640, 768, 768
    a = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    asm = rng.uniform(0.5, 2.0, K).astype(np.float32)
    b = (rng.standard_normal(N) * 0.02).astype(np.float32)
    q, s = quantise_weights(w, asm)
    ias = (np.float32(1.0) / asm).astype(np.float32)
    want = np.zeros((M, N), np.float32)
    orc.orc_gemm_i8_dequant(P(a), M, K, P(ias), P(q), P(s), P(b), N, P(want))
    slot = mxenc.stage_weight_i8(ctx, q, s, asm)
    _, dias = mxenc.weight_i8_scales(ctx, slot)
    aq, asc = ctx.empty((M, K), np.int8), ctx.empty((M,), np.float32)
    mxenc.quantise_a_int8(ctx, ctx.put(a), M, K, dias, aq, asc)
    C = ctx.empty((M, N), np.float32)
    mxenc.gemm_i8(ctx, aq, asc, M, K, K, slot, ctx.put(b), mxenc.MX_EPI_NONE, None, C, N)
    got = C.host()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ref = a.astype(np.float64) @ w.astype(np.float64) + b
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    assert rel < 3e-2, rel
    mxenc.check(mxenc.lib().mx_release_weight(ctx.handle, slot))


@pytest.mark.parametrize("cols,ybf", [(768, True), (384, False), (1024, True)])
def test_layernorm_quant(ctx, orc, cols, ybf):
    """add_norm_quant: the fp32 LayerNorm (within the LayerNorm bar of the
    oracle's) and the quantisation of that very output, bit for bit."""
    rng = np.random.default_rng(cols)
    rows = 333
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    y = (rng.standard_normal((rows, cols)) * 0.5).astype(np.float32)
    if ybf:
        y = mxenc.from_bf16_bits(mxenc.to_bf16_bits(y))
    g = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    bt = (rng.standard_normal(cols) * 0.1).astype(np.float32)
    ias = (1.0 / rng.uniform(0.5, 2.0, cols)).astype(np.float32)
    dx = ctx.put(x)
    dy = ctx.put(mxenc.to_bf16_bits(y) if ybf else y)
    dg, dbt, dias = ctx.put(g), ctx.put(bt), ctx.put(ias)
    # out of place first (cached accesses), then in place over x as the stack
    # calls it (streaming accesses): the same bits
    of = ctx.empty((rows, cols), np.float32)
    q0, s0 = ctx.empty((rows, cols), np.int8), ctx.empty((rows,), np.float32)
    mxenc.layernorm_i8(ctx, dx, dy, dg, dbt, 1e-12, rows, cols, of, dias, q0, s0)
    q, s = ctx.empty((rows, cols), np.int8), ctx.empty((rows,), np.float32)
    mxenc.layernorm_i8(ctx, dx, dy, dg, dbt, 1e-12, rows, cols, dx, dias, q, s)
    ln = dx.host()
    assert np.array_equal(ln.view(np.uint32), of.host().view(np.uint32))
    assert np.array_equal(q.host(), q0.host())
    assert np.array_equal(s.host().view(np.uint32), s0.host().view(np.uint32))
    want = x + y
    orc.orc_layer_norm_rows(P(want), rows, cols, P(g), P(bt), np.float32(1e-12))
    assert np.abs(ln - want).max() <= 2e-5 * max(1.0, float(np.abs(want).max()))
    want_q, want_s = _oracle_quantise(orc, ln, ias)
    assert np.array_equal(q.host(), want_q)
    assert np.array_equal(s.host().view(np.uint32), want_s.view(np.uint32))


def test_i8_refusals(ctx):
    import ctypes
    rng = np.random.default_rng(0)
    L = mxenc.lib()
    W = _i8(rng, (288, 64))
    slot = mxenc.stage_weight_i8(ctx, W, np.ones(64, np.float32), np.ones(288, np.float32))
    A, C = ctx.put(_i8(rng, (8, 288))), ctx.empty((8, 64), np.float32)
    sa = ctx.put(np.ones(8, np.float32))
    # K = 288 is not a whole number of 64-deep slabs: refused by name
    rc = L.mx_gemm_i8(ctx.stream, A.p, sa.p, 8, 288, 288, slot, None, 0, None, C.p,
                      mxenc.MX_F32, 64)
    assert rc == -3 and "64-deep slabs" in L.mx_last_error().decode()
    # an int8 slot is not a bf16 operand, and the other way round
    rc = L.mx_gemm(ctx.stream, A.p, 8, 288, 288, slot, None, 0, None, C.p, mxenc.MX_F32, 64)
    assert rc == -1 and "mx_gemm_i8" in L.mx_last_error().decode()
    bslot = ctypes.c_int()
    wb = np.zeros((256, 64), np.float32)
    mxenc.check(L.mx_stage_weight(ctx.handle, wb.ctypes.data, mxenc.MX_F32, 256, 64,
                                  ctypes.byref(bslot)))
    rc = L.mx_gemm_i8(ctx.stream, A.p, sa.p, 8, 256, 256, bslot.value, None, 0, None, C.p,
                      mxenc.MX_F32, 64)
    assert rc == -1 and "bf16 operand" in L.mx_last_error().decode()
    # dequantisation needs both scales; the raw product takes no bias
    Wt = ctx.put(np.zeros((64, 256), np.int8))
    rc = L.mx_gemm_i8_wt(ctx.stream, A.p, None, 8, 256, 256, Wt.p, None, 64, None, 0, None, C.p,
                         mxenc.MX_F32, 64)
    assert rc == -1 and "a_scale and wscale" in L.mx_last_error().decode()
    rc = L.mx_gemm_i8_wt(ctx.stream, A.p, None, 8, 256, 256, Wt.p, None, 64, sa.p, 0, None,
                         C.p, mxenc.MX_I32, 64)
    assert rc == -1 and "raw accumulator" in L.mx_last_error().decode()
    # K past the int32 accumulator's exact range
    rc = L.mx_gemm_i8_wt(ctx.stream, A.p, None, 8, 133184, 133184, Wt.p, None, 64, None, 0, None,
                         C.p, mxenc.MX_I32, 64)
    assert rc == -1 and "overflow" in L.mx_last_error().decode()
    mxenc.check(L.mx_release_weight(ctx.handle, slot))
    mxenc.check(L.mx_release_weight(ctx.handle, bslot.value))


# ---- the int8 encoder stack ----------------------------------------------------

from mxenc import synth  # noqa: E402
from orc import OrcI8, encoder_struct  # noqa: E402


def _cos(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return np.sum(a * b, -1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1))


def _oracle_embed(orc, m, ids, am, q8=None):
    """EmbedService::chunk on the host; q8: the int8 stack (orc_bert_run_i8) on
    those operands, else the fp32 stack."""
    B, S = ids.shape
    d = m["hidden"]
    emb = np.empty((B * S, d), np.float32)
    cm = np.empty((B, S), np.float32)
    orc.orc_embed_sum(P(ids), P(am), B, S, d, P(m["word"]), P(m["pos"]), P(m["type"]), P(emb),
                      P(cm))
    keep = []
    if q8 is None:
        orc.orc_bert_run(encoder_struct(m, keep), P(emb), P(cm), B, S, -1)
    else:
        ops = OrcI8()
        for i, (q, ws, sm) in enumerate(q8):
            ias = np.ascontiguousarray((np.float32(1.0) / sm).astype(np.float32))
            keep += [q, ws, ias]
            ops.wq[i], ops.wscale[i], ops.ias[i] = q.ctypes.data, ws.ctypes.data, ias.ctypes.data
        orc.orc_bert_run_i8(encoder_struct(m, keep), ops, P(emb), P(cm), B, S, -1)
    out = np.empty((B, d), np.float32)
    assert orc.orc_pool_rows(P(emb), P(am), B, S, d, int(m["cls_pool"]), 1, P(out)) == 0
    return out


def _gpu_embed(ctx, enc, ids, am):
    B, S = ids.shape
    out = ctx.empty((B, enc.desc.hidden), np.float32)
    enc.embed(ctx.put(ids), ctx.put(am), B, S, out)
    return out.host()


def _dequantised(m, q8):
    """The fp32 model whose GEMM operands are the int8 operands dequantised
    (W = q * wscale / asmooth): the host fp32 path of an int8 container."""
    md = dict(m)
    for key, (q, ws, sm) in zip(synth.GEMM_KEYS, q8):
        md[key] = (q.astype(np.float32) * ws[:, None, :] / sm[:, :, None]).astype(np.float32)
    return md


def _check_i8_parity(got8, host8, hostf, tag):
    """The int8 datapath's end-to-end bar. The integer product, the
    quantisation and the dequantisation are pinned bit for bit per op (above),
    and between the quantisers the GPU keeps the host's fp32 where the
    reference does (FFN-up's activation up to its quantiser, as
    dequant_act_quant; the attention-out and FFN-down results, as
    dequantise_c). Attention still runs on bf16 Q/K/V into a bf16 context,
    and a value that lands on the other side of an int8 rounding boundary
    moves by a whole step of the grid. So the GPU's departure from the host
    int8 result is measured against the int8 scheme's own error e (host int8
    against the host fp32 stack on the dequantised operands): (1) the GPU int8
    result is as accurate as the host's, within 10 %; (2) GPU and host int8
    differ by at most 1.75 e (two independent draws of the same grid noise
    differ by ~2 e; measured on bge-base: 1.39 e)."""
    e_scheme = 1.0 - _cos(host8, hostf)
    e_gpu = 1.0 - _cos(got8, hostf)
    e_pair = 1.0 - _cos(got8, host8)
    print(f"{tag}: 1-cos gpu8~host8 {e_pair.max():.3e}, host8~fp32 {e_scheme.max():.3e}, "
          f"gpu8~fp32 {e_gpu.max():.3e}")
    assert np.all(e_gpu <= 1.1 * e_scheme + 1e-5), (e_gpu, e_scheme)
    assert np.all(e_pair <= 1.75 * e_scheme + 1e-5), (e_pair, e_scheme)


def test_i8_stack_minilm_full_config(ctx, orc):
    """all-MiniLM-L6-v2 geometry (32 x 128, 6 layers, mean pooling) on the
    int8 datapath, whole batch, against the oracle's int8 stack (the array
    path's host halves restated): cosine >= 0.9999 per sequence, and the
    int8 bar of _check_i8_parity."""
    m = synth.make_model("minilm", ln_random=True)
    q8 = synth.quantise_model(m)
    ids, am, _ = synth.make_text_inputs(m)
    want = _oracle_embed(orc, m, ids, am, q8)
    enc = mxenc.Encoder(ctx, m, int8=q8)
    got = _gpu_embed(ctx, enc, ids, am)
    enc.close()
    assert _cos(got, want).min() >= 0.9999
    _check_i8_parity(got, want, _oracle_embed(orc, _dequantised(m, q8), ids, am), "minilm int8")
    assert np.max(np.abs(np.linalg.norm(got, axis=1) - 1)) < 1e-6


def test_i8_stack_bge_base_full_batch_subset_checked(ctx, orc):
    """bge-base geometry at its full shape (64 x 512, 12 layers, CLS pooling)
    on the int8 datapath; the shortest, the longest and one more sequence rerun
    on the oracle's int8 and fp32 stacks. CLS pooling keeps one row, so the
    int8 grid noise is not averaged away (1 - cos ~ 6e-4 for the host's own
    int8 against fp32)."""
    m = synth.make_model("bge_base")
    q8 = synth.quantise_model(m)
    ids, am, lens = synth.make_text_inputs(m)
    enc = mxenc.Encoder(ctx, m, int8=q8)
    got = _gpu_embed(ctx, enc, ids, am)
    enc.close()
    pick = [int(np.argmin(lens)), int(np.argmax(lens)), 5]
    ii, aa = np.ascontiguousarray(ids[pick]), np.ascontiguousarray(am[pick])
    _check_i8_parity(got[pick], _oracle_embed(orc, m, ii, aa, q8),
                     _oracle_embed(orc, _dequantised(m, q8), ii, aa), "bge-base int8")


def test_i8_stack_bge_base_every_sequence_gap_is_the_grid(ctx, orc):
    """bge-base at its full shape on the int8 datapath, every one of the 64
    sequences rerun on the oracle (chunks of 16; sequences are independent).

    What the GPU~host int8 gap is. Rounding Q, K, V and the attention context
    to bf16 in the oracle (ORC_ARR_ATTN_BF16, what the GPU's attention does)
    moves the oracle only ~5 % closer to the GPU, so that rounding is not the
    cause. The cause is the int8 grid itself: any ulp-level difference ahead
    of a quantiser (LayerNorm sum order, attention arithmetic) moves some
    values across a rounding boundary by a whole step, and from there the two
    runs carry independent draws of the grid noise. The same gap appears
    between two HOST runs that differ only by that bf16 rounding (e_self).
    So the bar: (1) the GPU differs from the host int8 stack by no more than
    the host differs from itself under that perturbation (means over the 64
    sequences, within 25 %); (2) the GPU int8 result is as accurate as the
    host's against the fp32 stack on the dequantised operands (mean within
    10 %, every sequence within 25 % of the host's worst); (3) no sequence
    differs from the host by more than 2.5 times the scheme's own error."""
    from orc import array_arith, ORC_ARR_ATTN_BF16
    m = synth.make_model("bge_base")
    q8 = synth.quantise_model(m)
    ids, am, lens = synth.make_text_inputs(m)
    enc = mxenc.Encoder(ctx, m, int8=q8)
    got = _gpu_embed(ctx, enc, ids, am)
    enc.close()
    host8, host8a, hostf = [], [], []
    md = _dequantised(m, q8)
    for lo in range(0, 64, 16):
        ii, aa = np.ascontiguousarray(ids[lo:lo + 16]), np.ascontiguousarray(am[lo:lo + 16])
        print(f"int8 bge-base oracle: sequences {lo}..{lo + 15}", flush=True)
        host8.append(_oracle_embed(orc, m, ii, aa, q8))
        with array_arith(ORC_ARR_ATTN_BF16):
            host8a.append(_oracle_embed(orc, m, ii, aa, q8))
        hostf.append(_oracle_embed(orc, md, ii, aa))
    host8, host8a, hostf = (np.concatenate(x) for x in (host8, host8a, hostf))
    e_pair = 1.0 - _cos(got, host8)
    e_pair_a = 1.0 - _cos(got, host8a)
    e_self = 1.0 - _cos(host8, host8a)
    e_scheme = 1.0 - _cos(host8, hostf)
    e_gpu = 1.0 - _cos(got, hostf)
    print(f"bge-base int8, 64 sequences, 1-cos mean / max: gpu~host8 {e_pair.mean():.3e} / "
          f"{e_pair.max():.3e}; gpu~host8(bf16 attention) {e_pair_a.mean():.3e} / "
          f"{e_pair_a.max():.3e}; host8~host8(bf16 attention) {e_self.mean():.3e} / "
          f"{e_self.max():.3e}; host8~fp32 {e_scheme.mean():.3e} / {e_scheme.max():.3e}; "
          f"gpu8~fp32 {e_gpu.mean():.3e} / {e_gpu.max():.3e}")
    assert e_pair.mean() <= 1.25 * e_self.mean(), (e_pair.mean(), e_self.mean())
    assert e_gpu.mean() <= 1.1 * e_scheme.mean(), (e_gpu.mean(), e_scheme.mean())
    assert e_gpu.max() <= 1.25 * e_scheme.max(), (e_gpu.max(), e_scheme.max())
    assert np.all(e_pair <= 2.5 * e_scheme), np.max(e_pair / e_scheme)


def test_i8_container_is_bitwise_the_set_encoder(tmp_path, ctx):
    """An --int8 container (I8 block panels with .wscale/.asmooth) loaded by
    mx_encoder_from_npue runs bit-identically to the same operands set by
    name; lane clones and the embed service keep those bits."""
    import npue_writer as nw
    m = synth.make_model("minilm", layers=2, ln_random=True)
    q8 = synth.quantise_model(m)
    path = str(tmp_path / "minilm_i8.npue")
    nw.bert_container(m, 64, 48, (8, 4), int8=q8).write(path)
    f = mxenc.Npue(path)
    assert f.config("a_dtype") == "i8"
    a_enc = mxenc.Encoder.from_npue(ctx, f)
    b_enc = mxenc.Encoder(ctx, m, int8=q8)
    ids, am, _ = synth.make_text_inputs(m, batch=10)
    a = _gpu_embed(ctx, a_enc, ids, am)
    b = _gpu_embed(ctx, b_enc, ids, am)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    svc = mxenc.EmbedService(b_enc, lanes=2, batch=4, seq=ids.shape[1])
    c = svc.embed(ids, am)
    svc.close()
    assert np.array_equal(c.view(np.uint32), b.view(np.uint32))
    a_enc.close()
    b_enc.close()
    f.close()


def test_i8_stack_mixed_datapath_refused(ctx):
    m = synth.make_model("minilm", layers=2)
    q8 = synth.quantise_model(m)
    enc = mxenc.Encoder(ctx, m, int8=q8)
    # one operand replaced by a bf16 one: the stack runs one datapath
    with pytest.raises(mxenc.MxError, match="one datapath"):
        enc.set("layer.1.ffn_up", m["w_up"][1])
        mxenc.check(mxenc.lib().mx_encoder_ready(enc.handle))
    enc.close()
