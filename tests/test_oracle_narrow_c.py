"""The oracle's narrowed-C arithmetic: the array designs that narrow C to bf16
on the core (c_elem_bytes == 2, the export default) and finish on the host
from the bf16 value -- dequantise_c's 2-byte branch, the bf16-C bias add and
dequant_act_bf16. Pinned against the reference's own dequantise_c compiled
into oracle/_ref, against oracle/_ref's gelu8 and to_bf16 composed on the
closed-form bias add, and against the closed form itself."""
import numpy as np
import pytest

from orc import P, aligned_empty, encoder_struct, array_arith, ORC_ARR_A_BF16, \
    ORC_ARR_C_BF16, ORC_ARR_ATTN_BF16
from mxenc import synth


def _bf16_bits(rng, shape, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def _widen(c):
    return (c.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("M,N", [(40, 1152), (9, 64), (3, 3072)])
def test_dequantise_c_bf16_matches_reference_bitwise(orc, ref, M, N):
    """dequantise_c with a 2-byte C, restated, against the reference's own
    template at c_bytes = 2 (its streaming loads need N % 16 == 0)."""
    rng = np.random.default_rng(M * N + 1)
    C = aligned_empty((M, N), np.uint16)
    C[:] = _bf16_bits(rng, (M, N), 3e4)
    C[0, :6] = [0x0000, 0x8000, 0x3F80, 0xBF80, 0x4B80, 0xCB80]  # +-0, +-1, +-2^24
    sa = rng.uniform(1e-4, 1e-1, M).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    o0, o1 = np.zeros((M, N), np.float32), np.zeros((M, N), np.float32)
    orc.orc_dequantise_c_bf16(P(C), M, N, P(sa), P(ws), P(bias), P(o0))
    assert ref.ref_dequantise_c_bf16(P(C), M, N, P(sa), P(ws), P(bias), P(o1)) == 0
    assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32))
    # the FMA form is what pins it: the two-rounding form differs somewhere
    two = (_widen(C) * sa[:, None]) * ws[None, :] + bias[None, :]
    assert not np.array_equal(two.astype(np.float32).view(np.uint32), o0.view(np.uint32))


def test_bias_c_bf16_is_the_widened_value_plus_bias(orc):
    rng = np.random.default_rng(5)
    M, N = 33, 768
    C = _bf16_bits(rng, (M, N), 4.0)
    bias = rng.standard_normal(N).astype(np.float32)
    out = np.zeros((M, N), np.float32)
    orc.orc_bias_c_bf16(P(C), M, N, P(bias), P(out))
    want = _widen(C) + bias[None, :]  # one IEEE fp32 add of an exact widening
    assert np.array_equal(out.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_dequant_act_bf16_is_gelu8_then_to_bf16_of_the_biased_value(orc, ref):
    """dequant_act_bf16's plain-GELU branch, composed from oracle/_ref's own
    gelu8 (AVX2 form, the one the host runs for N % 8 == 0) and bf16_fill."""
    rng = np.random.default_rng(11)
    M, N = 17, 1536
    C = _bf16_bits(rng, (M, N), 2.0)
    bias = rng.standard_normal(N).astype(np.float32)
    got = np.zeros((M, N), np.uint16)
    orc.orc_dequant_act_bf16(P(C), M, N, 0, P(bias), P(got))
    v = np.ascontiguousarray((_widen(C) + bias[None, :]).astype(np.float32))
    g = np.empty_like(v)
    ref.ref_gelu8_avx2(P(v), P(g), v.size)
    want = np.empty((M, N), np.uint16)
    ref.ref_bf16_fill(P(want), P(g), v.size)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("gated", [1, 2])
def test_dequant_act_bf16_gated_halves(orc, gated):
    """The gated branch: the widened, biased halves combined by the oracle's
    pinned glu (lo * act(hi), hi the second half), rounded once."""
    rng = np.random.default_rng(gated)
    M, f = 12, 256
    C = _bf16_bits(rng, (M, 2 * f), 2.0)
    bias = rng.standard_normal(2 * f).astype(np.float32)
    got = np.zeros((M, f), np.uint16)
    orc.orc_dequant_act_bf16(P(C), M, 2 * f, gated, P(bias), P(got))
    v = np.ascontiguousarray((_widen(C) + bias[None, :]).astype(np.float32))
    g = np.empty((M, f), np.float32)
    orc.orc_glu(P(v), M, f, gated, P(g))
    want = np.empty((M, f), np.uint16)
    orc.orc_bf16_fill(P(want), P(g), g.size)
    assert np.array_equal(got, want)
    # and the gate is the second half: swapping the halves changes the result
    sw = np.ascontiguousarray(np.concatenate([v[:, f:], v[:, :f]], axis=1))
    orc.orc_glu(P(sw), M, f, gated, P(g))
    orc.orc_bf16_fill(P(want), P(g), g.size)
    assert not np.array_equal(got, want)


def test_array_arith_switches_change_the_stack_only_as_stated(orc):
    """The whole-stack restatement with the array datapath's roundings: each
    switch moves the result (so it is applied), every switch keeps it within
    bf16 noise of the host path, and clearing them restores the host path bit
    for bit."""
    m = synth.make_model("minilm", layers=2, ln_random=True)
    ids, am, _ = synth.make_text_inputs(m, batch=2, seq=64)
    B, S, d = 2, 64, m["hidden"]
    emb = np.empty((B * S, d), np.float32)
    cm = np.empty((B, S), np.float32)
    orc.orc_embed_sum(P(ids), P(am), B, S, d, P(m["word"]), P(m["pos"]), P(m["type"]),
                      P(emb), P(cm))
    keep = []
    enc = encoder_struct(m, keep)

    def run(flags):
        x = emb.copy()
        with array_arith(flags):
            orc.orc_bert_run(enc, P(x), P(cm), B, S, -1)
        return x

    host = run(0)
    rows = am.reshape(-1) > 0
    for flags in (ORC_ARR_A_BF16, ORC_ARR_C_BF16, ORC_ARR_ATTN_BF16,
                  ORC_ARR_A_BF16 | ORC_ARR_C_BF16 | ORC_ARR_ATTN_BF16):
        x = run(flags)
        assert not np.array_equal(x, host), flags
        a, b = x[rows].astype(np.float64), host[rows].astype(np.float64)
        cos = np.sum(a * b, 1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))
        assert cos.min() > 0.999, (flags, cos.min())
    assert np.array_equal(run(0), host)
