"""The oracle's int8 W8A8 datapath (the array path's host halves and the
exact integer product), pinned against the reference's own quantise_a_int8
and dequantise_c compiled into oracle/_ref, a 64-bit integer product and the
scheme's closed-form bounds."""
import numpy as np
import pytest

from orc import P, aligned_empty, encoder_struct, quantise_weights, OrcI8
from mxenc import synth


def _rows(rng, M, K):
    a = (rng.standard_normal((M, K)) * rng.uniform(0.01, 30, size=(M, 1))).astype(np.float32)
    a[1] = 0.0                        # an all-zero row: scale 1, all zeros
    a[2, 5] = 1e30                    # one huge element
    a[3] = np.float32(0.5) * np.arange(K, dtype=np.float32) - 7.0  # exact halves
    return a


@pytest.mark.parametrize("M,K", [(64, 384), (33, 1536), (8, 64)])
def test_quantise_matches_reference_bitwise(orc, ref, M, K):
    rng = np.random.default_rng(M * K)
    a = _rows(rng, M, K)
    ias = (1.0 / rng.uniform(0.5, 2.0, K)).astype(np.float32)
    q0, s0 = np.zeros((M, K), np.int8), np.zeros(M, np.float32)
    q1, s1 = np.zeros((M, K), np.int8), np.zeros(M, np.float32)
    orc.orc_quantise_a_int8(P(a), M, K, P(ias), P(q0), P(s0))
    ref.ref_quantise_a_int8(P(a), M, K, P(ias), P(q1), P(s1))
    assert np.array_equal(q0, q1) and np.array_equal(s0.view(np.uint32), s1.view(np.uint32))
    # closed form: |q| <= 127, the row maximum maps to +-127, zero rows stay zero
    assert np.abs(q0.astype(np.int32)).max() <= 127
    nz = np.abs(a * ias).max(axis=1) > 0
    assert np.all(np.abs(q0[nz].astype(np.int32)).max(axis=1) == 127)
    assert s0[1] == 1.0 and not q0[1].any()
    # each value is within half a step of its quantised image
    err = np.abs(a * ias / s0[:, None] - q0)
    assert np.all(err[nz] <= 0.5 + 1e-3)


def test_gemm_i8_is_the_exact_integer_product(orc):
    rng = np.random.default_rng(7)
    M, K, N = 96, 3072, 72
    A = rng.integers(-127, 128, (M, K), dtype=np.int8)
    W = rng.integers(-127, 128, (K, N), dtype=np.int8)
    A[0] = 127
    W[:, 0] = 127                     # the largest accumulation: 3072 * 127^2 < 2^31
    C = np.zeros((M, N), np.int32)
    orc.orc_gemm_i8(P(A), M, K, P(W), N, P(C))
    want = A.astype(np.int64) @ W.astype(np.int64)
    assert np.array_equal(C.astype(np.int64), want)
    assert C[0, 0] == 3072 * 127 * 127


@pytest.mark.parametrize("M,N", [(40, 1152), (7, 64)])
def test_dequantise_matches_reference_bitwise(orc, ref, M, N):
    rng = np.random.default_rng(M + N)
    C = aligned_empty((M, N), np.int32)
    C[:] = rng.integers(-2**30, 2**30, (M, N), dtype=np.int32)
    C[0, :8] = [2**24 + 1, -(2**24 + 3), 0, 1, -1, 2**31 - 1, -2**31, 12345]
    sa = rng.uniform(1e-4, 1e-1, M).astype(np.float32)
    ws = rng.uniform(1e-4, 1e-2, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    o0, o1 = np.zeros((M, N), np.float32), np.zeros((M, N), np.float32)
    orc.orc_dequantise_c(P(C), M, N, P(sa), P(ws), P(bias), P(o0))
    assert ref.ref_dequantise_c(P(C), M, N, P(sa), P(ws), P(bias), P(o1)) == 0
    assert np.array_equal(o0.view(np.uint32), o1.view(np.uint32))


def test_int8_stack_tracks_the_fp32_stack(orc):
    """The int8 BERT stack over the packer's quantisation of the same weights
    stays within int8 noise of the host fp32 stack (a property, not a pin:
    the pins are the three functions above)."""
    m = synth.make_model("minilm", layers=2, ln_random=True)
    ids, am, _ = synth.make_text_inputs(m, batch=3, seq=64)
    B, S, d = 3, 64, m["hidden"]
    rng = np.random.default_rng(3)
    keep, ops = [], OrcI8()
    m_deq = dict(m)
    for i, (w, K) in enumerate([("w_qkv", d), ("w_ao", d), ("w_up", d), ("w_down", m["ffn"])]):
        asm = rng.uniform(0.5, 2.0, (m["layers"], K)).astype(np.float32)
        qs, ss = zip(*[quantise_weights(m[w][l], asm[l]) for l in range(m["layers"])])
        q = np.ascontiguousarray(np.stack(qs))
        s = np.ascontiguousarray(np.stack(ss))
        ias = np.ascontiguousarray((np.float32(1.0) / asm).astype(np.float32))
        keep += [q, s, ias]
        ops.wq[i], ops.wscale[i], ops.ias[i] = q.ctypes.data, s.ctypes.data, ias.ctypes.data
        m_deq[w] = (q.astype(np.float32) * s[:, None, :] / asm[:, :, None]).astype(np.float32)
    emb = np.empty((B * S, d), np.float32)
    cm = np.empty((B, S), np.float32)
    orc.orc_embed_sum(P(ids), P(am), B, S, d, P(m["word"]), P(m["pos"]), P(m["type"]),
                      P(emb), P(cm))
    x8, x32 = emb.copy(), emb.copy()
    orc.orc_bert_run_i8(encoder_struct(m, keep), ops, P(x8), P(cm), B, S, -1)
    orc.orc_bert_run(encoder_struct(m_deq, keep), P(x32), P(cm), B, S, -1)
    rows = am.reshape(-1) > 0
    a, b = x8[rows].astype(np.float64), x32[rows].astype(np.float64)
    cos = np.sum(a * b, 1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1))
    assert cos.min() > 0.99, cos.min()
