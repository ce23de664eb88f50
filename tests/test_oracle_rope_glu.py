"""The oracle's RoPE and gated-FFN restatements (the nomic / gte BERT archs),
pinned without retyping them: the table builder against the reference's own
gemma_rope_tables (oracle/_ref), the rotation against complex multiplication
and RoPE's relative-position property, SiLU against the reference's own
exp2_avx2 and both activations against their closed forms, and the whole
RoPE + gated stack against an fp64 restatement. CPU only."""
import math

import numpy as np
import pytest

from mxenc import synth
from orc import P, encoder_struct
from test_oracle_encoder import attention64, ln64


def _tables(orc, S, hd, theta, inv=None):
    c = np.empty((S, hd), np.float32)
    s = np.empty((S, hd), np.float32)
    inv = None if inv is None else np.ascontiguousarray(inv, np.float32)
    orc.orc_rope_tables(S, hd, theta, None if inv is None else P(inv), P(c), P(s))
    return c, s


@pytest.mark.parametrize("S,hd,theta", [(512, 64, 1000.0), (2048, 32, 10000.0), (7, 128, 1e6)])
def test_rope_tables_are_the_references(orc, ref, S, hd, theta):
    c0, s0 = _tables(orc, S, hd, theta)
    c1, s1 = np.empty_like(c0), np.empty_like(s0)
    ref.ref_gemma_rope_tables(S, hd, theta, P(c1), P(s1))
    assert np.array_equal(c0.view(np.uint32), c1.view(np.uint32))
    assert np.array_equal(s0.view(np.uint32), s1.view(np.uint32))


def test_rope_tables_from_frequencies(orc):
    """gte's explicit frequency set: the half duplicated, position 0 the
    identity, and cos^2 + sin^2 = 1 to fp32 rounding."""
    m = synth.make_model("gte", layers=1)
    hd = m["head_dim"]
    c, s = _tables(orc, 512, hd, 0.0, m["rope_inv_freq"])
    assert np.array_equal(c[:, :hd // 2], c[:, hd // 2:])
    assert np.array_equal(s[:, :hd // 2], s[:, hd // 2:])
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    assert np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1).max() < 3e-7
    # a slower frequency turns less at the same position
    ang = np.arctan2(s[100, :hd // 2].astype(np.float64), c[100, :hd // 2].astype(np.float64))
    assert abs(ang[-1]) < abs(ang[1])


def test_rope_rotation_is_complex_multiplication(orc):
    rng = np.random.default_rng(0)
    B, S, H, hd = 2, 9, 3, 16
    d, half = H * hd, hd // 2
    c, s = _tables(orc, S, hd, 100.0)
    qkv = rng.standard_normal((B * S, 3 * d)).astype(np.float32)
    got = qkv.copy()
    orc.orc_rope_qkv(P(got), B * S, S, H, hd, P(c), P(s))
    assert np.array_equal(got[:, 2 * d:], qkv[:, 2 * d:])          # V is never rotated
    pos = np.arange(B * S) % S
    for part in (0, 1):                                              # Q, then K
        for h in range(H):
            cols = part * d + h * hd
            z = qkv[:, cols:cols + half].astype(np.float64) + \
                1j * qkv[:, cols + half:cols + hd].astype(np.float64)
            rot = (c[pos, :half].astype(np.float64) + 1j * s[pos, :half].astype(np.float64))
            w = z * rot
            assert np.abs(got[:, cols:cols + half] - w.real).max() < 1e-5
            assert np.abs(got[:, cols + half:cols + hd] - w.imag).max() < 1e-5


def test_rope_depends_only_on_relative_position(orc):
    """q at position p against k at position t scores the same as at p + D,
    t + D: the property RoPE exists for (a wrong pairing, sign or index
    breaks it)."""
    rng = np.random.default_rng(1)
    S, H, hd = 64, 1, 32
    d = H * hd
    c, s = _tables(orc, S, hd, 1000.0)
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal(hd).astype(np.float32)
    qkv = np.zeros((S, 3 * d), np.float32)
    qkv[:, :d] = q
    qkv[:, d:2 * d] = k
    orc.orc_rope_qkv(P(qkv), S, S, H, hd, P(c), P(s))
    score = qkv[:, :d].astype(np.float64) @ qkv[:, d:2 * d].astype(np.float64).T
    for delta in (1, 5, 20):
        a = np.diagonal(score, offset=delta)          # q at p, k at p + delta
        assert np.abs(a - a[0]).max() < 1e-4 * max(1.0, abs(a[0]))
    assert abs(score[0, 0] - float(q.astype(np.float64) @ k)) < 1e-5


def test_glu_silu_is_the_references_exp2(orc, ref):
    rng = np.random.default_rng(2)
    rows, f = 37, 64
    up = (rng.standard_normal((rows, 2 * f)) * 6).astype(np.float32)
    up[0, f:f + 4] = [0.0, -0.0, 80.0, -80.0]
    got = np.empty((rows, f), np.float32)
    orc.orc_glu(P(up), rows, f, 1, P(got))
    lo, hi = up[:, :f], np.ascontiguousarray(up[:, f:])
    a = np.maximum((np.float32(0) - hi) * np.float32(1.4426950408889634), np.float32(-120))
    e = np.empty_like(a)
    ref.ref_exp2_avx2(P(np.ascontiguousarray(a)), P(e), a.size)
    want = lo * (hi / (np.float32(1) + e))
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    # and it is SiLU: lo * hi * sigmoid(hi)
    silu = lo.astype(np.float64) * hi / (1 + np.exp(-hi.astype(np.float64)))
    assert np.abs(got - silu).max() < 1e-5 * np.abs(silu).max()


def test_glu_gelu_erf_closed_form(orc):
    rng = np.random.default_rng(3)
    rows, f = 11, 40
    up = (rng.standard_normal((rows, 2 * f)) * 3).astype(np.float32)
    got = np.empty((rows, f), np.float32)
    orc.orc_glu(P(up), rows, f, 2, P(got))
    lo, hi = up[:, :f].astype(np.float64), up[:, f:].astype(np.float64)
    want = lo * 0.5 * hi * (1 + np.vectorize(math.erf)(hi / math.sqrt(2)))
    assert np.abs(got - want).max() < 1e-6 * np.abs(want).max()
    # the gate is the second half: swapping the halves is a different function
    assert np.abs(got - up[:, f:] * 0.5 * up[:, :f] *
                  (1 + np.vectorize(math.erf)(up[:, :f] / math.sqrt(2)))).max() > 1e-2


def rope64(qkv, S, H, hd, c, s):
    d, half = H * hd, hd // 2
    out = qkv.copy()
    pos = np.arange(qkv.shape[0]) % S
    cc, ss = c[pos].astype(np.float64), s[pos].astype(np.float64)
    for part in (0, 1):
        for h in range(H):
            b = part * d + h * hd
            x1, x2 = qkv[:, b:b + half], qkv[:, b + half:b + hd]
            out[:, b:b + half] = x1 * cc[:, :half] - x2 * ss[:, :half]
            out[:, b + half:b + hd] = x2 * cc[:, :half] + x1 * ss[:, :half]
    return out


def glu64(up, f, act):
    lo, hi = up[:, :f], up[:, f:]
    if act == 1:
        return lo * hi / (1 + np.exp(-hi))
    return lo * 0.5 * hi * (1 + np.vectorize(math.erf)(hi / math.sqrt(2)))


@pytest.mark.parametrize("name", ["nomic", "gte"])
def test_rope_gated_bert_run_vs_fp64(orc, name):
    m = synth.make_model(name, layers=2, hidden=64, heads=2, head_dim=32, ffn=128,
                         ln_random=True)
    B, S, H, hd, f = 2, 24, 2, 32, 128
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((B * S, 64)) * 0.5).astype(np.float32)
    mask = np.zeros((B, S), np.float32)
    mask[1, 17:] = -1e30
    keep = []
    enc = encoder_struct(m, keep)
    y = x.copy()
    orc.orc_bert_run(enc, P(y), P(mask), B, S, -1)
    c, s = _tables(orc, S, hd, m["rope_theta"], m.get("rope_inv_freq"))
    h = ln64(x.astype(np.float64), m["emb_ln_g"], m["emb_ln_b"], 1e-12)
    for l in range(2):
        qkv = rope64(h @ m["w_qkv"][l] + m["b_qkv"][l], S, H, hd, c, s)
        ctx = attention64(qkv, B, S, H, hd, mask, 1.0)
        h = ln64(h + ctx @ m["w_ao"][l] + m["b_ao"][l], m["ln1_g"][l], m["ln1_b"][l], 1e-12)
        g = glu64(h @ m["w_up"][l] + m["b_up"][l], f, m["gated"])
        h = ln64(h + g @ m["w_down"][l] + m["b_down"][l], m["ln2_g"][l], m["ln2_b"][l], 1e-12)
    assert np.max(np.abs(y - h)) < 5e-5
