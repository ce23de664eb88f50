"""The oracle's whole-encoder restatements against fp64 textbook stacks on tiny
shapes: post-LN BERT (BertEncoder::run), pre-LN ViT/Whisper bodies, Whisper's
conv front end, ViT im2col and head. CPU only."""
import math

import numpy as np

from mxenc import synth
from orc import P, encoder_struct

GELU8 = [-7.2340282171e-05, 1.8179518005e-03, -1.7707383379e-02, 8.4577147641e-02,
         -1.9228671834e-01, 9.8431124458e-02, 3.6137852062e-01, -4.9454128936e-01,
         -1.3007010117e-04]


def gelu_poly64(x):
    u = np.minimum(np.abs(x), 4.0)
    p = np.full_like(x, GELU8[0])
    for c in GELU8[1:]:
        p = p * u + c
    return np.maximum(x, 0) + p


def gelu_erf64(x):
    return 0.5 * x * (1 + np.vectorize(math.erf)(x / math.sqrt(2)))


def ln64(x, g, b, eps):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g + b


def attention64(qkv, B, S, H, hd, mask, scale):
    d = H * hd
    out = np.zeros((B * S, d))
    for b in range(B):
        r = slice(b * S, (b + 1) * S)
        for h in range(H):
            q = qkv[r, h * hd:(h + 1) * hd]
            k = qkv[r, d + h * hd:d + (h + 1) * hd]
            v = qkv[r, 2 * d + h * hd:2 * d + (h + 1) * hd]
            s = q @ k.T * scale
            if mask is not None:
                s = s + mask[b]
            e = np.exp(s - s.max(-1, keepdims=True))
            out[r, h * hd:(h + 1) * hd] = (e / e.sum(-1, keepdims=True)) @ v
    return out


def bert64(m, x, mask, B, S):
    d, H, hd = m["hidden"], m["heads"], m["head_dim"]
    x = ln64(x.astype(np.float64), m["emb_ln_g"], m["emb_ln_b"], 1e-12)
    for l in range(m["layers"]):
        qkv = x @ m["w_qkv"][l] + m["b_qkv"][l]
        ctx = attention64(qkv, B, S, H, hd, mask, 1.0)
        x = ln64(x + ctx @ m["w_ao"][l] + m["b_ao"][l], m["ln1_g"][l], m["ln1_b"][l], 1e-12)
        up = gelu_poly64(x @ m["w_up"][l] + m["b_up"][l])
        x = ln64(x + up @ m["w_down"][l] + m["b_down"][l], m["ln2_g"][l], m["ln2_b"][l], 1e-12)
    return x


def preln64(m, x, B, S, eps, scale):
    d, H, hd = m["hidden"], m["heads"], m["head_dim"]
    x = x.astype(np.float64)
    for l in range(m["layers"]):
        n = ln64(x, m["ln1_g"][l], m["ln1_b"][l], eps)
        qkv = n @ m["w_qkv"][l] + m["b_qkv"][l]
        x = x + attention64(qkv, B, S, H, hd, None, scale) @ m["w_ao"][l] + m["b_ao"][l]
        n = ln64(x, m["ln2_g"][l], m["ln2_b"][l], eps)
        x = x + gelu_erf64(n @ m["w_up"][l] + m["b_up"][l]) @ m["w_down"][l] + m["b_down"][l]
    return ln64(x, m["fin_ln_g"], m["fin_ln_b"], eps)


def tiny_bert():
    return synth.make_model("minilm", layers=2, hidden=64, heads=2, head_dim=32, ffn=128,
                            ln_random=True)


def test_bert_run_vs_fp64(orc):
    m = tiny_bert()
    B, S = 3, 16
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((B * S, 64)) * 0.5).astype(np.float32)
    mask = np.zeros((B, S), np.float32)
    mask[1, 9:] = -1e30
    mask[2, 3:] = -1e30
    keep = []
    enc = encoder_struct(m, keep)
    y = x.copy()
    orc.orc_bert_run(enc, P(y), P(mask), B, S, -1)
    want = bert64(m, x, mask, B, S)
    assert np.max(np.abs(y - want)) < 5e-5
    # one layer only: the first-layer result differs from the two-layer one
    y1 = x.copy()
    orc.orc_bert_run(enc, P(y1), P(mask), B, S, 1)
    m1 = dict(m, layers=1)
    assert np.max(np.abs(y1 - bert64(m1, x, mask, B, S))) < 5e-5


def test_bert_sequences_are_independent(orc):
    """A sequence's output does not depend on the other rows of the batch --
    what lets parity at full batch be checked on a subset of sequences."""
    m = tiny_bert()
    B, S = 4, 16
    rng = np.random.default_rng(1)
    x = rng.standard_normal((B * S, 64)).astype(np.float32)
    mask = np.zeros((B, S), np.float32)
    mask[2, 5:] = -1e30
    keep = []
    enc = encoder_struct(m, keep)
    y = x.copy()
    orc.orc_bert_run(enc, P(y), P(mask), B, S, -1)
    sub = x[2 * S:3 * S].copy()
    orc.orc_bert_run(enc, P(sub), P(mask[2:3].copy()), 1, S, -1)
    assert np.array_equal(sub, y[2 * S:3 * S])


def test_preln_run_vs_fp64(orc):
    m = synth.make_model("vit_base", layers=2, hidden=64, heads=2, head_dim=32, ffn=128,
                         ln_random=True, image=32, patch=16, labels=10)
    B, S = 2, 13  # odd length, like ViT's 197
    rng = np.random.default_rng(2)
    x = rng.standard_normal((B * S, 64)).astype(np.float32)
    keep = []
    enc = encoder_struct(m, keep)
    for eps, scale in ((1e-12, 1.0), (1e-5, 0.125)):
        y = x.copy()
        orc.orc_preln_run(enc, P(y), B, S, eps, scale, -1)
        assert np.max(np.abs(y - preln64(m, x, B, S, eps, scale))) < 5e-5


def test_conv_front_end_vs_fp64(orc):
    rng = np.random.default_rng(3)
    M, T, d = 5, 20, 8
    mel = rng.standard_normal((M, T)).astype(np.float32)
    w1 = rng.standard_normal((d, M, 3)).astype(np.float32) * 0.3
    b1 = rng.standard_normal(d).astype(np.float32) * 0.1
    w2 = rng.standard_normal((d, d, 3)).astype(np.float32) * 0.3
    b2 = rng.standard_normal(d).astype(np.float32) * 0.1
    out = np.empty((T // 2, d), np.float32)
    orc.orc_conv_front_end(P(mel), M, T, P(w1), P(b1), P(w2), P(b2), d, P(out))

    def conv(x, w, b, stride):
        cin, tin = x.shape
        xp = np.pad(x.astype(np.float64), ((0, 0), (1, 1)))
        tout = (tin + 2 - 3) // stride + 1
        y = np.zeros((w.shape[0], tout))
        for t in range(tout):
            y[:, t] = np.einsum("ock,ck->o", w, xp[:, t * stride:t * stride + 3]) + b
        return gelu_erf64(y)

    want = conv(conv(mel, w1, b1, 1), w2, b2, 2).T
    assert np.max(np.abs(out - want)) < 1e-5


def test_vit_patches_and_head(orc):
    rng = np.random.default_rng(4)
    img, p = 32, 16
    px = rng.standard_normal((3, img, img)).astype(np.float32)
    rows = np.empty(((img // p) ** 2, 3 * p * p), np.float32)
    orc.orc_vit_patches(P(px), img, p, P(rows))
    want = px.reshape(3, img // p, p, img // p, p).transpose(1, 3, 0, 2, 4).reshape(-1, 3 * p * p)
    assert np.array_equal(rows, want)
    d, nl = 24, 7
    head = rng.standard_normal((d, nl)).astype(np.float32)
    bias = rng.standard_normal(nl).astype(np.float32)
    cls = rng.standard_normal(d).astype(np.float32)
    lg = np.empty(nl, np.float32)
    orc.orc_head_matvec(P(head), P(bias), P(cls), d, nl, P(lg))
    assert np.max(np.abs(lg - (cls.astype(np.float64) @ head + bias))) < 1e-6
