"""Seeded synthetic encoders and inputs for the five workload geometries.

The weights follow the reference packer's conventions
(tools/pack/pack_npue.py:2630,2747; common/host_b.hpp:68-73):
  * GEMM operands are [K, N] row-major, fused QKV along N as Q|K|V, head h at
    columns h*head_dim of each block;
  * 1/sqrt(head_dim) is folded into Q's weight columns and Q's bias before the
    weight is rounded to bf16 (round-to-nearest-even), so attention runs at
    scale 1;
  * biases, LayerNorm parameters and embedding tables stay fp32.
Weights are N(0, 0.02). LayerNorm gamma = 1, beta = 0 unless `ln_random`
(the tests randomise them so a dropped gamma or beta is visible).
"""
import math

import numpy as np

SEED = 20260926

CONFIGS = {
    # all-MiniLM-L6-v2 geometry, mean pooling.
    "minilm": dict(kind="bert", layers=6, hidden=384, heads=12, head_dim=32, ffn=1536,
                   vocab=30522, max_pos=512, batch=32, seq=128, len_lo=16, len_hi=128,
                   cls_pool=False, sep=True),
    # bge-base geometry, CLS pooling.
    "bge_base": dict(kind="bert", layers=12, hidden=768, heads=12, head_dim=64, ffn=3072,
                     vocab=30522, max_pos=512, batch=64, seq=512, len_lo=64, len_hi=512,
                     cls_pool=True, sep=False),
    # bge-large geometry, CLS pooling, every sequence full length.
    "bge_large": dict(kind="bert", layers=24, hidden=1024, heads=16, head_dim=64, ffn=4096,
                      vocab=30522, max_pos=512, batch=128, seq=512, len_lo=512, len_hi=512,
                      cls_pool=True, sep=False),
    # The RoPE / gated-FFN BERT archs at bge-base geometry (no benchmark
    # workload names them; they exercise the nomic and gte encoder paths):
    # nomic-embed-text (SwiGLU, RoPE base 1000, mean pooling) and
    # gte-multilingual-base (exact-erf GeGLU, RoPE from an explicit frequency
    # set, CLS pooling).
    "nomic": dict(kind="bert", layers=12, hidden=768, heads=12, head_dim=64, ffn=3072,
                  vocab=30522, max_pos=512, batch=64, seq=512, len_lo=64, len_hi=512,
                  cls_pool=False, sep=True, gated=1, rope=True, rope_theta=1000.0),
    "gte": dict(kind="bert", layers=12, hidden=768, heads=12, head_dim=64, ffn=3072,
                vocab=30522, max_pos=512, batch=64, seq=512, len_lo=64, len_hi=512,
                cls_pool=True, sep=True, gated=2, rope=True, rope_theta=0.0),
    # ViT-base/16 at 224x224: 196 patches + CLS = 197 tokens, pre-LN.
    "vit_base": dict(kind="vit", layers=12, hidden=768, heads=12, head_dim=64, ffn=3072,
                     batch=256, image=224, patch=16, labels=1000, eps=1e-12),
    # Whisper-large-v3 encoder: 128 mels x 3000 frames -> 1500 positions, pre-LN.
    "whisper_enc": dict(kind="whisper", layers=32, hidden=1280, heads=20, head_dim=64,
                        ffn=5120, batch=8, mels=128, frames=3000, eps=1e-5),
}


def _bf16(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32)
    return r.view(np.float32)


def _normal(rng, shape, std=0.02):
    return (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std))


def make_layers(rng, L, d, heads, hd, f, ln_random=False, gated=0):
    """Per-layer tensors, contiguous over layers. gated: FFN-up is [d, 2f]
    (up half, then gate half) with a [2f] bias."""
    m = {}
    scale = np.float32(1.0 / math.sqrt(hd))
    w_qkv = _normal(rng, (L, d, 3 * d))
    b_qkv = _normal(rng, (L, 3 * d))
    w_qkv[:, :, :d] *= scale
    b_qkv[:, :d] *= scale
    m["w_qkv"] = _bf16(w_qkv)
    m["b_qkv"] = b_qkv
    m["w_ao"] = _bf16(_normal(rng, (L, d, d)))
    m["b_ao"] = _normal(rng, (L, d))
    fu = 2 * f if gated else f
    m["w_up"] = _bf16(_normal(rng, (L, d, fu)))
    m["b_up"] = _normal(rng, (L, fu))
    m["w_down"] = _bf16(_normal(rng, (L, f, d)))
    m["b_down"] = _normal(rng, (L, d))
    for n in ("ln1", "ln2"):
        if ln_random:
            m[n + "_g"] = (1.0 + _normal(rng, (L, d), 0.1)).astype(np.float32)
            m[n + "_b"] = _normal(rng, (L, d), 0.05)
        else:
            m[n + "_g"] = np.ones((L, d), np.float32)
            m[n + "_b"] = np.zeros((L, d), np.float32)
    return m


def make_model(name, seed=SEED, layers=None, ln_random=False, **over):
    """A synthetic model of configuration `name`, optionally with fewer layers
    or other overrides (hidden, heads, ...) for small tests."""
    cfg = dict(CONFIGS[name])
    cfg.update(over)
    if layers is not None:
        cfg["layers"] = layers
    rng = np.random.default_rng(seed)
    L, d, H, hd, f = cfg["layers"], cfg["hidden"], cfg["heads"], cfg["head_dim"], cfg["ffn"]
    assert H * hd == d
    m = dict(cfg)
    m.update(make_layers(rng, L, d, H, hd, f, ln_random, cfg.get("gated", 0)))
    if cfg.get("rope") and not cfg.get("rope_theta"):
        # gte-multilingual-base's frequency set: 160000^(-j/(hd/2)) / 8^(1/(hd/2))
        half = hd // 2
        j = np.arange(half, dtype=np.float64)
        m["rope_inv_freq"] = (160000.0 ** (-j / half) / 8.0 ** (1.0 / half)).astype(np.float32)
    ln = (lambda n: (1.0 + _normal(rng, (n,), 0.1)).astype(np.float32)) if ln_random else \
        (lambda n: np.ones((n,), np.float32))
    lb = (lambda n: _normal(rng, (n,), 0.05)) if ln_random else \
        (lambda n: np.zeros((n,), np.float32))
    if cfg["kind"] == "bert":
        m["word"] = _normal(rng, (cfg["vocab"], d))
        m["pos"] = _normal(rng, (cfg["max_pos"], d))
        m["type"] = _normal(rng, (2, d))
        m["emb_ln_g"], m["emb_ln_b"] = ln(d), lb(d)
    else:
        m["fin_ln_g"], m["fin_ln_b"] = ln(d), lb(d)
    if cfg["kind"] == "vit":
        pd = 3 * cfg["patch"] ** 2
        n_pos = (cfg["image"] // cfg["patch"]) ** 2 + 1
        m["patch_w"] = _bf16(_normal(rng, (pd, d)))
        m["patch_b"] = _normal(rng, (d,))
        m["cls_token"] = _normal(rng, (d,))
        m["pos"] = _normal(rng, (n_pos, d))
        m["head_w"] = _normal(rng, (d, cfg["labels"]))
        m["head_b"] = _normal(rng, (cfg["labels"],))
        m["seq"] = n_pos
    if cfg["kind"] == "whisper":
        m["conv1_w"] = _normal(rng, (d, cfg["mels"], 3))
        m["conv1_b"] = _normal(rng, (d,))
        m["conv2_w"] = _normal(rng, (d, d, 3))
        m["conv2_b"] = _normal(rng, (d,))
        m["seq"] = cfg["frames"] // 2
        m["pos"] = sinusoids(m["seq"], d)
    return m


def sinusoids(length, channels, max_timescale=10000.0):
    """Whisper's fixed encoder position table: [sin | cos] halves."""
    inc = math.log(max_timescale) / (channels // 2 - 1)
    inv = np.exp(-inc * np.arange(channels // 2, dtype=np.float64))
    t = np.arange(length, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.sin(t), np.cos(t)], axis=1).astype(np.float32)


def make_text_inputs(cfg, seed=SEED + 1, batch=None, seq=None):
    """Token ids and the 1/0 attention mask for a BERT configuration:
    ids U[1000, 30521], [CLS]=101 at 0, [SEP]=102 at len-1 when cfg['sep'],
    valid length U[len_lo, len_hi], id 0 and mask 0 past it."""
    rng = np.random.default_rng(seed)
    B = batch or cfg["batch"]
    S = seq or cfg["seq"]
    lo, hi = min(cfg["len_lo"], S), min(cfg["len_hi"], S)
    lens = rng.integers(lo, hi + 1, size=B)
    ids = rng.integers(1000, 30522, size=(B, S)).astype(np.int32)
    mask = np.zeros((B, S), np.float32)
    for b, n in enumerate(lens):
        ids[b, n:] = 0
        mask[b, :n] = 1.0
        ids[b, 0] = 101
        if cfg.get("sep"):
            ids[b, n - 1] = 102
    return ids, mask, lens


def make_pixels(cfg, seed=SEED + 2, batch=None):
    rng = np.random.default_rng(seed)
    B = batch or cfg["batch"]
    return rng.uniform(-1.0, 1.0, size=(B, 3, cfg["image"], cfg["image"])).astype(np.float32)


def make_mel(cfg, seed=SEED + 3, batch=None):
    rng = np.random.default_rng(seed)
    B = batch or cfg["batch"]
    return rng.standard_normal(size=(B, cfg["mels"], cfg["frames"]), dtype=np.float32)


def quantise_weights(w_kn, asmooth=None):
    """The reference packer's int8 operand scheme (tools/lib/gemm_i8.py:21-90):
    W' = W * asmooth[:, None] (the SmoothQuant fold), per column
    s = max_k |W'| / 127 (1 for an all-zero column), q = rint(W' / s) clipped
    to [-127, 127]. Returns (q int8 [K, N], s fp32 [N])."""
    w = np.asarray(w_kn, np.float32)
    if asmooth is not None:
        w = w * np.asarray(asmooth, np.float32)[:, None]
    s = (np.abs(w).max(axis=0) / np.float32(127.0)).astype(np.float32)
    s = np.where(s > 0, s, np.float32(1.0)).astype(np.float32)
    q = np.rint(w / s[None, :]).clip(-127, 127).astype(np.int8)
    return q, s


def quantise_weights_i4(w_kn, asmooth=None, group=32):
    """The reference packer's int4 operand scheme (tools/lib/gemm_i4.py:23-140):
    W' = W * asmooth[:, None]; the int8 column scale s8 = max_k |W'| / 127
    (1 for an all-zero column), kept as .wscale; per group g of `group` rows
    (0: one group over K) and column, s4 = max |W'| / 7 (1 when zero), the
    nibble t = rint(W' / s4) clipped to [-7, 7], and .gscale = s4 / s8.
    Returns (t int8 [K, N], s8 fp32 [N], gscale fp32 [ceil(K / group), N])."""
    w = np.asarray(w_kn, np.float32)
    if asmooth is not None:
        w = w * np.asarray(asmooth, np.float32)[:, None]
    K, N = w.shape
    g = int(group or K)
    s8 = (np.abs(w).max(axis=0) / np.float32(127.0)).astype(np.float32)
    s8 = np.where(s8 > 0, s8, np.float32(1.0)).astype(np.float32)
    G = -(-K // g)
    padded = np.zeros((G * g, N), np.float32)
    padded[:K] = w
    blocks = padded.reshape(G, g, N)
    s4 = (np.abs(blocks).max(axis=1) / np.float32(7.0)).astype(np.float32)
    s4 = np.where(s4 > 0, s4, np.float32(1.0)).astype(np.float32)
    t = np.rint(blocks / s4[:, None, :]).clip(-7, 7).astype(np.int8).reshape(G * g, N)[:K]
    return np.ascontiguousarray(t), s8, (s4 / s8[None, :]).astype(np.float32)


GEMM_KEYS = ("w_qkv", "w_ao", "w_up", "w_down")


def quantise_model(m, seed=SEED + 7, smooth=(0.5, 2.0)):
    """The int8 operands of a synthetic encoder, as an --int8 pack would carry
    them: per GEMM site a tuple (q [L, K, N] int8, wscale [L, N], asmooth
    [L, K]), the smoothing factors drawn uniform in `smooth` (None: all ones).
    Sites in the order qkv, attn_out, ffn_up, ffn_down."""
    rng = np.random.default_rng(seed)
    out = []
    for key in GEMM_KEYS:
        W = m[key]
        L, K, _ = W.shape
        if smooth is None:
            sm = np.ones((L, K), np.float32)
        else:
            sm = rng.uniform(smooth[0], smooth[1], (L, K)).astype(np.float32)
        qs, ss = zip(*[quantise_weights(W[l], sm[l]) for l in range(L)])
        out.append((np.ascontiguousarray(np.stack(qs)), np.ascontiguousarray(np.stack(ss)),
                    np.ascontiguousarray(sm)))
    return out


def quantise_model_i4(m, group=32, seed=SEED + 7, smooth=(0.5, 2.0)):
    """The int4 operands of a synthetic encoder, as an --int4 pack carries them:
    per GEMM site (t [L, K, N] int8 in [-7, 7], wscale [L, N], gscale
    [L, ceil(K / group), N], asmooth [L, K]); sites as quantise_model."""
    rng = np.random.default_rng(seed)
    out = []
    for key in GEMM_KEYS:
        W = m[key]
        L, K, _ = W.shape
        sm = (np.ones((L, K), np.float32) if smooth is None else
              rng.uniform(smooth[0], smooth[1], (L, K)).astype(np.float32))
        ts, ss, gs = zip(*[quantise_weights_i4(W[l], sm[l], group) for l in range(L)])
        out.append((np.ascontiguousarray(np.stack(ts)), np.ascontiguousarray(np.stack(ss)),
                    np.ascontiguousarray(np.stack(gs)), np.ascontiguousarray(sm)))
    return out
