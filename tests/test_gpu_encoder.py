"""The whole encoder stack on the GPU against the oracle's host path, through
the C ABI: pooled, L2-normalised embeddings must reach cosine >= 0.9999 per
sequence. Sequences are independent (test_oracle_encoder pins that on the
host), so at full batch the oracle checks a subset of the batch's sequences
exactly."""
import numpy as np
import pytest

import mxenc
from mxenc import synth
from orc import P, encoder_struct

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999


@pytest.fixture(scope="module")
def ctx():
    c = mxenc.Context(0)
    yield c
    c.close()


def cosines(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return np.sum(a * b, -1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1))


def oracle_embed(orc, m, ids, am):
    """EmbedService::chunk on the host: embedding sum, mask, run, pool."""
    B, S = ids.shape
    d = m["hidden"]
    emb = np.empty((B * S, d), np.float32)
    cm = np.empty((B, S), np.float32)
    orc.orc_embed_sum(P(ids), P(am), B, S, d, P(m["word"]), P(m["pos"]), P(m["type"]), P(emb),
                      P(cm))
    keep = []
    orc.orc_bert_run(encoder_struct(m, keep), P(emb), P(cm), B, S, -1)
    out = np.empty((B, d), np.float32)
    assert orc.orc_pool_rows(P(emb), P(am), B, S, d, int(m["cls_pool"]), 1, P(out)) == 0
    return out, emb


def gpu_embed(ctx, enc, ids, am):
    B, S = ids.shape
    d_ids, d_am = ctx.put(ids), ctx.put(am)
    out = ctx.empty((B, enc.desc.hidden), np.float32)
    enc.embed(d_ids, d_am, B, S, out)
    return out.host()


def test_minilm_full_config(ctx, orc):
    """all-MiniLM-L6-v2 geometry, batch 32 x seq 128, mean pooling, whole batch
    checked against the host path."""
    m = synth.make_model("minilm", ln_random=True)
    ids, am, lens = synth.make_text_inputs(m)
    want, _ = oracle_embed(orc, m, ids, am)
    enc = mxenc.Encoder(ctx, m)
    got = gpu_embed(ctx, enc, ids, am)
    cos = cosines(got, want)
    assert np.min(cos) >= COS_MIN, np.min(cos)
    # every output row is unit length (L2 in double on both sides)
    assert np.max(np.abs(np.linalg.norm(got, axis=1) - 1)) < 1e-6
    enc.close()


def test_bge_base_full_batch_every_sequence_checked(ctx, orc):
    """bge-base geometry at its full shape (batch 64 x seq 512, 12 layers, CLS
    pooling), the benchmark's own batch, on the GPU; every one of the 64
    sequences rerun on the host path (in chunks of 16: sequences are
    independent, which test_oracle_encoder pins on the host), cosine >= 0.9999
    each."""
    import os
    m = synth.make_model("bge_base")
    ids, am, lens = synth.make_text_inputs(m)
    enc = mxenc.Encoder(ctx, m)
    got = gpu_embed(ctx, enc, ids, am)
    enc.close()
    cpus = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else 8
    orc.orc_set_threads(max(1, min(16, cpus)))
    want = np.empty_like(got)
    for lo in range(0, ids.shape[0], 16):
        sl = slice(lo, lo + 16)
        want[sl], _ = oracle_embed(orc, m, np.ascontiguousarray(ids[sl]),
                                   np.ascontiguousarray(am[sl]))
        print(f"bge-base oracle: sequences {lo}..{lo + 15} done", flush=True)
    cos = cosines(got, want)
    print(f"bge-base 64 sequences: min cos {np.min(cos):.8f}, 1 - cos max {1 - np.min(cos):.2e}")
    assert np.min(cos) >= COS_MIN, cos


def test_streams_agree_bitwise(ctx):
    """Two lanes (streams) given the same batch produce identical bits, the
    reference's --pipeline lane agreement (run_execute.hpp:547-565)."""
    m = synth.make_model("minilm", layers=2)
    ids, am, _ = synth.make_text_inputs(m, batch=8)
    enc = mxenc.Encoder(ctx, m)
    a = gpu_embed(ctx, enc, ids, am)
    ctx2 = mxenc.Context(0)
    enc2 = mxenc.Encoder(ctx2, m)
    b = gpu_embed(ctx2, enc2, ids, am)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    enc2.close()
    ctx2.close()
    enc.close()


@pytest.mark.parametrize("S,valid", [(512, 512), (72, 41), (8, 1)])
def test_bge_base_single_sequence(ctx, orc, S, valid):
    """One sequence (batch 1) at the full length, with padding at a length
    that fills no tile, and of a single token: a one-row-tile GEMM, a partly
    filled key tile, attention over one key. (The host path's sequence length
    is a multiple of 8, as the reference's is.)"""
    m = synth.make_model("bge_base", layers=2, ln_random=True)
    ids, am, _ = synth.make_text_inputs(m, batch=1, seq=S)
    am[:] = 0.0
    am[0, :valid] = 1.0
    ids[0, valid:] = 0
    enc = mxenc.Encoder(ctx, m)
    got = gpu_embed(ctx, enc, ids, am)
    enc.close()
    want, _ = oracle_embed(orc, m, ids, am)
    cos = cosines(got, want)
    assert np.min(cos) >= COS_MIN, cos


def _preln_case(ctx, orc, name, B, layers, eps):
    m = synth.make_model(name, layers=layers, ln_random=True)
    S, d = m["seq"], m["hidden"]
    rng = np.random.default_rng(7)
    x = rng.standard_normal((B * S, d)).astype(np.float32)
    want = x.copy()
    keep = []
    orc.orc_preln_run(encoder_struct(m, keep), P(want), B, S, eps, 1.0, -1)
    enc = mxenc.Encoder(ctx, m)
    dx = ctx.put(x)
    enc.run(dx, None, None, B, S)
    got = dx.host()
    cos = cosines(got, want)
    assert np.min(cos) >= COS_MIN, np.min(cos)
    enc.close()


def test_vit_body_197_tokens(ctx, orc):
    """ViT-base/16 body: 12 pre-LN layers over 197 positions (odd length, no
    mask), exact-erf GELU, final LayerNorm; 2 images."""
    _preln_case(ctx, orc, "vit_base", 2, 12, 1e-12)


def test_whisper_body_1500_positions(ctx, orc):
    """Whisper-large-v3 encoder body at its width (d 1280, 20 heads, FFN 5120)
    over 1500 positions, unmasked, eps 1e-5; 2 of its 32 layers."""
    _preln_case(ctx, orc, "whisper_enc", 1, 2, 1e-5)


def test_partial_placement_refused(ctx):
    m = synth.make_model("minilm", layers=1)
    enc = mxenc.Encoder(ctx, m)
    L = mxenc.lib()
    try:
        assert L.mx_ops_parse(b"gemm,attn") == 0
        x = ctx.empty((128, 384), np.float32)
        with pytest.raises(mxenc.MxError, match="softm, layn, gelu"):
            enc.run(x, None, None, 1, 128)
        assert L.mx_ops_parse(b"gemm,attn,softm,layn,gelu") == 0
        enc.run(x, None, None, 1, 128)
    finally:
        L.mx_ops_parse(b"")
        enc.close()


def test_bge_large_full_batch_subset_checked(ctx, orc):
    """bge-large geometry at its full shape (batch 128 x seq 512, 24 layers,
    d 1024, 16 heads, every sequence full length): the whole batch on the GPU,
    nine sequences spread over it (every 16th and the last) rerun on the host
    path."""
    m = synth.make_model("bge_large")
    ids, am, _ = synth.make_text_inputs(m)
    enc = mxenc.Encoder(ctx, m)
    got = gpu_embed(ctx, enc, ids, am)
    enc.close()
    assert np.all(np.isfinite(got))
    pick = list(range(0, ids.shape[0], 16)) + [ids.shape[0] - 1]
    want, _ = oracle_embed(orc, m, np.ascontiguousarray(ids[pick]), np.ascontiguousarray(am[pick]))
    cos = cosines(got[pick], want)
    assert np.min(cos) >= COS_MIN, cos


def oracle_vit(orc, m, px):
    """VitEncoder::run + head_matvec on the host: im2col, patch GEMM + bias,
    [CLS; patches] + positions, pre-LN layers + final LN, head on the CLS row."""
    B, p, img, d = px.shape[0], m["patch"], m["image"], m["hidden"]
    npch, pd, labels = (img // p) ** 2, 3 * p * p, m["labels"]
    rows = np.empty((B * npch, pd), np.float32)
    for b in range(B):
        one = np.ascontiguousarray(px[b])
        blk = np.empty((npch, pd), np.float32)
        orc.orc_vit_patches(P(one), img, p, P(blk))
        rows[b * npch:(b + 1) * npch] = blk
    patch = np.empty((B * npch, d), np.float32)
    orc.orc_gemm_nt(P(rows), B * npch, P(m["patch_w"]), pd, d, P(m["patch_b"]), P(patch))
    S = npch + 1
    x = np.empty((B * S, d), np.float32)
    for b in range(B):
        x[b * S] = m["cls_token"]
        x[b * S + 1:(b + 1) * S] = patch[b * npch:(b + 1) * npch]
    x += np.tile(m["pos"], (B, 1))
    keep = []
    orc.orc_preln_run(encoder_struct(m, keep), P(x), B, S, 1e-12, 1.0, -1)
    logits = np.empty((B, labels), np.float32)
    for b in range(B):
        cls = np.ascontiguousarray(x[b * S])
        lg = np.empty(labels, np.float32)
        orc.orc_head_matvec(P(m["head_w"]), P(m["head_b"]), P(cls), d, labels, P(lg))
        logits[b] = lg
    return logits, x


def test_vit_cls_pruning_is_bitwise(ctx):
    """Without a hidden state to return, mx_encoder_vit runs the last layer's
    attention for the CLS query only and its attention-out, FFN and the final
    LayerNorm over the CLS rows (the rows the head reads): the logits equal
    those of the unpruned stack, and of a call that asks for the hidden state,
    bit for bit."""
    m = synth.make_model("vit_base", layers=2, ln_random=True)
    B = 8
    px = synth.make_pixels(m, batch=B)
    enc = mxenc.Encoder(ctx, m)
    d_px = ctx.put(px)
    out = []
    for prune, with_hidden in ((True, False), (False, False), (True, True)):
        enc.set_cls_pruning(prune)
        logits = ctx.empty((B, m["labels"]), np.float32)
        hid = ctx.empty((B * m["seq"], m["hidden"]), np.float32) if with_hidden else None
        enc.vit(d_px, B, logits, hid)
        out.append(logits.host())
    enc.set_cls_pruning(True)
    enc.close()
    assert np.all(np.isfinite(out[0]))
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
    assert np.array_equal(out[0].view(np.uint32), out[2].view(np.uint32))


def test_vit_and_whisper_lane_clones_are_bitwise_their_parent(ctx):
    """A lane clone (mx_encoder_clone) of a ViT or a Whisper encoder, run on a
    stream of its own, gives its parent's logits / hidden state bit for bit:
    the clone borrows the parent's weights and front-end tensors and has its
    own workspace."""
    lane_ctx = mxenc.Context(0)
    for name, B in (("vit_base", 4), ("whisper_enc", 1)):
        m = synth.make_model(name, layers=2, ln_random=True)
        enc = mxenc.Encoder(ctx, m)
        lane = enc.clone(lane_ctx)
        if name == "vit_base":
            x = synth.make_pixels(m, batch=B)
            shape = (B, m["labels"])
        else:
            x = synth.make_mel(m, batch=B)
            shape = (B * m["seq"], m["hidden"])
        got = []
        for e, c in ((enc, ctx), (lane, lane_ctx)):
            out = c.empty(shape, np.float32)
            if name == "vit_base":
                e.vit(c.put(x), B, out)
            else:
                e.whisper(c.put(x), B, out)
            got.append(out.host())
        lane.close()
        enc.close()
        assert np.all(np.isfinite(got[0])), name
        assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32)), name
    lane_ctx.close()


def test_vit_full_config(ctx, orc):
    """ViT-B/16 at 224x224, the configuration's batch of 256 images: patch
    embedding, CLS + positions, 12 pre-LN layers over 197 tokens, final LN and
    the 1000-way head, all on the GPU; every eighth image and the last (33)
    rerun on the host path (hidden state per token and the logits)."""
    m = synth.make_model("vit_base", ln_random=True)
    B, d, S = m["batch"], m["hidden"], m["seq"]
    px = synth.make_pixels(m)
    enc = mxenc.Encoder(ctx, m)
    d_px = ctx.put(px)
    logits = ctx.empty((B, m["labels"]), np.float32)
    hid = ctx.empty((B * S, d), np.float32)
    enc.vit(d_px, B, logits, hid)
    lg, h = logits.host(), hid.host()
    enc.close()
    assert np.all(np.isfinite(lg)) and np.all(np.isfinite(h))
    pick = list(range(0, B, 8)) + [B - 1]
    want_lg, want_x = oracle_vit(orc, m, np.ascontiguousarray(px[pick]))
    for i, b in enumerate(pick):
        cos = cosines(h[b * S:(b + 1) * S], want_x[i * S:(i + 1) * S])
        assert np.min(cos) >= COS_MIN, (b, np.min(cos))
        err = np.max(np.abs(lg[b] - want_lg[i])) / np.max(np.abs(want_lg[i]))
        assert err < 1e-2, (b, err)


def oracle_whisper(orc, m, mel):
    B, T, d = mel.shape[0], m["frames"], m["hidden"]
    S = T // 2
    x = np.empty((B * S, d), np.float32)
    for b in range(B):
        out = np.empty((S, d), np.float32)
        orc.orc_conv_front_end(P(np.ascontiguousarray(mel[b])), m["mels"], T, P(m["conv1_w"]),
                               P(m["conv1_b"]), P(m["conv2_w"]), P(m["conv2_b"]), d, P(out))
        x[b * S:(b + 1) * S] = out + m["pos"]
    keep = []
    orc.orc_preln_run(encoder_struct(m, keep), P(x), B, S, 1e-5, 1.0, -1)
    return x


def test_whisper_full_config(ctx, orc):
    """Whisper-large-v3 encoder geometry, the configuration's 8 x 128 mels x
    3000 frames: conv1 + GELU, conv2 (stride 2) + GELU, positions, 32 pre-LN
    layers over 1500 positions (unmasked) and the final LN on the GPU; the
    first and last samples rerun on the host path, every one of their 1500
    rows checked."""
    m = synth.make_model("whisper_enc", ln_random=True)
    B, d, S = m["batch"], m["hidden"], m["seq"]
    mel = synth.make_mel(m)
    enc = mxenc.Encoder(ctx, m)
    d_mel = ctx.put(mel)
    hid = ctx.empty((B * S, d), np.float32)
    enc.whisper(d_mel, B, hid)
    h = hid.host()
    enc.close()
    assert np.all(np.isfinite(h))
    pick = [0, B - 1]
    want = oracle_whisper(orc, m, np.ascontiguousarray(mel[pick]))
    for i, b in enumerate(pick):
        cos = cosines(h[b * S:(b + 1) * S], want[i * S:(i + 1) * S])
        assert np.min(cos) >= COS_MIN, (b, np.min(cos))
