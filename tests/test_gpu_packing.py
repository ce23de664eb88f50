"""Token packing in mx_encoder_embed: only the rows before each sequence's
kv_len are computed (the padding past it is never attended as a key and never
pooled), and the pooled output must be the padded computation's bit for bit
-- on the bge-base benchmark workload itself, on mean pooling, on masks with
holes, on fully masked and one-token sequences, under RoPE + gated FFN and on
the int8 datapath."""
import numpy as np
import pytest

import mxenc
from mxenc import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = mxenc.Context(0)
    yield c
    c.close()


def _embed(ctx, enc, ids, am, packing):
    B, S = ids.shape
    enc.set_packing(packing)
    out = ctx.empty((B, enc.desc.hidden), np.float32)
    enc.embed(ctx.put(ids), ctx.put(am), B, S, out)
    return out.host()


def _same(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_bge_base_workload_packed_equals_padded(ctx):
    """The benchmark's own batch (64 x 512, lengths U[64, 512], CLS pooling)."""
    m = synth.make_model("bge_base")
    ids, am, lens = synth.make_text_inputs(m)
    enc = mxenc.Encoder(ctx, m)
    packed = _embed(ctx, enc, ids, am, True)
    padded = _embed(ctx, enc, ids, am, False)
    enc.close()
    assert _same(packed, padded)
    assert lens.sum() < 0.7 * ids.size  # the padding that packing skips


def test_mean_pooling_holes_and_edge_lengths(ctx):
    m = synth.make_model("minilm", layers=3, ln_random=True)
    ids, am, _ = synth.make_text_inputs(m, batch=9, seq=128)
    am[1, 3] = 0.0          # a hole inside the sequence: masked key, not pooled
    am[1, 10:12] = 0.0
    am[2] = 0.0             # fully masked: kv_len = S, attends uniformly
    am[3] = 0.0
    am[3, 0] = 1.0          # a single token
    am[4] = 1.0             # full length
    # negative weights past the last positive one: masked keys, but pooled
    # (pool_rows weights every row with m != 0), so packing keeps their rows
    am[5, 40:] = 0.0
    am[5, 45] = -0.5
    am[5, 60] = -1.0
    am[6] = 0.0             # no positive weight at all: uniform attention
    am[6, 7] = -1.0
    enc = mxenc.Encoder(ctx, m)
    packed = _embed(ctx, enc, ids, am, True)
    padded = _embed(ctx, enc, ids, am, False)
    enc.close()
    assert _same(packed, padded)


@pytest.mark.parametrize("name", ["nomic", "gte"])
def test_rope_gated_packed_equals_padded(ctx, name):
    """RoPE rotates a packed row by its own position (row_pos), not by its
    packed index."""
    m = synth.make_model(name, layers=2, ln_random=True)
    ids, am, _ = synth.make_text_inputs(m, batch=7, seq=192)
    enc = mxenc.Encoder(ctx, m)
    packed = _embed(ctx, enc, ids, am, True)
    padded = _embed(ctx, enc, ids, am, False)
    enc.close()
    assert _same(packed, padded)


def test_int8_packed_equals_padded(ctx):
    m = synth.make_model("bge_base", layers=3)
    ids, am, _ = synth.make_text_inputs(m, batch=16, seq=512)
    enc = mxenc.Encoder(ctx, m, int8=synth.quantise_model(m))
    packed = _embed(ctx, enc, ids, am, True)
    padded = _embed(ctx, enc, ids, am, False)
    enc.close()
    assert _same(packed, padded)


def test_packed_count_on_the_device_whatever_the_tile_hint(ctx):
    """The packed row count stays on the device; the GEMM tile is picked from
    the previous call's count. Batches of very different packed counts in
    turn -- each call's hint is the other batch's count, or none on the
    first call -- give the padded computation's rows bit for bit."""
    m = synth.make_model("bge_base", layers=2)
    enc = mxenc.Encoder(ctx, m)
    ids, am, _ = synth.make_text_inputs(m, batch=32, seq=512)
    short = am.copy()
    short[:, 80:] = 0.0                       # ~2,560 packed rows
    full = np.ones_like(am)                   # 16,384 rows: the bound itself
    want = {}
    for name, mask in (("short", short), ("full", full), ("mixed", am)):
        want[name] = _embed(ctx, enc, ids, mask, False)
    for name in ("short", "full", "mixed", "short", "mixed", "full", "short"):
        mask = {"short": short, "full": full, "mixed": am}[name]
        assert _same(_embed(ctx, enc, ids, mask, True), want[name]), name
    enc.close()


def test_packing_then_a_longer_sequence(ctx):
    """Workspaces regrow when the sequence grows at a fixed batch (mask,
    positions and packed rows)."""
    m = synth.make_model("minilm", layers=2)
    enc = mxenc.Encoder(ctx, m)
    for S in (64, 128, 256):
        ids, am, _ = synth.make_text_inputs(m, batch=4, seq=S)
        assert _same(_embed(ctx, enc, ids, am, True), _embed(ctx, enc, ids, am, False))
    enc.close()



def _embed_pruned(ctx, enc, ids, am, packing, prune):
    enc.set_cls_pruning(prune)
    try:
        return _embed(ctx, enc, ids, am, packing)
    finally:
        enc.set_cls_pruning(True)


def test_cls_pruning_is_bitwise_the_full_last_layer(ctx):
    """CLS pooling: the last layer's attention-out, LayerNorms and FFN over each
    sequence's first row only give the pooled output of the last layer over
    every row, bit for bit -- on the benchmark's own batch, packed and padded."""
    m = synth.make_model("bge_base")
    ids, am, _ = synth.make_text_inputs(m)
    enc = mxenc.Encoder(ctx, m)
    for packing in (True, False):
        pruned = _embed_pruned(ctx, enc, ids, am, packing, True)
        full = _embed_pruned(ctx, enc, ids, am, packing, False)
        assert _same(pruned, full), f"packing={packing}"
    enc.close()


def test_cls_pruning_gte_rope_geglu(ctx):
    """gte (RoPE, GeGLU fused into FFN-up, CLS pooling): the pruned layer's
    gated FFN over the gathered rows."""
    m = synth.make_model("gte", layers=2, ln_random=True)
    assert m["cls_pool"]
    ids, am, _ = synth.make_text_inputs(m, batch=7, seq=192)
    enc = mxenc.Encoder(ctx, m)
    for packing in (True, False):
        assert _same(_embed_pruned(ctx, enc, ids, am, packing, True),
                     _embed_pruned(ctx, enc, ids, am, packing, False)), f"packing={packing}"
    enc.close()


def test_cls_pruning_int8_and_mean_pooling(ctx):
    """The int8 datapath (the context quantised from the gathered rows), and
    mean pooling, where pruning does not apply and changes nothing."""
    m = synth.make_model("bge_base", layers=3)
    ids, am, _ = synth.make_text_inputs(m, batch=16, seq=512)
    enc = mxenc.Encoder(ctx, m, int8=synth.quantise_model(m))
    assert _same(_embed_pruned(ctx, enc, ids, am, True, True),
                 _embed_pruned(ctx, enc, ids, am, True, False))
    enc.close()
    m = synth.make_model("minilm", layers=2)
    assert not m["cls_pool"]
    ids, am, _ = synth.make_text_inputs(m, batch=8, seq=128)
    enc = mxenc.Encoder(ctx, m)
    assert _same(_embed_pruned(ctx, enc, ids, am, True, True),
                 _embed_pruned(ctx, enc, ids, am, True, False))
    enc.close()


def test_cls_pruning_masked_cls_is_still_refused(ctx):
    """A sequence whose first token is masked cannot be CLS-pooled: refused
    by name with pruning on, as without it."""
    m = synth.make_model("bge_base", layers=1)
    ids, am, _ = synth.make_text_inputs(m, batch=4, seq=64)
    am[2, 0] = 0.0
    enc = mxenc.Encoder(ctx, m)
    out = ctx.empty((4, m["hidden"]), np.float32)
    for prune in (True, False):
        enc.set_cls_pruning(prune)
        with pytest.raises(mxenc.MxError, match="first token is masked"):
            enc.embed(ctx.put(ids), ctx.put(am), 4, 64, out)
    enc.close()
