"""mx_encoder_embed_static, the embed that allocates nothing: its workspace is
carved from the library's static device scratch (MX_STATIC_SCRATCH_BYTES per
GPU). Through the C ABI its pooled rows must be mx_encoder_embed's bit for bit
-- on two calls in a row, the second with a smaller batch, on each datapath
(bf16 BERT, the RoPE / gated-FFN BERT, the int8 design) and with token packing
on and off; batches past the scratch, timing and stale device tables are
refused by name, and the scratch serves the next call after a refusal."""
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


def embed_both(ctx, enc, ids, am):
    """(mx_encoder_embed's rows, mx_encoder_embed_static's rows) for one batch."""
    B, S = ids.shape
    d_ids, d_am = ctx.put(ids), ctx.put(am)
    out_a = ctx.empty((B, enc.desc.hidden), np.float32)
    out_b = ctx.empty((B, enc.desc.hidden), np.float32)
    enc.embed(d_ids, d_am, B, S, out_a)
    enc.embed_static(d_ids, d_am, B, S, out_b)
    return out_a.host(), out_b.host()


def small_model(name, **kw):
    return synth.make_model(name, layers=2, ln_random=True, **kw)


CASES = {
    "minilm": lambda: (small_model("minilm"), {}),
    "nomic": lambda: (small_model("nomic", hidden=256, heads=4, head_dim=64, ffn=512), {}),
    "gte": lambda: (small_model("gte", hidden=256, heads=4, head_dim=64, ffn=512), {}),
    "bge_int8": lambda: (lambda m: (m, {"int8": synth.quantise_model(m)}))(
        small_model("bge_base", hidden=256, heads=4, head_dim=64, ffn=1024)),
}


@pytest.mark.parametrize("packing", [True, False], ids=["packed", "padded"])
@pytest.mark.parametrize("name", sorted(CASES))
def test_static_embed_is_embed_bitwise_on_two_calls(ctx, name, packing):
    m, kw = CASES[name]()
    enc = mxenc.Encoder(ctx, m, **kw)
    enc.set_packing(packing)
    print(f"static embed: {name} packing={packing}", flush=True)
    # the first call at 24 x 128, the second smaller (6 x 40): the scratch
    # keeps the first call's contents, which the second must not read
    for B, S in ((24, 128), (6, 40)):
        ids, am, _ = synth.make_text_inputs(m, batch=B, seq=S, seed=B * 1000 + S)
        want, got = embed_both(ctx, enc, ids, am)
        assert np.isfinite(want).all()
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), (name, B, S)
    enc.close()


def test_static_embed_shared_scratch_two_encoders(ctx):
    """Two encoders take turns on the one scratch: each call's rows are its own
    encoder's embed."""
    m1, _ = CASES["minilm"]()
    m2, _ = CASES["nomic"]()
    e1, e2 = mxenc.Encoder(ctx, m1), mxenc.Encoder(ctx, m2)
    ids1, am1, _ = synth.make_text_inputs(m1, batch=16, seq=96)
    ids2, am2, _ = synth.make_text_inputs(m2, batch=8, seq=64)
    w1, g1 = embed_both(ctx, e1, ids1, am1)
    w2, g2 = embed_both(ctx, e2, ids2, am2)
    _, g1b = embed_both(ctx, e1, ids1, am1)
    assert np.array_equal(w1.view(np.uint32), g1.view(np.uint32))
    assert np.array_equal(w2.view(np.uint32), g2.view(np.uint32))
    assert np.array_equal(g1.view(np.uint32), g1b.view(np.uint32))
    e1.close()
    e2.close()


def test_static_embed_allocates_nothing_as_first_call(ctx):
    """On a freshly readied encoder that has never run mx_encoder_embed (so it
    has no workspace), mx_encoder_embed_static runs twice -- the second call
    smaller -- without a single device allocation by the library; the rows are
    then mx_encoder_embed's, bit for bit."""
    m, _ = CASES["minilm"]()
    enc = mxenc.Encoder(ctx, m)
    enc.ready()
    L = mxenc.lib()
    batches = []
    for B, S in ((24, 128), (6, 40)):
        ids, am, _ = synth.make_text_inputs(m, batch=B, seq=S, seed=B * 7 + S)
        batches.append((ids, am, ctx.put(ids), ctx.put(am),
                        ctx.empty((B, m["hidden"]), np.float32)))
    before = L.mx_device_allocations()
    for ids, am, d_ids, d_am, out in batches:
        B, S = ids.shape
        enc.embed_static(d_ids, d_am, B, S, out)
    ctx.sync()
    assert L.mx_device_allocations() == before
    for ids, am, d_ids, d_am, out in batches:
        B, S = ids.shape
        got = out.host()
        want = ctx.empty((B, m["hidden"]), np.float32)
        enc.embed(d_ids, d_am, B, S, want)
        assert np.array_equal(want.host().view(np.uint32), got.view(np.uint32)), (B, S)
    # mx_encoder_embed does allocate (its workspace): the counter sees it
    assert L.mx_device_allocations() > before
    enc.close()


def test_static_embed_refuses_an_overlapping_call(ctx):
    """While another call holds this GPU's static scratch (here: the guard held
    as a call holds it), mx_encoder_embed_static is refused by name before it
    touches the scratch; once the guard is back, the same call runs and gives
    mx_encoder_embed's rows. Nothing depends on timing."""
    m, _ = CASES["minilm"]()
    enc = mxenc.Encoder(ctx, m)
    ids, am, _ = synth.make_text_inputs(m, batch=4, seq=64)
    d_ids, d_am = ctx.put(ids), ctx.put(am)
    out = ctx.empty((4, m["hidden"]), np.float32)
    L = mxenc.lib()
    assert L.mx_static_guard_hold(0) == mxenc.MX_OK
    try:
        with pytest.raises(RuntimeError, match="in use by another call"):
            enc.embed_static(d_ids, d_am, 4, 64, out)
    finally:
        assert L.mx_static_guard_release(0) == mxenc.MX_OK
    want, got = embed_both(ctx, enc, ids, am)
    assert np.array_equal(want.view(np.uint32), got.view(np.uint32))
    # the guard is free again after a call (and after a refused one)
    assert L.mx_static_guard_hold(0) == mxenc.MX_OK
    assert L.mx_static_guard_release(0) == mxenc.MX_OK
    enc.close()


def test_static_embed_refusals(ctx):
    m = synth.make_model("bge_base", layers=1)
    enc = mxenc.Encoder(ctx, m)
    d = m["hidden"]
    # padded: 64 x 512 rows of bge-base need ~600 MB; refused before any launch
    enc.set_packing(False)
    B, S = 64, 512
    ids, am, _ = synth.make_text_inputs(m, batch=B, seq=S)
    d_ids, d_am = ctx.put(ids), ctx.put(am)
    out = ctx.empty((B, d), np.float32)
    with pytest.raises(RuntimeError, match="MX_STATIC_SCRATCH_BYTES"):
        enc.embed_static(d_ids, d_am, B, S, out)
    # packed: the same batch packs to more rows than the scratch holds
    enc.set_packing(True)
    with pytest.raises(RuntimeError, match="packs to [0-9]+ rows"):
        enc.embed_static(d_ids, d_am, B, S, out)
    # after the refusals the scratch serves a batch that fits
    ids, am, _ = synth.make_text_inputs(m, batch=4, seq=64)
    want, got = embed_both(ctx, enc, ids, am)
    assert np.array_equal(want.view(np.uint32), got.view(np.uint32))
    # timing on: refused (its events are created on demand)
    enc.set_timing(True)
    small_ids, small_am = ctx.put(ids), ctx.put(am)
    small_out = ctx.empty((4, d), np.float32)
    with pytest.raises(RuntimeError, match="timing"):
        enc.embed_static(small_ids, small_am, 4, 64, small_out)
    enc.set_timing(False)
    enc.close()
    # stale device tables: a gated encoder whose FFN-up weight was set again
    # after it was made ready; mx_encoder_ready brings it back
    mg, _ = CASES["nomic"]()
    eg = mxenc.Encoder(ctx, mg)
    eg.set("layer.0.ffn_up", mg["w_up"][0])
    ids, am, _ = synth.make_text_inputs(mg, batch=4, seq=64)
    gi, ga = ctx.put(ids), ctx.put(am)
    gout = ctx.empty((4, mg["hidden"]), np.float32)
    with pytest.raises(RuntimeError, match="not built"):
        eg.embed_static(gi, ga, 4, 64, gout)
    eg.ready()
    want, got = embed_both(ctx, eg, ids, am)
    assert np.array_equal(want.view(np.uint32), got.view(np.uint32))
    eg.close()
