"""mx_encoder_embed_async: the embed queued without its closing wait. Batches
queued back to back on one stream give the synchronous call's rows bit for
bit; a data refusal waits in the stream's flag until mx_sync reports it; a
batch that outgrows the workspace waits for the queued ones first."""
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


def _same(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _batches(m, n, batch, seq):
    out = []
    for i in range(n):
        ids, am, _ = synth.make_text_inputs(m, seed=100 + i, batch=batch, seq=seq)
        out.append((ids, am))
    return out


def test_queued_batches_equal_the_synchronous_call(ctx):
    m = synth.make_model("bge_base", layers=2)
    enc = mxenc.Encoder(ctx, m)
    d = m["hidden"]
    batches = _batches(m, 4, 16, 256)
    want = []
    for ids, am in batches:
        out = ctx.empty((16, d), np.float32)
        enc.embed(ctx.put(ids), ctx.put(am), 16, 256, out)
        want.append(out.host())
    dev = [(ctx.put(ids), ctx.put(am), ctx.empty((16, d), np.float32)) for ids, am in batches]
    ctx.sync()
    for _ in range(2):  # twice over, the second time on a warm tile hint
        for di, da, out in dev:
            enc.embed_async(di, da, 16, 256, out)
        ctx.sync()
        for (_, _, out), w in zip(dev, want):
            assert _same(out.host(), w)
    enc.close()


def test_refusal_waits_for_sync_and_is_cleared(ctx):
    m = synth.make_model("minilm", layers=1)
    enc = mxenc.Encoder(ctx, m)
    ids, am, _ = synth.make_text_inputs(m, batch=4, seq=64)
    bad = ids.copy()
    bad[2, 5] = m["vocab"]  # one past the vocabulary
    out = ctx.empty((4, m["hidden"]), np.float32)
    d_bad, d_am = ctx.put(bad), ctx.put(am)
    ctx.sync()
    enc.embed_async(d_bad, d_am, 4, 64, out)   # queued: no refusal yet
    with pytest.raises(mxenc.MxError, match="outside the vocabulary"):
        ctx.sync()
    ctx.sync()                                  # cleared
    good = ctx.empty((4, m["hidden"]), np.float32)
    enc.embed(ctx.put(ids), d_am, 4, 64, good)  # the synchronous call is clean again
    want = good.host()
    enc.embed_async(ctx.put(ids), d_am, 4, 64, out)
    ctx.sync()
    assert _same(out.host(), want)
    enc.close()


def test_workspace_growth_waits_for_queued_batches(ctx):
    m = synth.make_model("minilm", layers=2)
    enc = mxenc.Encoder(ctx, m)
    d = m["hidden"]
    shapes = [(4, 64), (8, 128), (16, 256)]  # each larger than every one before
    inputs = [synth.make_text_inputs(m, seed=7 + i, batch=B, seq=S)[:2]
              for i, (B, S) in enumerate(shapes)]
    ref = mxenc.Encoder(ctx, m)
    want = []
    for (B, S), (ids, am) in zip(shapes, inputs):
        out = ctx.empty((B, d), np.float32)
        ref.embed(ctx.put(ids), ctx.put(am), B, S, out)
        want.append(out.host())
    ref.close()
    dev = [(ctx.put(ids), ctx.put(am), ctx.empty((B, d), np.float32))
           for (B, S), (ids, am) in zip(shapes, inputs)]
    ctx.sync()
    for (B, S), (di, da, out) in zip(shapes, dev):
        enc.embed_async(di, da, B, S, out)
    ctx.sync()
    for (_, _, out), w in zip(dev, want):
        assert _same(out.host(), w)
    enc.close()
