"""The embedding service (mx_embed_service, EmbedService::embed minus the
tokenizer) on the GPU: chunks over lanes give exactly the rows one encoder
call over the whole request gives, whatever the lane count and chunk size,
and the first failing chunk's refusal is the call's."""
import numpy as np
import pytest

import mxenc
from mxenc import synth
from test_gpu_encoder import COS_MIN, cosines, gpu_embed, oracle_embed

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = mxenc.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def model():
    return synth.make_model("minilm", layers=2, ln_random=True)


@pytest.fixture(scope="module")
def enc(ctx, model):
    e = mxenc.Encoder(ctx, model)
    yield e
    e.close()


@pytest.mark.parametrize("lanes,batch", [(1, 8), (3, 8), (4, 5), (2, 64)])
def test_service_rows_equal_one_call(ctx, model, enc, orc, lanes, batch):
    ids, am, _ = synth.make_text_inputs(model, batch=37)
    want = gpu_embed(ctx, enc, ids, am)
    svc = mxenc.EmbedService(enc, lanes, batch, ids.shape[1])
    got = svc.embed(ids, am)
    svc.close()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if lanes == 3:
        ref, _ = oracle_embed(orc, model, ids[:6].copy(), am[:6].copy())
        assert np.min(cosines(got[:6], ref)) >= COS_MIN


def test_service_repeated_calls_and_empty_request(ctx, model, enc):
    ids, am, _ = synth.make_text_inputs(model, batch=20)
    svc = mxenc.EmbedService(enc, 3, 4, ids.shape[1])
    a = svc.embed(ids, am)
    b = svc.embed(ids, am)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert svc.embed(ids[:0], am[:0]).shape == (0, model["hidden"])
    svc.close()


def test_service_first_error_is_the_calls(ctx):
    m = synth.make_model("minilm", layers=1, cls_pool=True)
    e = mxenc.Encoder(ctx, m)
    ids, am, _ = synth.make_text_inputs(m, batch=24)
    am[13, 0] = 0.0  # CLS pooling refuses a sequence whose first token is masked
    svc = mxenc.EmbedService(e, 3, 4, ids.shape[1])
    with pytest.raises(mxenc.MxError, match="first token is masked"):
        svc.embed(ids, am)
    am[13, 0] = 1.0
    assert np.all(np.isfinite(svc.embed(ids, am)))  # the service recovers
    svc.close()
    e.close()


def test_service_one_lane_refusal_mid_request(ctx):
    # One lane holds two chunks in flight: the refusal of chunk 2 (of 6) is
    # read while chunk 3 is queued. The call fails with it; the next request
    # gives the clean rows bit for bit (no flag or slot left over).
    m = synth.make_model("minilm", layers=1, cls_pool=True)
    e = mxenc.Encoder(ctx, m)
    ids, am, _ = synth.make_text_inputs(m, batch=24)
    svc = mxenc.EmbedService(e, 1, 4, ids.shape[1])
    want = gpu_embed(ctx, e, ids, am)
    bad = am.copy()
    bad[9, 0] = 0.0
    with pytest.raises(mxenc.MxError, match="first token is masked"):
        svc.embed(ids, bad)
    got = svc.embed(ids, am)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    svc.close()
    e.close()


def test_service_and_clone_refusals(ctx, enc):
    with pytest.raises(mxenc.MxError, match="lanes must be 1..64"):
        mxenc.EmbedService(enc, 0, 8, 128)
    import ctypes
    h = ctypes.c_void_p()
    mxenc.check(mxenc.lib().mx_encoder_clone(enc.handle, ctypes.byref(h)))
    a = np.zeros(8, np.float32)
    rc = mxenc.lib().mx_encoder_set(h.value, b"layer.0.ln1.bias", a.ctypes.data, mxenc.MX_F32, 8)
    assert rc == -4 and b"borrows" in mxenc.lib().mx_last_error()
    mxenc.lib().mx_encoder_destroy(h.value)


def test_clone_pins_the_owners_weights(ctx, model):
    """While a lane clone is alive its owner refuses weight changes by name
    (the clone reads the owner's device tensors); destroying the owner first
    leaves the clone running on the same weights, and the last clone's
    destroy frees them."""
    import ctypes
    ids, am, _ = synth.make_text_inputs(model, batch=6)
    owner = mxenc.Encoder(ctx, model)
    want = gpu_embed(ctx, owner, ids, am)
    lane = owner.clone(ctx)
    ln = np.zeros(model["hidden"], np.float32)
    rc = mxenc.lib().mx_encoder_set(owner.handle, b"layer.0.ln1.bias", ln.ctypes.data,
                                    mxenc.MX_F32, ln.size)
    assert rc == -4 and b"lane clone(s) borrow" in mxenc.lib().mx_last_error()
    h = ctypes.c_void_p()
    mxenc.check(mxenc.lib().mx_encoder_clone(lane.handle, ctypes.byref(h)))  # clone of a clone
    rc = mxenc.lib().mx_encoder_set(owner.handle, b"layer.0.ln1.bias", ln.ctypes.data,
                                    mxenc.MX_F32, ln.size)
    assert rc == -4 and b"2 lane clone(s)" in mxenc.lib().mx_last_error()
    mxenc.lib().mx_encoder_destroy(h.value)
    owner.close()  # the weights stay: the lane still borrows them
    got = gpu_embed(ctx, lane, ids, am)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    lane.close()
    # an owner whose clones are gone takes weight changes again
    owner = mxenc.Encoder(ctx, model)
    lane = owner.clone(ctx)
    lane.close()
    owner.set("layer.0.ln1.bias", ln)
    owner.close()
