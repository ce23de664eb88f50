"""The .npue container on the GPU: pre-tiled bf16 operands untiled by the GPU
kernel land exactly where the host untile puts them, and an encoder built
straight from a BERT container computes bit for bit what the same weights
given tensor by tensor compute (whose parity with the host path
test_gpu_encoder pins)."""
import ctypes

import numpy as np
import pytest

import mxenc
import npue_writer as nw
from mxenc import synth
from orc import P
from test_gpu_encoder import COS_MIN, cosines, gpu_embed, oracle_embed
from test_npue_cpu import I4_CASES, _fold_i4_numpy, _i4_operand

pytestmark = pytest.mark.gpu

TILINGS = [(768, 2304, 64, 48, 8, 4), (3072, 768, 64, 64, 8, 8), (384, 1152, 32, 32, 4, 8),
           (1024, 96, 128, 96, 8, 8)]


@pytest.fixture(scope="module")
def ctx():
    c = mxenc.Context(0)
    yield c
    c.close()


def _gemm_slot(ctx, A, M, K, slot, N, bias):
    C = ctx.empty((M, N), np.float32)
    mxenc.check(mxenc.lib().mx_gemm(ctx.stream, A.p, M, K, K, slot, bias.p, mxenc.MX_EPI_NONE,
                                    None, C.p, mxenc.MX_F32, N))
    return C.host()


@pytest.mark.parametrize("K,N,tk,tn,s,t", TILINGS)
def test_panel_staging_equals_row_major_staging(ctx, orc, K, N, tk, tn, s, t):
    """mx_stage_weight_panel (container bytes, untiled on the GPU) and
    mx_stage_weight (row-major) of the same operand give bit-identical GEMMs,
    and the untiled operand is the oracle's untile of the same bytes."""
    rng = np.random.default_rng(K + N + tk)
    W = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    bits = nw.to_bf16_bits(W)
    panel = nw.tile_panel(bits, tk, tn, s, t)
    kn = np.zeros_like(bits)
    assert orc.orc_untile_b_panel(P(panel), K, N, tk, tn, s, t, P(kn)) == 0
    assert np.array_equal(kn, bits)
    sp = mxenc.stage_weight_panel(ctx, panel, K, N, tk, tn, s, t)
    sr = ctypes.c_int()
    mxenc.check(mxenc.lib().mx_stage_weight(ctx.handle, bits.ctypes.data, mxenc.MX_BF16, K, N,
                                            ctypes.byref(sr)))
    M = 512
    A = ctx.put(nw.to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32)))
    bias = ctx.put((rng.standard_normal(N) * 0.1).astype(np.float32))
    a = _gemm_slot(ctx, A, M, K, sp, N, bias)
    b = _gemm_slot(ctx, A, M, K, sr.value, N, bias)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    mxenc.check(mxenc.lib().mx_release_weight(ctx.handle, sp))
    mxenc.check(mxenc.lib().mx_release_weight(ctx.handle, sr.value))


def test_panel_staging_refusals(ctx):
    panel = np.zeros(64 * 96, np.uint16)
    with pytest.raises(mxenc.MxError, match="does not tile"):
        mxenc.stage_weight_panel(ctx, panel, 64, 96, 64, 64, 8, 8)
    with pytest.raises(mxenc.MxError, match="does not tile"):
        mxenc.stage_weight_panel(ctx, panel, 64, 96, 64, 48, 6, 4)
    with pytest.raises(mxenc.MxError, match="64 KB of LDS"):
        mxenc.stage_weight_panel(ctx, np.zeros(512 * 512, np.uint16), 512, 512, 512, 512, 8, 8)


@pytest.mark.parametrize("tiling,cls_pool", [((64, 48, (8, 4)), False), ((32, 64, (4, 8)), True)])
def test_encoder_from_npue_is_bitwise_the_set_encoder(tmp_path, ctx, orc, tiling, cls_pool):
    m = synth.make_model("minilm", layers=2, ln_random=True, cls_pool=cls_pool)
    tk, tn, mac = tiling
    path = str(tmp_path / "minilm.npue")
    nw.bert_container(m, tk, tn, mac).write(path)
    f = mxenc.Npue(path)
    a_enc = mxenc.Encoder.from_npue(ctx, f)
    b_enc = mxenc.Encoder(ctx, m)
    ids, am, lens = synth.make_text_inputs(m, batch=8)
    a = gpu_embed(ctx, a_enc, ids, am)
    b = gpu_embed(ctx, b_enc, ids, am)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    want, _ = oracle_embed(orc, m, ids, am)
    assert np.min(cosines(a, want)) >= COS_MIN
    a_enc.close()
    b_enc.close()
    f.close()


@pytest.mark.parametrize("over,why", [
    (dict(arch="gemma3_mqa_rope_geglu"), "other archs share its tensor names"),
    (dict(arch="nomic_bert_rope_swiglu"), "position_embedding_type is not 'rope'"),
    (dict(gemm_layout="host"), "gemm_layout \"host\""),
    (dict(pooling="max"), "unknown pooling mode 'max'"),
])
def test_encoder_from_npue_refusals(tmp_path, ctx, over, why):
    m = synth.make_model("minilm", layers=1)
    path = str(tmp_path / "bad.npue")
    arch = over.pop("arch", "bert_abs_gelu_postln")
    nw.bert_container(m, 64, 64, (8, 8), arch=arch, extra_config=over).write(path)
    f = mxenc.Npue(path)
    with pytest.raises(mxenc.MxError, match=why):
        mxenc.Encoder.from_npue(ctx, f)
    f.close()


def test_encoder_from_npue_refuses_short_i4_mixed_and_missing_tensors(tmp_path, ctx):
    m = synth.make_model("minilm", layers=1)
    c = nw.bert_container(m, 64, 64, (8, 8))
    for e in c.entries:
        if e["name"] == "layer.0.attn_out":
            e["dtype"] = "I4"  # bf16-sized bytes under an I4 tag
    path = str(tmp_path / "i4.npue")
    c.write(path)
    f = mxenc.Npue(path)
    with pytest.raises(mxenc.MxError, match="int4 operand"):
        mxenc.Encoder.from_npue(ctx, f)
    f.close()
    # an int8 operand among bf16 ones: one datapath per stack
    q8 = synth.quantise_model(m)
    c = nw.bert_container(m, 64, 64, (8, 8))
    c.entries = [e for e in c.entries if e["name"] != "layer.0.attn_out"]
    q, ws, sm = q8[1]
    c.add_gemm_i8("layer.0.attn_out", q[0], ws[0], sm[0], 64, 64, 8, 8)
    path = str(tmp_path / "mixed.npue")
    c.write(path)
    f = mxenc.Npue(path)
    with pytest.raises(mxenc.MxError, match="one datapath"):
        mxenc.Encoder.from_npue(ctx, f)
    f.close()
    c = nw.bert_container(m, 64, 64, (8, 8))
    c.entries = [e for e in c.entries if e["name"] != "layer.0.ln2.bias"]
    path = str(tmp_path / "missing.npue")
    c.write(path)
    f = mxenc.Npue(path)
    with pytest.raises(mxenc.MxError, match="no tensor named layer.0.ln2.bias"):
        mxenc.Encoder.from_npue(ctx, f)
    f.close()


@pytest.mark.parametrize("act,gated", [("gelu", mxenc.MX_GATED_GELU_ERF), (None, mxenc.MX_GATED_SILU)])
def test_gated_bert_container_reads_its_activation(tmp_path, ctx, act, gated):
    """A gated FFN on the plain BERT arch (absolute positions) takes its gate
    activation from the container's 'activation' key, SiLU when the key is
    missing, as set_model_shape reads it for every gated arch but gemma."""
    m = dict(synth.make_model("gte", layers=2, ln_random=True))
    m["rope"] = False
    m.pop("rope_inv_freq", None)
    m["gated"] = gated
    extra = {"gated_ffn": True}
    c = nw.bert_container(m, 64, 64, (8, 8), extra_config=extra)
    if act is None:
        c.config.pop("activation", None)
    else:
        c.config["activation"] = act
    path = str(tmp_path / "gated.npue")
    c.write(path)
    f = mxenc.Npue(path)
    a_enc = mxenc.Encoder.from_npue(ctx, f)
    b_enc = mxenc.Encoder(ctx, m)
    ids, am, _ = synth.make_text_inputs(m, batch=4, seq=128)
    a = gpu_embed(ctx, a_enc, ids, am)
    b = gpu_embed(ctx, b_enc, ids, am)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    a_enc.close()
    b_enc.close()
    f.close()


def test_gated_bert_container_unknown_activation_refused(tmp_path, ctx):
    m = dict(synth.make_model("gte", layers=1))
    m["rope"] = False
    m.pop("rope_inv_freq", None)
    c = nw.bert_container(m, 64, 64, (8, 8), extra_config={"gated_ffn": True,
                                                           "activation": "relu"})
    path = str(tmp_path / "relu.npue")
    c.write(path)
    f = mxenc.Npue(path)
    with pytest.raises(mxenc.MxError, match="unknown gated-FFN activation 'relu'"):
        mxenc.Encoder.from_npue(ctx, f)
    f.close()


# ---- int4 storage over the int8 datapath (common/int4_panel.hpp) --------------------

I4_GPU_CASES = I4_CASES + [
    (768, 2304, 64, 48, 8, 4, 32),   # bge-base QKV operand
    (3072, 768, 64, 64, 8, 8, 0),    # bge-base FFN-down, one group over K
]


@pytest.mark.parametrize("K,N,tk,tn,s,t,group", I4_GPU_CASES)
def test_widen_panel_i4_is_the_oracle_widening(ctx, orc, K, N, tk, tn, s, t, group):
    """mx_widen_panel_i4 on the GPU and the oracle (pinned to the reference's
    gemm_b_panel) widen the same stored bytes to identical int8 runs: ties
    to even, clipping at +-127, groups straddling the sub-tile rows."""
    tv, gs = _i4_operand(K, N, group, K * N + group + 1)
    packed = nw.pack_i4(nw.tile_panel(tv, tk, tn, s, t))
    want = np.zeros(K * N, np.int8)
    assert orc.orc_widen_i4_panel(P(packed), K, N, tk, tn, s, t, P(gs), group, P(want)) == 0
    out = ctx.empty((K * N,), np.int8)
    mxenc.widen_panel_i4(ctx, ctx.put(packed), ctx.put(gs), group, K, N, tk, tn, s, t, out)
    assert np.array_equal(out.host(), want)


def test_widen_panel_i4_refusals(ctx):
    buf = ctx.empty((64 * 64,), np.uint8)
    gs = ctx.empty((64 * 64,), np.float32)
    out = ctx.empty((64 * 64,), np.int8)
    with pytest.raises(mxenc.MxError, match="odd number of nibbles"):
        mxenc.widen_panel_i4(ctx, buf, gs, 0, 63, 1, 63, 1, 1, 1, out)
    with pytest.raises(mxenc.MxError, match="must be >= 0"):
        mxenc.widen_panel_i4(ctx, buf, gs, -1, 64, 64, 64, 64, 8, 8, out)
    with pytest.raises(mxenc.MxError, match="does not tile"):
        mxenc.widen_panel_i4(ctx, buf, gs, 0, 64, 64, 48, 64, 8, 8, out)


@pytest.mark.parametrize("group", [32, 0])
def test_i4_container_is_bitwise_its_widened_i8_container(tmp_path, ctx, group):
    """An --int4 pack (I4 nibbles, .gscale, config int4_group) loaded by
    mx_encoder_from_npue embeds bit for bit what the --int8 pack holding the
    widened panels (the packer's fold, pinned to gemm_b_panel) embeds: int4 is
    storage over the int8 datapath, and nothing downstream of the widening
    differs."""
    m = synth.make_model("minilm", layers=2, ln_random=True)
    q4 = synth.quantise_model_i4(m, group=group)
    q8 = []
    for t, ws, gs, sm in q4:
        q8.append((np.stack([_fold_i4_numpy(t[l], gs[l], group) for l in range(t.shape[0])]),
                   ws, sm))
    p4, p8 = str(tmp_path / "m4.npue"), str(tmp_path / "m8.npue")
    nw.bert_container(m, 64, 48, (8, 4), int4=q4, int4_group=group).write(p4)
    nw.bert_container(m, 64, 48, (8, 4), int8=q8).write(p8)
    f4, f8 = mxenc.Npue(p4), mxenc.Npue(p8)
    e4, e8 = mxenc.Encoder.from_npue(ctx, f4), mxenc.Encoder.from_npue(ctx, f8)
    ids, am, _ = synth.make_text_inputs(m, batch=8)
    a, b = gpu_embed(ctx, e4, ids, am), gpu_embed(ctx, e8, ids, am)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.all(np.isfinite(a))
    e4.close()
    e8.close()
    f4.close()
    f8.close()


def test_i4_container_refusals(tmp_path, ctx):
    """The loader refuses an int4 pack as gemm_b_panel does (int4_panel.hpp:
    127-173): no int4_group, a negative one, no .gscale, a .gscale whose rows
    do not match the group size."""
    m = synth.make_model("minilm", layers=1)
    q4 = synth.quantise_model_i4(m, group=32)

    def load(c, name):
        path = str(tmp_path / name)
        c.write(path)
        f = mxenc.Npue(path)
        try:
            mxenc.Encoder.from_npue(ctx, f).close()
        finally:
            f.close()

    c = nw.bert_container(m, 64, 64, (8, 8), int4=q4)
    del c.config["int4_group"]
    with pytest.raises(mxenc.MxError, match="states no int4_group"):
        load(c, "nogroup.npue")
    c = nw.bert_container(m, 64, 64, (8, 8), int4=q4, int4_group=-4)
    with pytest.raises(mxenc.MxError, match="must be >= 0"):
        load(c, "neg.npue")
    c = nw.bert_container(m, 64, 64, (8, 8), int4=q4)
    c.entries = [e for e in c.entries if e["name"] != "layer.0.qkv.gscale"]
    with pytest.raises(mxenc.MxError, match="no layer.0.qkv.gscale"):
        load(c, "nogs.npue")
    c = nw.bert_container(m, 64, 64, (8, 8), int4=q4, int4_group=16)
    with pytest.raises(mxenc.MxError, match="gscale is F32"):
        load(c, "rows.npue")


def test_cxx_caller_embeds_what_the_binding_embeds(tmp_path, ctx):
    """The C++17 caller (tests/abi_cxx/abi_check.cpp over include/
    mx_gpu_backend.hpp, built by the host compiler and linked to the library)
    loads a container and embeds a batch in a process of its own; its pooled
    rows are bit for bit the ctypes binding's. In the same process it checks
    the queued embed and the embed service (two lanes, chunks of 3) give the
    same rows."""
    import os
    import subprocess
    m = synth.make_model("minilm", layers=2, ln_random=True)
    path = str(tmp_path / "m.npue")
    nw.bert_container(m, 64, 48, (8, 4)).write(path)
    ids, am, _ = synth.make_text_inputs(m, batch=6)
    B, S = ids.shape
    ids.tofile(str(tmp_path / "ids.bin"))
    am.astype(np.float32).tofile(str(tmp_path / "mask.bin"))
    exe = os.path.join(os.path.dirname(mxenc.LIB_PATH), "abi_check")
    print("abi_check gpu: minilm 2 layers, B", B, "S", S, flush=True)
    r = subprocess.run([exe, "gpu", path, str(tmp_path / "ids.bin"), str(tmp_path / "mask.bin"),
                        str(B), str(S), str(tmp_path / "out.bin")], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and r.stdout.strip().endswith("gpu ok"), r.stdout + r.stderr
    got = np.fromfile(str(tmp_path / "out.bin"), np.float32).reshape(B, m["hidden"])
    f = mxenc.Npue(path)
    enc = mxenc.Encoder.from_npue(ctx, f)
    want = gpu_embed(ctx, enc, ids, am)
    enc.close()
    f.close()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
