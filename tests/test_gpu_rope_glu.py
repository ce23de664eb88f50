"""GPU parity of the RoPE / gated-FFN BERT archs (nomic_bert_rope_swiglu,
gte_new_rope_geglu) through the C ABI: the standalone RoPE rotation and GLU
against the oracle (bit for bit where the arithmetic is the same), the whole
stack against the oracle's host path (cosine >= 0.9999), containers of both
archs loaded by mx_encoder_from_npue, and the int8 datapath on them."""
import numpy as np
import pytest

import mxenc
import npue_writer as nw
from mxenc import synth
from orc import OrcI8, P, encoder_struct

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = mxenc.Context(0)
    yield c
    c.close()


def _cos(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return np.sum(a * b, -1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1))


def test_rope_tables_match_oracle(orc):
    for theta, inv in ((1000.0, None), (0.0, synth.make_model("gte", layers=1)["rope_inv_freq"])):
        c0, s0 = mxenc.rope_tables(300, 64, theta, inv)
        c1, s1 = np.empty_like(c0), np.empty_like(s0)
        iv = None if inv is None else np.ascontiguousarray(inv, np.float32)
        orc.orc_rope_tables(300, 64, theta, None if iv is None else P(iv), P(c1), P(s1))
        assert np.array_equal(c0, c1) and np.array_equal(s0, s1)


@pytest.mark.parametrize("B,S,H,hd,pad", [(3, 77, 12, 64, 0), (2, 128, 12, 32, 0),
                                          (2, 50, 3, 36, 0), (2, 77, 12, 64, 2)])
def test_rope_qkv_bit_exact(ctx, orc, B, S, H, hd, pad):
    """On bf16 values the GPU rotates with the host's operations (products
    rounded, no fused multiply-add) and narrows once: bit for bit the oracle's
    rotation of the same values, narrowed by to_bf16. Four pairs per thread,
    and two where head_dim % 8 != 0 or a row stride (3d + pad) leaves rows
    only 4-byte aligned; the padding columns stay untouched."""
    rng = np.random.default_rng(S)
    d = H * hd
    qkv = mxenc.from_bf16_bits(mxenc.to_bf16_bits(
        rng.standard_normal((B * S, 3 * d)).astype(np.float32) * 2))
    c, s = mxenc.rope_tables(S, hd, 1000.0)
    want = qkv.copy()
    orc.orc_rope_qkv(P(want), B * S, S, H, hd, P(c), P(s))
    bits = np.full((B * S, 3 * d + pad), 0x1234, np.uint16)
    bits[:, :3 * d] = mxenc.to_bf16_bits(qkv)
    dq = ctx.put(bits)
    mxenc.rope_qkv(ctx, dq, 3 * d + pad, B, S, H, hd, ctx.put(c), ctx.put(s))
    got = dq.host()
    assert np.array_equal(got[:, :3 * d], mxenc.to_bf16_bits(want))
    assert (got[:, 3 * d:] == 0x1234).all()


@pytest.mark.parametrize("act", [mxenc.MX_GATED_SILU, mxenc.MX_GATED_GELU_ERF])
def test_glu(ctx, orc, act):
    rng = np.random.default_rng(act)
    rows, f = 515, 3072
    up = (rng.standard_normal((rows, 2 * f)) * 3).astype(np.float32)
    want = np.empty((rows, f), np.float32)
    orc.orc_glu(P(up), rows, f, act, P(want))
    out = ctx.empty((rows, f), np.float32)
    mxenc.glu(ctx, ctx.put(up), out, rows, f, act)
    got = out.host()
    if act == mxenc.MX_GATED_SILU:
        # the host's exp2 polynomial, division and products: bit for bit
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        # fp32 erf on the GPU, double erf rounded once on the host
        assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()
    # bf16 in and out: the bf16 path of the stack
    ub = mxenc.to_bf16_bits(up)
    wb = np.empty((rows, f), np.float32)
    orc.orc_glu(P(mxenc.from_bf16_bits(ub)), rows, f, act, P(wb))
    ob = ctx.empty((rows, f), np.uint16)
    mxenc.glu(ctx, ctx.put(ub), ob, rows, f, act)
    gb = mxenc.from_bf16_bits(ob.host())
    assert np.abs(gb - wb).max() <= 2 ** -8 * np.abs(wb).max()


def _oracle_embed(orc, m, ids, am, q8=None):
    B, S = ids.shape
    d = m["hidden"]
    emb = np.empty((B * S, d), np.float32)
    cm = np.empty((B, S), np.float32)
    orc.orc_embed_sum(P(ids), P(am), B, S, d, P(m["word"]), P(m["pos"]), P(m["type"]), P(emb),
                      P(cm))
    keep = []
    enc = encoder_struct(m, keep)
    if q8 is None:
        orc.orc_bert_run(enc, P(emb), P(cm), B, S, -1)
    else:
        ops = OrcI8()
        for i, (q, ws, sm) in enumerate(q8):
            ias = np.ascontiguousarray((np.float32(1.0) / sm).astype(np.float32))
            keep += [q, ws, ias]
            ops.wq[i], ops.wscale[i], ops.ias[i] = q.ctypes.data, ws.ctypes.data, ias.ctypes.data
        orc.orc_bert_run_i8(enc, ops, P(emb), P(cm), B, S, -1)
    out = np.empty((B, d), np.float32)
    assert orc.orc_pool_rows(P(emb), P(am), B, S, d, int(m["cls_pool"]), 1, P(out)) == 0
    return out


def _gpu_embed(ctx, enc, ids, am):
    B, S = ids.shape
    out = ctx.empty((B, enc.desc.hidden), np.float32)
    enc.embed(ctx.put(ids), ctx.put(am), B, S, out)
    return out.host()


@pytest.mark.parametrize("name", ["nomic", "gte"])
def test_rope_gated_stack_vs_oracle(ctx, orc, name):
    """The arch's stack at bge-base width (768, 12 heads, FFN 2 x 3072 gated),
    4 layers, batch 8 x seq 256, every sequence checked on the host path."""
    m = synth.make_model(name, layers=4, ln_random=True)
    ids, am, _ = synth.make_text_inputs(m, batch=8, seq=256)
    want = _oracle_embed(orc, m, ids, am)
    enc = mxenc.Encoder(ctx, m)
    got = _gpu_embed(ctx, enc, ids, am)
    enc.close()
    cos = _cos(got, want)
    assert cos.min() >= 0.9999, cos
    # RoPE and the gate are live: the same weights read as plain BERT differ
    plain = dict(m, rope=False, rope_inv_freq=None, gated=0, w_up=m["w_up"][:, :, :m["ffn"]],
                 b_up=m["b_up"][:, :m["ffn"]])
    enc = mxenc.Encoder(ctx, plain)
    other = _gpu_embed(ctx, enc, ids, am)
    enc.close()
    assert _cos(other, want).min() < 0.999


@pytest.mark.parametrize("name", ["nomic", "gte"])
def test_rope_gated_bench_geometry(ctx, orc, name):
    """The arch at its benchmark shape (12 layers at bge-base width, batch 64 x
    seq 512, valid lengths U[64, 512]): the whole batch on the GPU, every
    eighth sequence and the last rerun on the host path."""
    m = synth.make_model(name, ln_random=True)
    ids, am, _ = synth.make_text_inputs(m)
    enc = mxenc.Encoder(ctx, m)
    got = _gpu_embed(ctx, enc, ids, am)
    enc.close()
    assert np.all(np.isfinite(got))
    pick = list(range(0, ids.shape[0], 8)) + [ids.shape[0] - 1]
    want = _oracle_embed(orc, m, np.ascontiguousarray(ids[pick]),
                         np.ascontiguousarray(am[pick]))
    cos = _cos(got[pick], want)
    assert cos.min() >= 0.9999, cos


@pytest.mark.parametrize("name", ["nomic", "gte"])
def test_rope_gated_container_is_bitwise_the_set_encoder(tmp_path, ctx, name):
    m = synth.make_model(name, layers=2, ln_random=True)
    path = str(tmp_path / f"{name}.npue")
    arch = "nomic_bert_rope_swiglu" if name == "nomic" else "gte_new_rope_geglu"
    nw.bert_container(m, 64, 64, (8, 8), arch=arch).write(path)
    f = mxenc.Npue(path)
    a_enc = mxenc.Encoder.from_npue(ctx, f)
    b_enc = mxenc.Encoder(ctx, m)
    ids, am, _ = synth.make_text_inputs(m, batch=6, seq=128)
    a = _gpu_embed(ctx, a_enc, ids, am)
    b = _gpu_embed(ctx, b_enc, ids, am)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    a_enc.close()
    b_enc.close()
    f.close()


@pytest.mark.parametrize("name,drop,why", [
    ("nomic", "swiglu_halves", "swiglu_halves"),
    ("nomic", "position_embedding_type", "position_embedding_type"),
    ("gte", "rope_inv_freq", "rope_inv_freq"),
    ("gte", "activation", "activation"),
])
def test_rope_gated_container_refusals(tmp_path, ctx, name, drop, why):
    m = synth.make_model(name, layers=1)
    arch = "nomic_bert_rope_swiglu" if name == "nomic" else "gte_new_rope_geglu"
    c = nw.bert_container(m, 64, 64, (8, 8), arch=arch)
    del c.config[drop]
    path = str(tmp_path / "bad.npue")
    c.write(path)
    f = mxenc.Npue(path)
    with pytest.raises(mxenc.MxError, match=why):
        mxenc.Encoder.from_npue(ctx, f)
    f.close()


def test_nomic_int8_stack(ctx, orc):
    """The int8 datapath under RoPE and SwiGLU: within the int8 scheme's own
    error of the oracle's int8 stack (the bar of test_gpu_i8)."""
    from test_gpu_i8 import _check_i8_parity, _dequantised
    m = synth.make_model("nomic", layers=2, ln_random=True)
    q8 = synth.quantise_model(m)
    ids, am, _ = synth.make_text_inputs(m, batch=6, seq=128)
    enc = mxenc.Encoder(ctx, m, int8=q8)
    got = _gpu_embed(ctx, enc, ids, am)
    enc.close()
    _check_i8_parity(got, _oracle_embed(orc, m, ids, am, q8),
                     _oracle_embed(orc, _dequantised(m, q8), ids, am), "nomic int8")


# (arch, int8 datapath, model overrides, B, S): the row counts put FFN-up's
# fused kernel on each tile -- 128 rows: 128 x 128; 1000: 128 x 256; 2048: the
# 256 x 256 tile (on 128-byte slabs, or on 64-byte slabs for a hidden width
# that is not a multiple of 64). The int8 datapath keeps FFN-up's activation
# in fp32 up to its quantiser (dequant_act_quant), so it always runs the GEMM
# and the gated-FFN pass apart: its cases check the switch leaves it as it is.
FUSED_CASES = [
    ("nomic", False, {}, 4, 512),
    ("gte", False, {}, 2, 64),
    ("gte", False, {}, 2, 500),
    ("nomic", False, dict(hidden=288, heads=9, head_dim=32), 4, 512),
    ("nomic", True, {}, 4, 512),
    ("gte", True, {}, 2, 64),
    ("nomic", True, {}, 2, 500),
    ("gte", True, dict(hidden=448, heads=7, head_dim=64), 4, 512),
]


@pytest.mark.parametrize("name,int8,over,B,S", FUSED_CASES)
def test_fused_glu_is_bitwise_the_unfused_pair(ctx, name, int8, over, B, S):
    """FFN-up with lo * act(hi) in its epilogue (the default) against the
    GEMM into the [M, 2f] intermediate followed by the gated-FFN pass: every
    row of the hidden state equal bit for bit, on both datapaths; then a new
    FFN-up bias reaches the fused path (its interleaved copies are rebuilt)."""
    m = synth.make_model(name, layers=2, ln_random=True, **over)
    d = m["hidden"]
    enc = mxenc.Encoder(ctx, m, int8=synth.quantise_model(m) if int8 else None)
    x = np.random.default_rng(B * S).standard_normal((B * S, d)).astype(np.float32)

    def run(fused):
        enc.set_fusion(fused)
        dx = ctx.put(x)
        enc.run(dx, None, None, B, S)
        return dx.host()

    try:
        a, b = run(True), run(False)
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        rng = np.random.default_rng(5)
        enc.set("layer.1.ffn_up.bias",
                rng.standard_normal(2 * m["ffn"]).astype(np.float32) * 0.5)
        c, e = run(True), run(False)
        assert np.array_equal(c.view(np.uint32), e.view(np.uint32))
        assert not np.array_equal(c.view(np.uint32), a.view(np.uint32))
    finally:
        enc.close()


def test_fused_glu_lane_clone_is_bitwise_its_parent(ctx):
    """A lane clone runs the parent's interleaved operands: the same rows."""
    m = synth.make_model("nomic", layers=2, ln_random=True)
    enc = mxenc.Encoder(ctx, m)
    lane = enc.clone(ctx)
    x = np.random.default_rng(3).standard_normal((1024, m["hidden"])).astype(np.float32)
    outs = []
    try:
        for e in (enc, lane):
            dx = ctx.put(x)
            e.run(dx, None, None, 2, 512)
            outs.append(dx.host())
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    finally:
        lane.close()
        enc.close()
