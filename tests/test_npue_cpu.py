"""The .npue container on the CPU: the product's reader (mx_npue_*, host code
in libmx_encoder.so) and the oracle's B-panel untile, pinned against the
reference's own reader and host_b_kn compiled into oracle/_ref
(runtime/src/model.cpp, common/host_b.hpp), a hand-worked tile, and the
tiling written as reshapes (tests/npue_writer.py)."""
import ctypes
import json

import numpy as np
import pytest

import mxenc
import npue_writer as nw
from orc import P

TILINGS = [  # (K, N, tile_k, tile_n, mac_s, mac_t): the packer's npu1/npu2 sub-tiles
    (128, 96, 64, 48, 8, 4),
    (64, 128, 64, 64, 8, 8),
    (96, 64, 32, 32, 4, 8),
    (16, 24, 8, 8, 2, 4),
]


def _rand_kn(K, N, seed):
    return (np.random.default_rng(seed).standard_normal((K, N)) * 0.05).astype(np.float32)


def test_untile_hand_worked_tile(orc):
    """One 2 x 4 tile of 2 x 2 sub-tiles: the container holds W[0,0:2],
    W[1,0:2], W[0,2:4], W[1,2:4] in that order."""
    W = np.array([[0, 1, 2, 3], [4, 5, 6, 7]], np.uint16)
    stored = np.array([0, 1, 4, 5, 2, 3, 6, 7], np.uint16)
    assert np.array_equal(nw.tile_panel(W, 2, 4, 2, 2), stored)
    out = np.zeros((2, 4), np.uint16)
    assert orc.orc_untile_b_panel(P(stored), 2, 4, 2, 4, 2, 2, P(out)) == 0
    assert np.array_equal(out, W)


@pytest.mark.parametrize("K,N,tk,tn,s,t", TILINGS)
def test_untile_inverts_the_tiling(orc, K, N, tk, tn, s, t):
    bits = np.random.default_rng(K * N + tk).integers(0, 65536, (K, N)).astype(np.uint16)
    out = np.zeros_like(bits)
    assert orc.orc_untile_b_panel(P(nw.tile_panel(bits, tk, tn, s, t)), K, N, tk, tn, s, t,
                                  P(out)) == 0
    assert np.array_equal(out, bits)


def test_untile_refuses_what_host_b_kn_refuses(orc):
    buf = np.zeros(64 * 64, np.uint16)
    out = np.zeros_like(buf)
    for args in [(64, 64, 48, 64, 8, 8), (64, 64, 64, 48, 8, 8), (64, 64, 64, 64, 6, 8),
                 (64, 64, 64, 64, 8, 5), (0, 64, 64, 64, 8, 8)]:
        assert orc.orc_untile_b_panel(P(buf), *args, P(out)) == -1


@pytest.mark.parametrize("K,N,tk,tn,s,t", TILINGS)
def test_untile_matches_reference_host_b_kn(tmp_path, orc, ref, K, N, tk, tn, s, t):
    """The reference's npue::File + hostb::host_b_kn read the written file; the
    oracle untiles the same stored bytes: identical, and equal to the bf16
    rounding of the matrix that was packed."""
    W = _rand_kn(K, N, K + N + tk)
    c = nw.Container({"arch": "bert_abs_gelu_postln"})
    c.add_gemm("layer.0.qkv", W, tk, tn, s, t)
    path = str(tmp_path / "w.npue")
    c.write(path)
    got = np.zeros((K, N), np.float32)
    err = ctypes.create_string_buffer(512)
    n = ref.ref_npue_host_b_kn(path.encode(), b"layer.0.qkv", P(got), got.size, err, 512)
    assert n == K * N, err.value
    stored = np.frombuffer(mxenc.Npue(path).bytes("layer.0.qkv"), np.uint16)
    mine = np.zeros((K, N), np.uint16)
    assert orc.orc_untile_b_panel(P(np.ascontiguousarray(stored)), K, N, tk, tn, s, t,
                                  P(mine)) == 0
    assert np.array_equal(mxenc.from_bf16_bits(mine).view(np.uint32), got.view(np.uint32))
    assert np.array_equal(mine, nw.to_bf16_bits(W))


def _config_cases():
    return {
        "arch": "bert_abs_gelu_postln", "num_layers": 12, "hidden": 768, "eps": 1e-12,
        "neg": -3, "flag": True, "off": False, "nothing": None,
        "quote": 'say "hi" \\ back/slash\ttab\nline', "latin": "café ß",
        "cjk": "模型", "nested": {"a": [1, 2, {"b": "c\"d"}], "e": {}},
        "list": [1, 2.5, "x", [], True], "empty": "",
    }


def test_reader_matches_reference_reader(tmp_path, ref):
    cfg = _config_cases()
    c = nw.Container(cfg)
    W = _rand_kn(64, 48, 1)
    c.add_gemm("layer.0.ffn_up", W, 32, 48, 8, 4)
    c.add_f32("layer.0.ffn_up.bias", np.arange(48, dtype=np.float32), "bias")
    c.add("tokenizer.vocab", np.frombuffer(b"[PAD]\n[CLS]\n", np.uint8), "U8", "tokenizer",
          [12])
    path = str(tmp_path / "c.npue")
    c.write(path)
    f = mxenc.Npue(path)
    buf = ctypes.create_string_buffer(4096)
    err = ctypes.create_string_buffer(512)
    for key in cfg:
        n = ref.ref_npue_config(path.encode(), key.encode(), buf, 4096, err, 512)
        assert n >= 0, err.value
        assert f.config(key).encode("utf-8") == buf.raw[:n], key
    # strings come back unescaped; non-string values as their JSON text
    assert f.config("quote") == cfg["quote"]
    assert f.config("latin") == cfg["latin"]
    assert json.loads(f.config("nested")) == cfg["nested"]
    assert f.config("flag") == "true" and f.config("nothing") == "null"
    assert f.names() == ["layer.0.ffn_up", "layer.0.ffn_up.bias", "tokenizer.vocab"]
    for name in f.names():
        info = f.info(name)
        dt = ctypes.create_string_buffer(8)
        padded = np.zeros(4, np.int64)
        lay = np.zeros(4, np.int64)
        nd = ctypes.c_int()
        nb = ctypes.c_ulonglong()
        raw = np.zeros(1 << 16, np.uint8)
        assert ref.ref_npue_tensor(path.encode(), name.encode(), dt, P(padded),
                                   ctypes.byref(nd), P(lay), P(raw), raw.size,
                                   ctypes.byref(nb)) == 0
        assert info.dtype == dt.value and info.ndim == nd.value
        assert list(info.padded_shape[:info.ndim]) == list(padded[:nd.value])
        assert [info.tile_k, info.tile_n, info.mac_s, info.mac_t] == list(lay)
        assert info.nbytes == nb.value
        assert f.bytes(name) == raw[:nb.value].tobytes()
    assert f.info("layer.0.ffn_up").block_panel == 1
    assert f.info("layer.0.ffn_up.bias").block_panel == 0
    with pytest.raises(mxenc.MxError, match="no config key absent"):
        f.config("absent")
    with pytest.raises(mxenc.MxError, match="no tensor named layer.9.qkv"):
        f.info("layer.9.qkv")
    f.close()


def test_surrogate_pairs_decode_to_utf8(tmp_path):
    """json.dumps writes a character beyond the BMP as a \\u surrogate pair;
    the reader joins the pair into one 4-byte UTF-8 sequence."""
    c = nw.Container({"emoji": "a\U0001F600b"})
    path = str(tmp_path / "e.npue")
    c.write(path)
    assert mxenc.Npue(path).config("emoji") == "a\U0001F600b"


def _malformed(tmp_path, name, **kw):
    c = nw.Container({"arch": "bert_abs_gelu_postln"})
    c.add_f32("x", np.ones(4, np.float32), "bias")
    path = str(tmp_path / name)
    c.write(path, **kw)
    return path, c


@pytest.mark.parametrize("kw,why", [
    (dict(magic=b"NPUX"), "not a .npue file"),
    (dict(version=2), "version 2, expected 1"),
    (dict(data_align=16), "data_offset is not 4096-aligned"),
    (dict(trailing=b"\0"), "size does not match"),
])
def test_reader_refusals_match_reference(tmp_path, ref, kw, why):
    path, _ = _malformed(tmp_path, "bad.npue", **kw)
    with pytest.raises(mxenc.MxError, match=why):
        mxenc.Npue(path)
    err = ctypes.create_string_buffer(512)
    assert ref.ref_npue_open(path.encode(), err, 512) == -1
    assert why.split(",")[0] in err.value.decode()


def test_reader_refuses_a_tensor_past_the_data(tmp_path, ref):
    c = nw.Container({"arch": "bert_abs_gelu_postln"})
    e = c.add_f32("x", np.ones(4, np.float32), "bias")
    e["nbytes"] = 1 << 20
    path = str(tmp_path / "past.npue")
    c.write(path)
    with pytest.raises(mxenc.MxError, match="tensor x runs past the data segment"):
        mxenc.Npue(path)
    err = ctypes.create_string_buffer(512)
    assert ref.ref_npue_open(path.encode(), err, 512) == -1
    assert "runs past the data segment" in err.value.decode()


@pytest.mark.parametrize("raw,why", [
    (b'{"config":{"k":"a\\qb"},"tensors":[]}', "unknown escape"),
    (b'{"config":{"k":"a\\ud83d"},"tensors":[]}', "surrogate"),
    (b'{"config":{"k":"abc},"tensors":[]}', "expected"),
    (b'{"config":{"k":1,},"tensors":[]}', "directory byte"),
])
def test_reader_refuses_malformed_directories(tmp_path, raw, why):
    path, _ = _malformed(tmp_path, "dir.npue", raw_json=raw)
    with pytest.raises(mxenc.MxError, match=why):
        mxenc.Npue(path)


def test_missing_file_is_refused_by_name(tmp_path):
    with pytest.raises(mxenc.MxError, match="cannot open"):
        mxenc.Npue(str(tmp_path / "nope.npue"))


# ---- int4 storage over the int8 datapath (common/int4_panel.hpp) --------------------

I4_CASES = [  # (K, N, tile_k, tile_n, mac_s, mac_t, int4_group)
    (128, 96, 64, 48, 8, 4, 32),
    (128, 96, 64, 48, 8, 4, 0),    # one group over the whole K
    (96, 64, 32, 32, 4, 8, 24),    # groups straddle mac_s runs: per-row group index
    (64, 128, 64, 64, 8, 8, 7),    # a group size no tiling divides; ceil(K/g) rows
    (16, 24, 8, 8, 2, 4, 16),
]


def _i4_operand(K, N, group, seed):
    """int4 values over the full [-8, 7] range and a gscale with exact
    half-integer products (1.5, 2.5: ties for rint to break to even) beside
    random ones, some large enough to clip at +-127."""
    rng = np.random.default_rng(seed)
    t = rng.integers(-8, 8, (K, N)).astype(np.int8)
    G = -(-K // (group or K))
    gs = rng.uniform(0.5, 20.0, (G, N)).astype(np.float32)
    gs[:, ::3] = 1.5
    gs[:, 1::7] = 2.5
    gs[:, 2::11] = 40.0  # |t| * 40 > 127 for |t| >= 4: clipped
    return t, gs


def _fold_i4_numpy(t, gs, group):
    """The packer's arithmetic (tools/lib/npue.py fold_i4, :394-430) on the
    logical [K, N] panel: clip(rint(t * gscale[k // g]), -127, 127)."""
    K = t.shape[0]
    row = np.arange(K) // int(group or K)
    return np.clip(np.rint(t.astype(np.float32) * gs[row, :]), -127, 127).astype(np.int8)


def test_i4_nibble_order_hand_worked(orc):
    """Two bytes, four values: element 0 in byte 0's low nibble, element 1 in
    its high nibble; 0xF is -1 and 0x8 is -8 after sign extension."""
    packed = np.array([0x8F, 0x71], np.uint8)  # elements -1, -8, 1, 7
    out = np.zeros(4, np.int8)
    gs = np.ones((1, 2), np.float32)  # [2, 2] operand, one group, one 2 x 2 tile of 1 x 2
    assert orc.orc_widen_i4_panel(P(packed), 2, 2, 2, 2, 1, 2, P(gs), 0, P(out)) == 0
    assert list(out) == [-1, -8, 1, 7]
    assert list(nw.pack_i4(np.array([-1, -8, 1, 7], np.int8))) == [0x8F, 0x71]


@pytest.mark.parametrize("K,N,tk,tn,s,t,group", I4_CASES)
def test_widen_i4_matches_reference_gemm_b_panel(tmp_path, orc, ref, K, N, tk, tn, s, t, group):
    """The reference's npue::gemm_b_panel widens the I4 operand of a written
    container; the oracle widens the same stored bytes: identical int8 runs,
    and equal to the packer's fold of the logical panel, tiled."""
    tv, gs = _i4_operand(K, N, group, K * N + group)
    c = nw.Container({"arch": "bert_abs_gelu_postln", "int4_group": group})
    c.add_gemm_i4("layer.0.qkv", tv, np.ones(N, np.float32), gs, np.ones(K, np.float32),
                  tk, tn, s, t)
    path = str(tmp_path / "i4.npue")
    c.write(path)
    want = np.zeros(K * N, np.int8)
    err = ctypes.create_string_buffer(512)
    n = ref.ref_npue_gemm_b_panel(path.encode(), b"layer.0.qkv", 1, P(want), want.size, err, 512)
    assert n == K * N, err.value
    stored = np.frombuffer(mxenc.Npue(path).bytes("layer.0.qkv"), np.uint8)
    assert stored.size == K * N // 2
    mine = np.zeros(K * N, np.int8)
    assert orc.orc_widen_i4_panel(P(np.ascontiguousarray(stored)), K, N, tk, tn, s, t, P(gs),
                                  group, P(mine)) == 0
    assert np.array_equal(mine, want)
    assert np.array_equal(mine, nw.tile_panel(_fold_i4_numpy(tv, gs, group), tk, tn, s, t))
    # the ties broke to even and the large factors clipped
    assert np.any(np.abs(mine) == 127)


def test_widen_i4_refuses_what_gemm_b_panel_refuses(tmp_path, orc, ref):
    buf = np.zeros(64 * 64, np.uint8)
    gs = np.ones((64, 64), np.float32)
    out = np.zeros(64 * 64, np.int8)
    for args in [(64, 64, 48, 64, 8, 8, 0), (64, 64, 64, 64, 6, 8, 0), (63, 1, 63, 1, 1, 1, 0),
                 (64, 64, 64, 64, 8, 8, -1), (0, 64, 64, 64, 8, 8, 0)]:
        assert orc.orc_widen_i4_panel(P(buf), *args[:6], P(gs), args[6], P(out)) == -1
    # the reference's refusals of an I4 container the loader must also refuse
    tv, g = _i4_operand(64, 32, 32, 5)
    cases = {
        "no int4_group": ({"arch": "x"}, g, "int4_group"),
        "negative group": ({"arch": "x", "int4_group": -2}, g, "must be >= 0"),
        "gscale rows": ({"arch": "x", "int4_group": 16}, g, ".gscale"),
    }
    for what, (cfg, gsc, why) in cases.items():
        c = nw.Container(cfg)
        c.add_gemm_i4("w", tv, np.ones(32, np.float32), gsc, np.ones(64, np.float32),
                      32, 32, 8, 8)
        path = str(tmp_path / "r.npue")
        c.write(path)
        err = ctypes.create_string_buffer(512)
        wbuf = np.zeros(64 * 32, np.int8)
        assert ref.ref_npue_gemm_b_panel(path.encode(), b"w", 1, P(wbuf), wbuf.size, err,
                                         512) == -1, what
        assert why in err.value.decode(), (what, err.value)
