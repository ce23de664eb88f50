"""Writes .npue containers for the tests (fixture code, not product).

The container layout is the reference packer's (tools/lib/npue.py: header
struct "<4sIII QQQQ 16s" at :261, writer :790-870, tile_b :491-556,
gemm_b_layout :580-596, layout_hash :777-785), restated here so that the GPU
loader, the oracle and the reference's own reader (oracle/_ref) can be fed the
same file:

  [0, 64)          "NPUE", version 1, arch, flags, json_offset = 64,
                   json_length, data_offset (4096-aligned), data_length,
                   16 zero bytes
  [64, ...)        compact JSON {"config": ..., "tensors": [...]}
  [data_offset..)  each tensor's bytes at its "offset", padded to 4096

A GEMM operand [K, N] is stored as bf16 bits in tiles of tile_k x tile_n in
(k-block, n-block) order, each tile as mac_s x mac_t sub-tiles, row-major
inside.
"""
import hashlib
import json
import struct

import numpy as np

ALIGN = 4096
ARCH_BERT = 0
FLAG_PRETILED = 1


def to_bf16_bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def tile_panel(kn, tile_k, tile_n, mac_s, mac_t):
    """[K, N] -> the container's flat block_panel order (any element dtype).

    Element (k, n) with k = bk*tile_k + r*mac_s + si and n = bn*tile_n +
    c*mac_t + ti goes to position (bk, bn, r, c, si, ti) of the flat run."""
    K, N = kn.shape
    assert K % tile_k == 0 and N % tile_n == 0
    assert tile_k % mac_s == 0 and tile_n % mac_t == 0
    x = kn.reshape(K // tile_k, tile_k // mac_s, mac_s, N // tile_n, tile_n // mac_t, mac_t)
    return np.ascontiguousarray(x.transpose(0, 3, 1, 4, 2, 5)).reshape(-1)


def pack_i4(flat):
    """int4 values (int8 in [-8, 7]) -> bytes, two per byte, even index in the
    low nibble (tools/lib/npue.py:347-374)."""
    f = np.ascontiguousarray(flat, np.int8).reshape(-1)
    assert f.size % 2 == 0
    lo = (f[0::2].astype(np.int16) & 0x0F).astype(np.uint8)
    hi = (f[1::2].astype(np.int16) & 0x0F).astype(np.uint8)
    return (lo | (hi << 4)).astype(np.uint8)


def panel_layout(tile_k, tile_n, mac_s, mac_t, dtype="BF16"):
    return {"kind": "block_panel", "tile_k": tile_k, "tile_n": tile_n, "order": "k,n,kt,nt",
            "inner": "s,t", "mac_s": mac_s, "mac_t": mac_t, "dtype": dtype}


def layout_digest(layout):
    text = json.dumps(layout, sort_keys=True, separators=(",", ":"))
    return hashlib.sha256(text.encode("utf-8")).hexdigest()


class Container:
    """Collects tensors, then writes one .npue file."""

    def __init__(self, config, arch=ARCH_BERT, flags=FLAG_PRETILED):
        self.config = dict(config)
        self.arch, self.flags = arch, flags
        self.entries, self.blobs, self.offset = [], [], 0

    def add(self, name, data, dtype_tag, role, logical_shape, layout=None, padded_shape=None):
        blob = np.ascontiguousarray(data).tobytes()
        entry = {"name": name, "role": role, "dtype": dtype_tag,
                 "logical_shape": [int(v) for v in logical_shape],
                 "padded_shape": [int(v) for v in (padded_shape or logical_shape)],
                 "offset": self.offset, "nbytes": len(blob)}
        if layout is not None:
            entry["layout"] = layout
            entry["layout_hash"] = layout_digest(layout)
        self.entries.append(entry)
        pad = (-len(blob)) % ALIGN
        self.blobs.append(blob + b"\0" * pad)
        self.offset += len(blob) + pad
        return entry

    def add_f32(self, name, arr, role, shape=None):
        a = np.ascontiguousarray(arr, dtype="<f4")
        return self.add(name, a, "F32", role, shape or list(a.shape))

    def add_gemm(self, name, kn, tile_k, tile_n, mac_s, mac_t):
        """A [K, N] operand (fp32 values, rounded to bf16) as a pre-tiled panel."""
        kn = np.asarray(kn, np.float32)
        flat = tile_panel(to_bf16_bits(kn), tile_k, tile_n, mac_s, mac_t)
        return self.add(name, flat, "BF16", "gemm_b", list(kn.shape),
                        layout=panel_layout(tile_k, tile_n, mac_s, mac_t))

    def add_gemm_i8(self, name, q_kn, wscale, asmooth, tile_k, tile_n, mac_s, mac_t):
        """An int8 design's operand (tools/lib/gemm_i8.py:21-90): the [K, N] int8
        panel pre-tiled with an I8 layout, then .wscale [N] and .asmooth [K]."""
        q_kn = np.asarray(q_kn, np.int8)
        K, N = q_kn.shape
        flat = tile_panel(q_kn, tile_k, tile_n, mac_s, mac_t)
        self.add(name, flat, "I8", "gemm_b", [K, N],
                 layout=panel_layout(tile_k, tile_n, mac_s, mac_t, dtype="I8"))
        self.add_f32(name + ".wscale", wscale, "quant_scale")
        self.add_f32(name + ".asmooth", asmooth, "quant_smooth")

    def add_gemm_i4(self, name, t_kn, wscale, gscale, asmooth, tile_k, tile_n, mac_s, mac_t):
        """An --int4 pack's operand (tools/lib/gemm_i4.py:23-140): the int4 values
        t [K, N] in [-8, 7] pre-tiled in the I8 layout's order and packed two per
        byte, low nibble first (tools/lib/npue.py pack_i4, :347-374), as dtype
        "I4"; then .wscale [N], .gscale [G, N] and .asmooth [K]."""
        t_kn = np.asarray(t_kn, np.int8)
        K, N = t_kn.shape
        assert int(t_kn.min(initial=0)) >= -8 and int(t_kn.max(initial=0)) <= 7
        flat = tile_panel(t_kn, tile_k, tile_n, mac_s, mac_t)
        self.add(name, pack_i4(flat), "I4", "gemm_b", [K, N],
                 layout=panel_layout(tile_k, tile_n, mac_s, mac_t, dtype="I8"))
        self.add_f32(name + ".wscale", wscale, "quant_scale")
        self.add_f32(name + ".gscale", gscale, "quant_group")
        self.add_f32(name + ".asmooth", asmooth, "quant_smooth")

    def write(self, path, version=1, magic=b"NPUE", data_align=ALIGN, raw_json=None,
              trailing=b""):
        """raw_json (bytes) replaces the directory; trailing bytes are appended
        after the data (both only to build malformed files for refusal tests)."""
        js = raw_json if raw_json is not None else json.dumps(
            {"config": self.config, "tensors": self.entries},
            separators=(",", ":")).encode("utf-8")
        data_offset = 64 + len(js)
        data_offset += (-data_offset) % data_align
        header = struct.pack("<4sIIIQQQQ16s", magic, version, self.arch, self.flags, 64,
                             len(js), data_offset, self.offset, b"\0" * 16)
        with open(path, "wb") as f:
            f.write(header)
            f.write(js)
            f.write(b"\0" * (data_offset - 64 - len(js)))
            for b in self.blobs:
                f.write(b)
            f.write(trailing)
        return data_offset


def bert_container(m, tile_k=64, tile_n=64, mac=(8, 8), arch="bert_abs_gelu_postln",
                   pooling=None, extra_config=None, int8=None, int4=None, int4_group=32):
    """A BERT container of a synthetic model dict (mxenc.synth.make_model):
    the packer's tensor names, roles and config keys
    (tools/pack/pack_npue.py:2630-2760). int8: the model's int8 operands
    (mxenc.synth.quantise_model) -- the container is then an --int8 pack; int4:
    its int4 operands (mxenc.synth.quantise_model_i4 at int4_group rows per
    group) -- an --int4 pack."""
    d, f, L = m["hidden"], m["ffn"], m["layers"]
    cfg = {"arch": arch, "source_repo": "synthetic/bert", "source_sha256": "0" * 64,
           "num_layers": L, "num_heads": m["heads"], "hidden": d, "head_dim": m["head_dim"],
           "intermediate": f, "layer_norm_eps": 1e-12, "vocab_size": m["vocab"],
           "max_seq_len": m["max_pos"],
           "pooling": pooling or ("cls" if m.get("cls_pool") else "mean"),
           "l2_normalize": True, "activation": "gelu_erf_exact", "gemm_layout": "pretiled_bf16",
           "tile_k": tile_k, "tile_n": tile_n, "mac_s": mac[0], "mac_t": mac[1],
           "a_dtype": "i8" if (int8 or int4) else "bf16",
           "fusions": {"qkv_fused": True, "transposed_to_kn": True,
                       "qk_scale_folded_into_q": True}}
    if m.get("rope"):
        # the RoPE / gated-FFN archs' keys (tools/pack/pack_npue.py; read by
        # app::set_model_shape, app_state.hpp:440-550)
        cfg.update({"position_embedding_type": "rope", "gated_ffn": True})
        if m.get("rope_inv_freq") is not None:
            cfg.update({"glu_halves": "up_first|gate_second (ffn_up = [up | gate])",
                        "rope_inv_freq": [float(v) for v in m["rope_inv_freq"]],
                        "activation": "gelu"})
        else:
            cfg.update({"swiglu_halves": "fc11_up|fc12_gate", "rope_theta": m["rope_theta"],
                        "activation": "silu"})
    if int4:
        cfg["int4_group"] = int4_group
    cfg.update(extra_config or {})
    c = Container(cfg)
    c.add_f32("embeddings.word", m["word"], "embedding")
    c.add_f32("embeddings.position", m["pos"], "embedding")
    c.add_f32("embeddings.token_type", m["type"], "embedding")
    c.add_f32("embeddings.ln.weight", m["emb_ln_g"], "layernorm")
    c.add_f32("embeddings.ln.bias", m["emb_ln_b"], "layernorm")
    names = [("qkv", "w_qkv", "b_qkv"), ("attn_out", "w_ao", "b_ao"),
             ("ffn_up", "w_up", "b_up"), ("ffn_down", "w_down", "b_down")]
    for l in range(L):
        for i, (n, w, b) in enumerate(names):
            if int4:
                t, ws, gs, sm = int4[i]
                c.add_gemm_i4(f"layer.{l}.{n}", t[l], ws[l], gs[l], sm[l], tile_k, tile_n,
                              mac[0], mac[1])
            elif int8:
                q, ws, sm = int8[i]
                c.add_gemm_i8(f"layer.{l}.{n}", q[l], ws[l], sm[l], tile_k, tile_n, mac[0],
                              mac[1])
            else:
                c.add_gemm(f"layer.{l}.{n}", m[w][l], tile_k, tile_n, mac[0], mac[1])
            c.add_f32(f"layer.{l}.{n}.bias", m[b][l], "bias")
        for n, key in (("ln1.weight", "ln1_g"), ("ln1.bias", "ln1_b"),
                       ("ln2.weight", "ln2_g"), ("ln2.bias", "ln2_b")):
            c.add_f32(f"layer.{l}.{n}", m[key][l], "layernorm")
    return c
