"""ctypes binding of the oracle (oracle/_build/liborc.so) and of
oracle/_ref/libref.so, for the tests, smoke() and bench.py's CPU baseline.

The oracle is the checker, never the thing measured as the product."""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORC_SO = os.path.join(ROOT, "oracle", "_build", "liborc.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libref.so")

_c_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


def P(a):
    """Raw pointer of a numpy array (None passes NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


class OrcEncoder(ctypes.Structure):
    _fields_ = [("layers", _c_i64), ("hidden", _c_i64), ("heads", _c_i64),
                ("head_dim", _c_i64), ("ffn", _c_i64)] + [
        (n, _vp) for n in ("w_qkv", "b_qkv", "w_ao", "b_ao", "w_up", "b_up",
                           "w_down", "b_down", "ln1_g", "ln1_b", "ln2_g", "ln2_b",
                           "emb_ln_g", "emb_ln_b", "fin_ln_g", "fin_ln_b")] + [
        ("gated", _c_i64), ("rope_cos", _vp), ("rope_sin", _vp)]


class OrcI8(ctypes.Structure):
    _fields_ = [("wq", _vp * 4), ("wscale", _vp * 4), ("ias", _vp * 4)]


_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(ORC_SO):
        subprocess.check_call(["make", "-s", "-C", os.path.join(ROOT, "oracle")])
    lib = ctypes.CDLL(ORC_SO)
    sig = {
        "orc_set_threads": (None, [ctypes.c_int]),
        "orc_lane_begin": (ctypes.c_int, [ctypes.c_int]),
        "orc_lane_end": (None, []),
        "orc_threads": (ctypes.c_int, []),
        "orc_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_from_bf16": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_bf16_fill": (None, [_vp, _vp, ctypes.c_size_t]),
        "orc_round_bf16_inplace": (None, [_vp, ctypes.c_size_t]),
        "orc_gelu8": (ctypes.c_float, [ctypes.c_float]),
        "orc_gelu_poly_inplace": (None, [_vp, ctypes.c_size_t]),
        "orc_gelu_erf_exact": (ctypes.c_float, [ctypes.c_float]),
        "orc_gelu_erf_inplace": (None, [_vp, ctypes.c_size_t]),
        "orc_exp2_poly": (None, [_vp, _vp, ctypes.c_size_t]),
        "orc_softmax_rows_poly": (None, [_vp, _c_i64, _c_i64, _vp, _c_i64]),
        "orc_softmax_rows_exact": (None, [_vp, _c_i64, _c_i64, _vp, _c_i64]),
        "orc_layer_norm_rows": (None, [_vp, _c_i64, _c_i64, _vp, _vp, ctypes.c_float]),
        "orc_layernorm_rows_f64": (None, [_vp, _c_i64, _c_i64, _vp, _vp, ctypes.c_double]),
        "orc_add_into": (None, [_vp, _vp, _vp, ctypes.c_size_t]),
        "orc_gemm_nt": (None, [_vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp]),
        "orc_qk": (None, [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp]),
        "orc_av": (None, [_vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp]),
        "orc_whisper_attention": (None, [_vp, _c_i64, _vp, _c_i64, _c_i64, _c_i64,
                                         _c_i64, _c_i64, _c_i64, ctypes.c_float, _vp]),
        "orc_embed_sum": (None, [_vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _vp]),
        "orc_pool_rows": (ctypes.c_int, [_vp, _vp, _c_i64, _c_i64, _c_i64, ctypes.c_int,
                                         ctypes.c_int, _vp]),
        "orc_aie_softmax_bf16": (None, [_vp, _vp, _c_i64, _c_i64]),
        "orc_aie_layernorm_bf16": (None, [_vp, _vp, _c_i64, _c_i64, _vp, _vp, ctypes.c_float]),
        "orc_aie_gelu_erf_bf16": (None, [_vp, _vp, _c_i64]),
        "orc_aie_gelu_poly_bf16": (None, [_vp, _vp, _c_i64]),
        "orc_narrow_f32_bf16": (None, [_vp, _vp, _c_i64]),
        "orc_narrow_i32_bf16": (None, [_vp, _vp, _c_i64]),
        "orc_narrow_i32_bf16_twice": (None, [_vp, _vp, _c_i64]),
        "orc_bert_run": (None, [ctypes.POINTER(OrcEncoder), _vp, _vp, _c_i64, _c_i64, _c_i64]),
        "orc_preln_run": (None, [ctypes.POINTER(OrcEncoder), _vp, _c_i64, _c_i64,
                                 ctypes.c_double, ctypes.c_float, _c_i64]),
        "orc_conv_front_end": (None, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _c_i64, _vp]),
        "orc_vit_patches": (None, [_vp, _c_i64, _c_i64, _vp]),
        "orc_head_matvec": (None, [_vp, _vp, _vp, _c_i64, _c_i64, _vp]),
        "orc_untile_b_panel": (ctypes.c_int, [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                              _c_i64, _vp]),
        "orc_widen_i4_panel": (ctypes.c_int, [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                              _c_i64, _vp, _c_i64, _vp]),
        "orc_quantise_a_int8": (None, [_vp, _c_i64, _c_i64, _vp, _vp, _vp]),
        "orc_gemm_i8": (None, [_vp, _c_i64, _c_i64, _vp, _c_i64, _vp]),
        "orc_dequantise_c": (None, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp]),
        "orc_gemm_i8_dequant": (None, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp, _c_i64, _vp]),
        "orc_bert_run_i8": (None, [ctypes.POINTER(OrcEncoder), ctypes.POINTER(OrcI8), _vp, _vp,
                                   _c_i64, _c_i64, _c_i64]),
        "orc_rope_tables": (None, [_c_i64, _c_i64, ctypes.c_double, _vp, _vp, _vp]),
        "orc_rope_qkv": (None, [_vp, _c_i64, _c_i64, _c_i64, _c_i64, _vp, _vp]),
        "orc_glu": (None, [_vp, _c_i64, _c_i64, ctypes.c_int, _vp]),
        "orc_dequantise_c_bf16": (None, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp]),
        "orc_bias_c_bf16": (None, [_vp, _c_i64, _c_i64, _vp, _vp]),
        "orc_dequant_act_bf16": (None, [_vp, _c_i64, _c_i64, ctypes.c_int, _vp, _vp]),
        "orc_set_array_arith": (ctypes.c_int, [ctypes.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def load_ref():
    if not os.path.exists(REF_SO):
        return None
    lib = ctypes.CDLL(REF_SO)
    sig = {
        "ref_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
        "ref_bf16_fill_bits": (None, [ctypes.c_uint32, ctypes.c_uint64, _vp]),
        "ref_bf16_fill": (None, [_vp, _vp, ctypes.c_size_t]),
        "ref_gelu8_scalar": (ctypes.c_float, [ctypes.c_float]),
        "ref_gelu8_avx2": (None, [_vp, _vp, ctypes.c_size_t]),
        "ref_exp2_avx2": (None, [_vp, _vp, ctypes.c_size_t]),
        "ref_hsum8": (ctypes.c_float, [_vp]),
        "ref_gemm_nt": (None, [_vp, _c_i64, _vp, _c_i64, _c_i64, _vp, _vp, ctypes.c_int]),
        "ref_quantise_a_int8": (None, [_vp, _c_i64, _c_i64, _vp, _vp, _vp]),
        "ref_dequantise_c": (ctypes.c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp]),
        "ref_dequantise_c_bf16": (ctypes.c_int, [_vp, _c_i64, _c_i64, _vp, _vp, _vp, _vp]),
        "ref_npue_host_b_kn": (ctypes.c_longlong, [ctypes.c_char_p, ctypes.c_char_p, _vp,
                                                   ctypes.c_longlong, ctypes.c_char_p,
                                                   ctypes.c_size_t]),
        "ref_npue_gemm_b_panel": (ctypes.c_longlong, [ctypes.c_char_p, ctypes.c_char_p,
                                                      ctypes.c_longlong, _vp, ctypes.c_longlong,
                                                      ctypes.c_char_p, ctypes.c_size_t]),
        "ref_npue_config": (ctypes.c_longlong, [ctypes.c_char_p, ctypes.c_char_p,
                                                ctypes.c_char_p, ctypes.c_size_t,
                                                ctypes.c_char_p, ctypes.c_size_t]),
        "ref_npue_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]),
        "ref_npue_tensor": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                                           _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]),
        "ref_gemma_rope_tables": (None, [_c_i64, _c_i64, ctypes.c_double, _vp, _vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


ORC_ARR_A_BF16, ORC_ARR_C_BF16, ORC_ARR_ATTN_BF16 = 1, 2, 4


class array_arith:
    """Context manager: the oracle's whole-stack restatements run with the
    array datapath's arithmetic bits (orc_set_array_arith) set."""

    def __init__(self, flags):
        self.flags = flags

    def __enter__(self):
        self.prev = load().orc_set_array_arith(self.flags)
        return self

    def __exit__(self, *exc):
        load().orc_set_array_arith(self.prev)


def bf16_round(x):
    """Round fp32 to the nearest bf16 (the reference's to_bf16), kept as fp32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.astype(np.uint32).view(np.float32)


def encoder_struct(m, keep):
    """OrcEncoder over the numpy arrays of a synthetic model dict; `keep`
    collects the arrays so they outlive the call."""
    s = OrcEncoder()
    s.layers, s.hidden, s.heads, s.head_dim, s.ffn = (
        m["layers"], m["hidden"], m["heads"], m["head_dim"], m["ffn"])
    for n in ("w_qkv", "b_qkv", "w_ao", "b_ao", "w_up", "b_up", "w_down", "b_down",
              "ln1_g", "ln1_b", "ln2_g", "ln2_b", "emb_ln_g", "emb_ln_b", "fin_ln_g",
              "fin_ln_b"):
        a = m.get(n)
        if a is None:
            setattr(s, n, None)
        else:
            a = np.ascontiguousarray(a, dtype=np.float32)
            keep.append(a)
            setattr(s, n, a.ctypes.data)
    s.gated = int(m.get("gated", 0))
    if m.get("rope"):
        # tables for every position the model has; a run indexes rows s < S
        n_pos, hd = int(m.get("max_pos", 512)), m["head_dim"]
        c = np.empty((n_pos, hd), np.float32)
        sn = np.empty((n_pos, hd), np.float32)
        inv = m.get("rope_inv_freq")
        inv = None if inv is None else np.ascontiguousarray(inv, np.float32)
        load().orc_rope_tables(n_pos, hd, float(m.get("rope_theta", 0.0)),
                               None if inv is None else inv.ctypes.data, P(c), P(sn))
        keep += [c, sn] + ([inv] if inv is not None else [])
        s.rope_cos, s.rope_sin = c.ctypes.data, sn.ctypes.data
    return s


def aligned_empty(shape, dtype, align=64):
    """An uninitialised array whose data starts on an `align`-byte boundary."""
    dtype = np.dtype(dtype)
    n = int(np.prod(shape)) * dtype.itemsize
    raw = np.empty(n + align, np.uint8)
    off = (-raw.ctypes.data) % align
    return raw[off:off + n].view(dtype).reshape(shape)


def quantise_weights(w_kn, asmooth=None):
    """The packer's int8 operand scheme (tools/lib/gemm_i8.py:21-90), as the
    synthetic-model generator implements it."""
    from mxenc import synth
    return synth.quantise_weights(w_kn, asmooth)
