"""The C ABI without a GPU: the library loads, exports every function
include/mx_encoder.h declares, and the placement registry behaves like the
reference's --npu-ops parser (npu_ops_flag.hpp:75-268)."""
import ctypes
import os
import re

import pytest

import mxenc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(mxenc.LIB_PATH):
        import importlib.util
        spec = importlib.util.spec_from_file_location(
            "mx_build", os.path.join(ROOT, "npu-embeddings-xdna1_amd", "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return mxenc.lib()


def declared_functions():
    text = open(os.path.join(ROOT, "include", "mx_encoder.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_function(L):
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the Python binding describes each one
    assert sorted(mxenc.SIGNATURES) == names


def test_version_and_codes(L):
    assert L.mx_version() == 1
    assert L.mx_op_codes().decode() == "gemm, gelu, layn, softm, conv, attn, mproj, fft, logit"


def test_ops_parse_like_the_reference(L):
    assert L.mx_ops_parse(b" gemm ,attn,, softm,layn , gelu,") == 0
    for c in (b"gemm", b"attn", b"softm", b"layn", b"gelu"):
        assert L.mx_op_on_gpu(c) == 1
    assert L.mx_op_on_gpu(b"conv") == 0
    # an unknown code is refused by name and leaves the previous set in place
    rc = L.mx_ops_parse(b"gemm,flash")
    assert rc == mxenc.MX_OK - 1
    msg = L.mx_last_error().decode()
    assert "'flash'" in msg and "gemm, gelu, layn" in msg
    assert L.mx_op_on_gpu(b"attn") == 1
    # replacing, not merging: the last list wins
    assert L.mx_ops_parse(b"gemm") == 0
    assert L.mx_op_on_gpu(b"gemm") == 1 and L.mx_op_on_gpu(b"attn") == 0
    assert L.mx_ops_parse(b"") == 0
    assert L.mx_op_on_gpu(b"gemm") == 0


@pytest.mark.parametrize("flag,hint", [("--npu-eltwise", "gelu,layn,softm"),
                                       ("--host-ln", "without layn"),
                                       ("--npu-extra-ops", "--npu-ops")])
def test_removed_flags_refused(L, flag, hint):
    assert L.mx_ops_check_flag(flag.encode()) == -1
    assert hint in L.mx_last_error().decode()
    assert L.mx_ops_check_flag(b"--npu-ops") == 0


def test_static_scratch_guard_refuses_an_overlap(L):
    """The per-GPU guard mx_encoder_embed_static holds for its whole call, taken
    here as a call would take it: a second holder on the same device is refused
    by name (that is the overlap refusal), other devices are independent, and
    releasing makes it available again. Host-only: no GPU, no timing."""
    assert L.mx_static_guard_hold(3) == mxenc.MX_OK
    assert L.mx_static_guard_hold(3) == mxenc.MX_E_STATE
    msg = L.mx_last_error().decode()
    assert "device 3" in msg and "in use by another call" in msg
    assert L.mx_static_guard_hold(4) == mxenc.MX_OK  # another GPU's scratch
    assert L.mx_static_guard_release(3) == mxenc.MX_OK
    assert L.mx_static_guard_release(3) == mxenc.MX_E_STATE  # not held any more
    assert "not held" in L.mx_last_error().decode()
    assert L.mx_static_guard_hold(3) == mxenc.MX_OK
    for dev in (3, 4):
        assert L.mx_static_guard_release(dev) == mxenc.MX_OK
    assert L.mx_static_guard_hold(-1) == -1


def test_device_allocation_count_starts_at_zero_without_a_device(L):
    """Nothing has allocated device memory in a process without a GPU."""
    assert L.mx_device_allocations() == 0


def test_null_arguments_refused_without_a_device(L):
    assert L.mx_create(0, None) == -1
    assert "null" in L.mx_last_error().decode()
    assert L.mx_gemm_wt(None, None, 1, 8, 8, None, 8, None, 0, None, None, 0, 8) == -1
    assert L.mx_attention(None, None, 0, 1, 1, 1, 64, 1.0, None, None, None, 64) == -1
    assert L.mx_softmax_rows(None, None, 0, 1, 1, 1, None, 1, 0) == -1
    assert L.mx_encoder_create(None, None, None) == -1
    for fn in ("mx_encoder_embed", "mx_encoder_embed_async", "mx_encoder_embed_static"):
        assert getattr(L, fn)(None, None, None, None, 1, 1, None) == -1, fn
        err = L.mx_last_error().decode()
        assert "null" in err and fn[3:] in err, (fn, err)
    assert L.mx_sync(None) == -1 and "null stream" in L.mx_last_error().decode()


def test_no_silent_cpu_fallback(L):
    """Without a GPU the context cannot open: there is no host path to fall to."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r); import mxenc, ctypes; "
            "h = ctypes.c_void_p(); rc = mxenc.lib().mx_create(0, ctypes.byref(h)); "
            "print(rc, mxenc.lib().mx_last_error().decode())"
            % os.path.join(ROOT, "npu-embeddings-xdna1_amd"))
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env,
                       timeout=120)
    rc = int(r.stdout.split()[0])
    assert rc != 0


def test_gemm_rows_beyond_32bit_offsets_leave_the_lds_kernel(L):
    """The LDS-pipelined GEMM addresses a tile's rows by 32-bit byte offsets
    (row < 256 times lda or K, times the element size). A bf16 call whose
    lda or K reaches 2^23 elements goes to the register-staged kernel (64-bit
    indexing); an int8 call whose lda or K reaches 2^24 is refused by name
    before anything is launched."""
    plan = lambda K: L.mx_gemm_plan_for(1024, 1024, K, mxenc.MX_BF16, 0, 0).decode()  # noqa: E731
    assert plan((1 << 23) - 64).startswith("lds_")
    assert plan(1 << 23).startswith("staged_")
    # (s, A, a_scale, M, K, lda, Wt, wscale, N, bias, epilogue, residual, C, c_dtype, ldc)
    args = [None, None, None, 1024, 1024, 1 << 24, None, None, 1024, None, 0, None, None,
            mxenc.MX_BF16, 1024]
    assert L.mx_gemm_i8_wt(*args) == -3
    msg = L.mx_last_error().decode()
    assert "32-bit byte offsets" in msg and "2^24" in msg
    args[5] = 1024  # in range: the next refusal is the missing stream
    assert L.mx_gemm_i8_wt(*args) == -1 and "null stream" in L.mx_last_error().decode()


def test_cxx_caller_refusal_paths(tmp_path):
    """A C++17 program built by the host compiler against include/
    (mx_gpu_backend.hpp over mx_encoder.h) and linked to the library runs the
    registry, reader and null-argument refusals through the wrapper, each as
    std::runtime_error("gpu: ...") naming its reason; and reads a container's
    config through the wrapper, a value longer than its first buffer included."""
    import subprocess

    import npue_writer as nw
    from mxenc import synth
    exe = os.path.join(os.path.dirname(mxenc.LIB_PATH), "abi_check")
    assert os.path.exists(exe), "build() builds the C++ caller beside the library"
    r = subprocess.run([exe, "cpu"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "cpu ok", r.stdout + r.stderr
    m = synth.make_model("minilm", layers=1, hidden=64, heads=2, head_dim=32, ffn=128, vocab=64,
                         max_pos=16)
    note = "n" * 3000
    path = str(tmp_path / "m.npue")
    nw.bert_container(m, 32, 32, (8, 8), extra_config={"note": note}).write(path)
    for key, value in (("arch", "bert_abs_gelu_postln"), ("note", note), ("hidden", "64")):
        r = subprocess.run([exe, "cpu", path, key, value], capture_output=True, text=True,
                           timeout=60)
        assert r.returncode == 0 and r.stdout.strip() == "cpu ok", (key, r.stdout + r.stderr)
    r = subprocess.run([exe, "cpu", path, "hidden", "65"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 1 and "config value" in r.stdout
