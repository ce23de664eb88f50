"""The host code that reads untrusted input, and the oracle, under
AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

- The .npue reader and its JSON parser (csrc/mx_npue.cpp) and the error state
  and --npu-ops registry (csrc/mx_host.cpp) are compiled with g++
  -fsanitize=address,undefined into tests/abi_cxx/npue_san.cpp's driver,
  which opens a corpus of valid and malformed containers: truncations, every
  header field set to edge values, random byte mutations of the directory,
  deep nesting, tensors past the data, overflowing offsets, bad escapes.
  Each file opens or is refused by name; no sanitizer report.
- The oracle (oracle/*.c) is compiled the same way with
  tests/abi_cxx/oracle_san.c, which runs its ops on small and edge shapes.
"""
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import npue_writer as nw
from mxenc import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "npu-embeddings-xdna1_amd", "csrc")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
           UBSAN_OPTIONS="print_stacktrace=1")


def _have(tool):
    return shutil.which(tool) is not None


def _build(tmp, out, cmd):
    r = subprocess.run(cmd + ["-o", str(tmp / out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return str(tmp / out)


def _corpus(tmp):
    """Valid containers (bf16, int8, int4) and malformed variants of one."""
    files = []
    m = synth.make_model("minilm", layers=1, hidden=64, heads=2, head_dim=32, ffn=128, vocab=64,
                         max_pos=16)
    for name, kw in (("bf16", {}), ("i8", {"int8": synth.quantise_model(m)}),
                     ("i4", {"int4": synth.quantise_model_i4(m, group=32)})):
        p = tmp / f"ok_{name}.npue"
        nw.bert_container(m, 32, 32, (8, 8), **kw).write(str(p))
        files.append(p)
    base = files[0].read_bytes()
    _, _, _, _, jo, jl, do, dl = struct.unpack("<4sIIIQQQQ", base[:48])
    # truncations
    for n in sorted({0, 1, 10, 63, 64, 65, 100, jo + jl - 1, jo + jl, do - 1, do, do + 17,
                     len(base) - 1}):
        p = tmp / f"trunc_{n}.npue"
        p.write_bytes(base[:max(0, n)])
        files.append(p)
    # every 8-byte header field (and the 4-byte ones) at edge values
    edges64 = [0, 1, 63, 64, 4095, 4096, len(base), len(base) + 1, 2**32, 2**63, 2**64 - 1]
    for off in (16, 24, 32, 40):
        for v in edges64:
            b = bytearray(base)
            b[off:off + 8] = struct.pack("<Q", v)
            p = tmp / f"hdr_{off}_{v}.npue"
            p.write_bytes(bytes(b))
            files.append(p)
    for off in (4, 8, 12):
        for v in (0, 2, 2**31, 2**32 - 1):
            b = bytearray(base)
            b[off:off + 4] = struct.pack("<I", v)
            p = tmp / f"hdr4_{off}_{v}.npue"
            p.write_bytes(bytes(b))
            files.append(p)
    # random byte mutations inside the directory
    rng = np.random.default_rng(20260926)
    for k in range(400):
        b = bytearray(base)
        for _ in range(int(rng.integers(1, 4))):
            b[int(rng.integers(jo, jo + jl))] = int(rng.integers(0, 256))
        p = tmp / f"mut_{k}.npue"
        p.write_bytes(bytes(b))
        files.append(p)

    def raw(name, js):
        c = nw.Container({"arch": "bert_abs_gelu_postln"})
        c.add_f32("x", np.ones(4, np.float32), "bias")
        p = tmp / name
        c.write(str(p), raw_json=js)
        files.append(p)

    raw("deep_array.npue", b'{"config":{"k":' + b"[" * 200000 + b"]" * 200000 + b'},"tensors":[]}')
    raw("deep_object.npue", b'{"config":{"k":' + b'{"a":' * 5000 + b"1" + b"}" * 5000 +
        b'},"tensors":[]}')
    raw("deep_open.npue", b"[" * 100000)
    raw("huge_offset.npue", b'{"config":{},"tensors":[{"name":"x","offset":18446744073709551615,'
        b'"nbytes":16}]}')
    raw("wrap_size.npue", b'{"config":{},"tensors":[{"name":"x","offset":8,'
        b'"nbytes":9223372036854775807}]}')
    raw("neg_size.npue", b'{"config":{},"tensors":[{"name":"x","offset":0,"nbytes":-16}]}')
    raw("bigint.npue", b'{"config":{"n":123456789012345678901234567890},"tensors":[{"name":"x",'
        b'"offset":99999999999999999999999,"nbytes":16}]}')
    raw("dup.npue", b'{"config":{},"tensors":[{"name":"x","offset":0,"nbytes":16},'
        b'{"name":"x","offset":0,"nbytes":16}]}')
    raw("noname.npue", b'{"config":{},"tensors":[{"offset":0,"nbytes":16}]}')
    raw("shapes.npue", b'{"config":{},"tensors":[{"name":"x","offset":0,"nbytes":16,'
        b'"padded_shape":[9223372036854775807,-1,0,1,2,3,4,5],"logical_shape":[],'
        b'"layout":{"kind":"block_panel","tile_k":-1,"tile_n":0,"mac_s":1e400,"mac_t":[]}}]}')
    raw("escapes.npue", b'{"config":{"a":"\\ud800","b":"\\udc00x","c":"\\u12","d":"\\x",'
        b'"e":"\x01"},"tensors":[]}')
    raw("unterminated.npue", b'{"config":{"a":"abc')
    raw("empty.npue", b"")
    raw("nul.npue", b'{"config":{"a":"a\x00b"},"tensors":[]}')
    return files


@pytest.mark.skipif(not _have("g++"), reason="needs g++")
def test_npue_reader_and_registry_under_asan_ubsan(tmp_path):
    exe = _build(tmp_path, "npue_san",
                 ["g++", "-std=c++17"] + SAN + ["-I", os.path.join(ROOT, "include"),
                                                os.path.join(ROOT, "tests", "abi_cxx",
                                                             "npue_san.cpp"),
                                                os.path.join(CSRC, "mx_host.cpp"),
                                                os.path.join(CSRC, "mx_npue.cpp")])
    files = _corpus(tmp_path)
    r = subprocess.run([exe] + [str(f) for f in files], capture_output=True, text=True,
                       timeout=300, env=ENV)
    report = r.stdout + r.stderr
    assert r.returncode == 0, report[-4000:]
    assert "Sanitizer" not in report and "runtime error" not in report, report[-4000:]
    opened, refused = (int(x) for x in r.stdout.split()[1::2])
    assert opened + refused == len(files)
    assert opened >= 3 and refused >= 60  # the valid three open; the malformed mostly refused


@pytest.mark.skipif(not _have("gcc"), reason="needs gcc")
def test_oracle_under_asan_ubsan(tmp_path):
    srcs = [os.path.join(ROOT, "oracle", f) for f in
            ("orc_pool.c", "orc_numerics.c", "orc_ops.c", "orc_encoders.c")]
    exe = _build(tmp_path, "oracle_san",
                 ["gcc", "-std=gnu11", "-march=x86-64-v3", "-ffp-contract=off"] + SAN +
                 ["-I", os.path.join(ROOT, "oracle"),
                  os.path.join(ROOT, "tests", "abi_cxx", "oracle_san.c")] + srcs +
                 ["-lm", "-lpthread"])
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=ENV)
    report = r.stdout + r.stderr
    assert r.returncode == 0, report[-4000:]
    assert "Sanitizer" not in report and "runtime error" not in report, report[-4000:]
    assert r.stdout.strip().endswith("oracle ok"), report[-2000:]
