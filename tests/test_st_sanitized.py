"""CPU: the safetensors reader (csrc/st_reader.cpp, host code) built with
AddressSanitizer and UndefinedBehaviorSanitizer and run over a corpus of
valid files, a sharded directory and crafted or mutated headers (the
reference keeps ubsan targets per suite, Makefile:224-229). Every path must
open cleanly or be refused with an error, every read must either succeed
into a buffer of the reported size or be refused, and the sanitizers must
report nothing.
"""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "apus-qwen3.6-35b-a3b_amd", "csrc")
HERE = os.path.join(ROOT, "tests", "st_fuzz")
CXX = "/opt/rocm/llvm/bin/clang++"


def _build(tmp):
    flags = ["-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
             "-fno-sanitize-recover=undefined", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
             "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
    objs = []
    for src, lang in ((os.path.join(CSRC, "st_reader.cpp"), "c++"),
                      (os.path.join(CSRC, "apus_rt.cpp"), "c++"),
                      (os.path.join(HERE, "st_stubs.cpp"), "c++"),
                      (os.path.join(HERE, "st_drv.c"), "c")):
        o = os.path.join(tmp, os.path.basename(src) + ".o")
        subprocess.run([CXX] + flags + ["-x", lang, "-c", src, "-o", o], check=True,
                       capture_output=True)
        objs.append(o)
    exe = os.path.join(tmp, "st_drv")
    subprocess.run([CXX, "-fsanitize=address,undefined"] + objs +
                   ["-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-o", exe],
                   check=True, capture_output=True)
    return exe


def _st(path, header, payload=b"", hlen=None):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h) if hlen is None else hlen) + h + payload)


def _corpus(d, rng):
    paths = []
    good = {"a": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 12]},
            "b": {"dtype": "F32", "shape": [4], "data_offsets": [12, 28]},
            "__metadata__": {"format": "pt"}}
    p = os.path.join(d, "good.st")
    _st(p, good, bytes(range(28)))
    paths.append(p)
    crafted = {
        "neg_dim": {"a": {"dtype": "BF16", "shape": [-2, 3], "data_offsets": [0, 12]}},
        "float_dim": {"a": {"dtype": "BF16", "shape": [2.5, 3], "data_offsets": [0, 12]}},
        "huge_dim": {"a": {"dtype": "BF16", "shape": [2 ** 62, 2 ** 62], "data_offsets": [0, 12]}},
        "big_offsets": {"a": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [2 ** 63, 2 ** 64]}},
        "swapped": {"a": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [12, 0]}},
        "past_end": {"a": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 1 << 20]}},
        "size_mismatch": {"a": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 10]}},
        "bad_dtype": {"a": {"dtype": "Q4", "shape": [2, 3], "data_offsets": [0, 12]}},
        "not_object": [1, 2, 3],
        "nine_dims": {"a": {"dtype": "BF16", "shape": [1] * 9, "data_offsets": [0, 2]}},
        "long_name": {"x" * 5000: {"dtype": "BF16", "shape": [1], "data_offsets": [0, 2]}},
        "missing_fields": {"a": {"dtype": "BF16"}},
    }
    for name, hdr in crafted.items():
        p = os.path.join(d, name + ".st")
        _st(p, hdr, bytes(32))
        paths.append(p)
    raw = {
        "deep": b"[" * 5000 + b"]" * 5000,
        "bad_escape": b'{"a\\u12": 1}',
        "unterminated": b'{"a": {"dtype": "BF16", "shape": [2',
        "empty": b"",
        "nul": b'{"a\x00": 1}',
        "num_junk": b'{"a": {"dtype": "BF16", "shape": [1e999], "data_offsets": [0, 2]}}',
    }
    for name, hdr in raw.items():
        p = os.path.join(d, name + ".st")
        _st(p, hdr, bytes(16))
        paths.append(p)
    # header length past the file, and a file shorter than the length word
    p = os.path.join(d, "hlen_past.st")
    _st(p, good, bytes(28), hlen=10 ** 6)
    paths.append(p)
    p = os.path.join(d, "short.st")
    with open(p, "wb") as f:
        f.write(b"\x01\x02")
    paths.append(p)
    # random single-byte mutations of the valid header
    base = open(os.path.join(d, "good.st"), "rb").read()
    for i in range(60):
        b = bytearray(base)
        for _ in range(int(rng.integers(1, 4))):
            b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
        p = os.path.join(d, f"mut{i}.st")
        with open(p, "wb") as f:
            f.write(bytes(b))
        paths.append(p)
    # a sharded directory, and one whose index names a missing shard
    sd = os.path.join(d, "sharded")
    os.makedirs(sd)
    _st(os.path.join(sd, "s1.safetensors"), {"a": good["a"]}, bytes(12))
    _st(os.path.join(sd, "s2.safetensors"), {"b": {"dtype": "F32", "shape": [4],
                                                   "data_offsets": [0, 16]}}, bytes(16))
    with open(os.path.join(sd, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": {"a": "s1.safetensors", "b": "s2.safetensors"}}, f)
    paths.append(sd)
    bd = os.path.join(d, "badindex")
    os.makedirs(bd)
    with open(os.path.join(bd, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": {"a": "../good.st", "b": "nope.safetensors"}}, f)
    paths.append(bd)
    return paths


def test_reader_under_sanitizers(tmp_path):
    if not os.path.exists(CXX):
        pytest.skip("clang++ not found")
    tmp = str(tmp_path)
    try:
        exe = _build(tmp)
    except subprocess.CalledProcessError as e:
        pytest.skip(f"sanitizer build unavailable: {e.stderr.decode()[-300:]}")
    d = os.path.join(tmp, "corpus")
    os.makedirs(d)
    paths = _corpus(d, np.random.default_rng(5))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe] + paths + ["--", "a", "b", "x" * 5000], capture_output=True,
                       text=True, env=env, timeout=120)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-3000:]
    assert "Sanitizer" not in out and "runtime error" not in out, out[-3000:]
    lines = {l.split(" -> ")[0]: l for l in r.stdout.splitlines() if " -> " in l}
    assert lines[os.path.join(d, "good.st")].endswith("-> 0 (2 reads)"), lines
    assert lines[os.path.join(d, "sharded")].endswith("-> 0 (2 reads)"), lines
    for name in ("neg_dim", "float_dim", "huge_dim", "big_offsets", "swapped", "past_end",
                 "size_mismatch", "deep", "hlen_past", "short", "badindex"):
        key = os.path.join(d, name) if name == "badindex" else os.path.join(d, name + ".st")
        assert " -> 0 " not in lines[key], lines[key]
