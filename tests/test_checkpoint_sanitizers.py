"""The safetensors reader and writer (host code of libq8hip,
lama32_mojo_amd/csrc/q8_safetensors.cpp) built on the CPU with g++ under
AddressSanitizer and UndefinedBehaviorSanitizer, driven by
tests/sanitize/st_driver.cpp over: files written by the safetensors library
(every dtype, metadata, empty tensors), a sharded directory, the corrupt
headers of test_checkpoint.py, its own writer's output, and seeded
mutations of a valid file (header bytes, JSON structure, length prefix,
truncation).  Any out-of-bounds access, leak or undefined behaviour aborts
the driver, so each run must exit 0 with no sanitizer report.  Headers are
untrusted input: this is the reader's parse (src/safetensors.mojo:64-87)
under the tools that find what its bounds checks miss."""

import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

safetensors_numpy = pytest.importorskip("safetensors.numpy")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all",
             "-fno-omit-frame-pointer"]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    assert gxx, "g++ is needed for the sanitizer build"
    out = str(tmp_path_factory.mktemp("san") / "st_driver")
    cmd = [gxx, "-std=c++17", "-g", "-O1", *SAN_FLAGS,
           os.path.join(ROOT, "tests", "sanitize", "st_driver.cpp"),
           os.path.join(ROOT, "lama32_mojo_amd", "csrc", "q8_safetensors.cpp"),
           "-I", os.path.join(ROOT, "include"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    return out


def run(driver, *args):
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:abort_on_error=0:exitcode=97"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1:exitcode=98"
    r = subprocess.run([driver, *map(str, args)], capture_output=True, text=True, timeout=300,
                       env=env)
    report = r.stderr
    assert "Sanitizer" not in report and "runtime error" not in report, report[-4000:]
    assert r.returncode == 0, (r.returncode, report[-4000:])


def library_files(tmp_path):
    rng = np.random.default_rng(3)
    t = {"w": rng.standard_normal((5, 64)).astype(np.float16),
         "n": rng.standard_normal(16).astype(np.float32),
         "c": rng.integers(-128, 127, (3, 7), dtype=np.int8),
         "e": np.zeros((0, 4), np.float16),
         "d": rng.standard_normal((2, 3)).astype(np.float64),
         "i": rng.integers(0, 1 << 40, (3,), dtype=np.int64),
         "m": rng.integers(0, 2, (6,)).astype(np.bool_),
         "u": rng.integers(0, 65535, (4,), dtype=np.uint16)}
    one = tmp_path / "one.safetensors"
    safetensors_numpy.save_file(t, str(one), metadata={"format": "pt", "q8": "G64"})
    shard = tmp_path / "sharded"
    shard.mkdir()
    safetensors_numpy.save_file({"x": t["w"]}, str(shard / "model-00001-of-00002.safetensors"))
    safetensors_numpy.save_file({"y": t["n"]}, str(shard / "model-00002-of-00002.safetensors"))
    (shard / "model.safetensors.index.json").write_text(json.dumps(
        {"metadata": {}, "weight_map": {"x": "model-00001-of-00002.safetensors",
                                        "y": "model-00002-of-00002.safetensors"}}))
    return [one, shard]


def corrupt_files(tmp_path):
    good = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    cases = {"json": b'{"a": {', "nodtype": {"a": {"shape": [2], "data_offsets": [0, 8]}},
             "dtype": {"a": dict(good, dtype="Q7")},
             "past_end": {"a": dict(good, data_offsets=[0, 16])},
             "size": {"a": dict(good, data_offsets=[0, 4])},
             "shape": {"a": dict(good, shape=[-2])},
             "huge_shape": {"a": dict(good, shape=[1 << 40, 1 << 40])},
             "offsets": {"a": dict(good, data_offsets=[8, 0])},
             "dup_meta": {"__metadata__": {"k": 3}, "a": good},
             "deep": b"[" * 5000 + b"]" * 5000,
             "escape": b'{"a\\u12": {}}', "nul": b'{"a\x00": 1}'}
    out = []
    for name, hdr in cases.items():
        body = hdr if isinstance(hdr, bytes) else json.dumps(hdr).encode()
        p = tmp_path / f"bad_{name}.safetensors"
        p.write_bytes(struct.pack("<Q", len(body)) + body + b"\0" * 8)
        out.append(p)
    short = tmp_path / "bad_short.safetensors"
    short.write_bytes(b"\x01\x02")
    out.append(short)
    big = tmp_path / "bad_len.safetensors"
    big.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    out.append(big)
    return out


def test_reader_on_library_files_and_shards(driver, tmp_path):
    run(driver, "read", *library_files(tmp_path))


def test_reader_on_corrupt_headers(driver, tmp_path):
    run(driver, "read", *corrupt_files(tmp_path))


def test_writer_then_reader(driver, tmp_path):
    run(driver, "write", tmp_path / "w.safetensors")


@pytest.mark.parametrize("seed", [1, 2])
def test_reader_on_mutated_headers(driver, tmp_path, seed):
    one = library_files(tmp_path)[0]
    run(driver, "fuzz", one, seed, 3000)
