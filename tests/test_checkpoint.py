"""Packed checkpoint files on the CPU: the safetensors reader and writer of
libq8hip (q8_st_*, q8_stw_*) against the safetensors library (0.8.0 here,
the writer behind qwen3_mojo/scripts/quantize.py:59-61): byte-identical
files for the same tensors, the same parsed tensors, shards through
model.safetensors.index.json, and clean errors on corrupt headers."""

import json
import os
import struct

import numpy as np
import pytest

from lama32_mojo_amd import checkpoint as ck
from lama32_mojo_amd import q8hip

safetensors_numpy = pytest.importorskip("safetensors.numpy")


def tensors(seed=0):
    rng = np.random.default_rng(seed)
    return {
        "model.layers.0.mlp.down_proj.weight": rng.standard_normal((5, 64)).astype(np.float16),
        "model.norm.weight": rng.standard_normal(16).astype(np.float32),
        "b": rng.integers(-128, 127, (3, 7), dtype=np.int8),
        "a": rng.integers(0, 65535, (4,), dtype=np.uint16),
        "z.empty": np.zeros((0, 4), np.float16),
        "lm_head.weight": rng.standard_normal((2, 3)).astype(np.float64),
        "ids": rng.integers(0, 1 << 40, (3,), dtype=np.int64),
        "mask": rng.integers(0, 2, (6,)).astype(np.bool_),
        "u8": rng.integers(0, 255, (9,), dtype=np.uint8),
        "i32": rng.integers(-5, 5, (2, 2), dtype=np.int32),
    }


def test_writer_bytes_equal_the_safetensors_library(tmp_path):
    t = tensors()
    ours, theirs = tmp_path / "ours.safetensors", tmp_path / "theirs.safetensors"
    ck.save_file(t, str(ours))
    safetensors_numpy.save_file(t, str(theirs))
    assert ours.read_bytes() == theirs.read_bytes()
    # with one metadata entry
    ck.save_file(t, str(ours), metadata={"format": "pt"})
    safetensors_numpy.save_file(t, str(theirs), metadata={"format": "pt"})
    assert ours.read_bytes() == theirs.read_bytes()


def test_writer_bf16_and_f16_order_matches_torch_save_file(tmp_path):
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file as torch_save
    rng = np.random.default_rng(1)
    w = rng.standard_normal((4, 8)).astype(np.float32)
    bits = torch.from_numpy(w).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    f16 = rng.standard_normal((3, 5)).astype(np.float16)
    ours, theirs = tmp_path / "o.safetensors", tmp_path / "t.safetensors"
    ck.save_file({"w": ck.Raw("BF16", bits), "v": f16}, str(ours))
    torch_save({"w": torch.from_numpy(w).to(torch.bfloat16), "v": torch.from_numpy(f16)},
               str(theirs))
    assert ours.read_bytes() == theirs.read_bytes()


def test_reader_parses_library_files(tmp_path):
    t = tensors(2)
    path = tmp_path / "m.safetensors"
    safetensors_numpy.save_file(t, str(path), metadata={"k": "v"})
    with ck.SafeTensors(str(path)) as st:
        assert st.num_tensors() == len(t)
        assert st.metadata == {"k": "v"}
        for name, arr in t.items():
            info = st.get(name)
            assert info.shape == list(arr.shape)
            assert info.nbytes() == arr.nbytes
            assert info.path == str(path)
            assert np.array_equal(st.read(name), arr)
        assert not st.has("nope")
        # header order is the library's: dtype descending, then name
        order = [i.name for i in st.infos]
        raw = path.read_bytes()
        n = struct.unpack("<Q", raw[:8])[0]
        assert order == [k for k in json.loads(raw[8:8 + n]) if k != "__metadata__"]


def test_directory_with_shard_index(tmp_path):
    a = {"x.weight": np.arange(6, dtype=np.float32).reshape(2, 3)}
    b = {"y.weight": np.ones((2,), np.float16), "w.weight": np.zeros((1, 1), np.int8)}
    safetensors_numpy.save_file(a, str(tmp_path / "model-00002-of-00002.safetensors"))
    safetensors_numpy.save_file(b, str(tmp_path / "model-00001-of-00002.safetensors"))
    idx = {"metadata": {"total_size": 0},
           "weight_map": {"y.weight": "model-00001-of-00002.safetensors",
                          "x.weight": "model-00002-of-00002.safetensors",
                          "w.weight": "model-00001-of-00002.safetensors"}}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(idx))
    with ck.SafeTensors(str(tmp_path)) as st:
        # shard order: first appearance in weight_map; header order inside
        assert [i.name for i in st.infos] == ["y.weight", "w.weight", "x.weight"]
        assert st.get("x.weight").path.endswith("model-00002-of-00002.safetensors")
        assert np.array_equal(st.read("x.weight"), a["x.weight"])
    # no index: the one model.safetensors
    d = tmp_path / "single"
    d.mkdir()
    safetensors_numpy.save_file(a, str(d / "model.safetensors"))
    with ck.SafeTensors(str(d)) as st:
        assert [i.name for i in st.infos] == ["x.weight"]


def corrupt(tmp_path, header: bytes, payload: bytes = b"", length=None):
    p = tmp_path / "bad.safetensors"
    n = len(header) if length is None else length
    p.write_bytes(struct.pack("<Q", n) + header + payload)
    return str(p)


@pytest.mark.parametrize("case", ["short", "len", "json", "nodtype", "dtype", "past_end",
                                  "size", "shape", "offsets", "dup_meta"])
def test_corrupt_headers_fail_cleanly(tmp_path, case):
    good = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    hdr = {"short": None, "len": None, "json": b'{"a": {',
           "nodtype": {"a": {"shape": [2], "data_offsets": [0, 8]}},
           "dtype": {"a": dict(good, dtype="Q7")},
           "past_end": {"a": dict(good, data_offsets=[0, 8])},
           "size": {"a": dict(good, data_offsets=[0, 4])},
           "shape": {"a": dict(good, shape=[-2])},
           "offsets": {"a": dict(good, data_offsets=[8, 0])},
           "dup_meta": {"__metadata__": {"k": 3}, "a": good}}[case]
    if case == "short":
        p = tmp_path / "bad.safetensors"
        p.write_bytes(b"\x01\x02")
        path = str(p)
    elif case == "len":
        path = corrupt(tmp_path, b"{}", length=1 << 40)
    elif isinstance(hdr, bytes):
        path = corrupt(tmp_path, hdr)
    else:
        payload = b"" if case == "past_end" else b"\0" * 8
        path = corrupt(tmp_path, json.dumps(hdr).encode(), payload)
    with pytest.raises(q8hip.Q8Error) as ei:
        ck.SafeTensors(path)
    assert ei.value.code in (q8hip.Q8_ERR_SHAPE, q8hip.Q8_ERR_UNSUPPORTED, q8hip.Q8_ERR_ARG)
    assert ei.value.msg


def test_json_escapes_and_unicode_names(tmp_path):
    t = {'we"ird\\name\né中': np.ones(2, np.float32), "tab\tname": np.zeros(1, np.int8)}
    ours, theirs = tmp_path / "o.safetensors", tmp_path / "t.safetensors"
    ck.save_file(t, str(ours))
    safetensors_numpy.save_file(t, str(theirs))
    assert ours.read_bytes() == theirs.read_bytes()
    with ck.SafeTensors(str(ours)) as st:
        assert sorted(i.name for i in st.infos) == sorted(t)


def test_writer_errors(tmp_path):
    w = ck.Writer(str(tmp_path / "w.safetensors"), [("a", "F32", [2]), ("b", "I8", [3])])
    with pytest.raises(q8hip.Q8Error):
        w.put("a", np.zeros(3, np.float32))            # wrong size
    w.put("a", np.zeros(2, np.float32))
    with pytest.raises(q8hip.Q8Error):
        w.close()                                       # "b" never written
    with pytest.raises(q8hip.Q8Error):
        ck.Writer(str(tmp_path / "x.safetensors"), [("a", "F32", [2]), ("a", "F32", [2])])
    with pytest.raises(q8hip.Q8Error):
        ck.Writer(str(tmp_path / "x.safetensors"), [("a", "Q9", [2])])


def test_upload_validation_without_a_device(tmp_path):
    path = tmp_path / "m.safetensors"
    safetensors_numpy.save_file({"a": np.ones(8, np.float32)}, str(path))
    ctx = q8hip.Context(q8hip.Q8_DEVICE_NONE)
    try:
        buf = ctx.alloc(64)
        with ck.SafeTensors(str(path)) as st:
            lib = q8hip.lib()
            assert lib.q8_st_upload(ctx.h, st.h, 0, 0, 32, buf.h, 0) == q8hip.Q8_ERR_NODEVICE
            assert lib.q8_st_upload(ctx.h, st.h, 0, 0, 33, buf.h, 0) == q8hip.Q8_ERR_RANGE
            assert lib.q8_st_upload(ctx.h, st.h, 0, 0, 32, buf.h, 40) == q8hip.Q8_ERR_RANGE
            assert lib.q8_st_upload(ctx.h, st.h, 1, 0, 32, buf.h, 0) == q8hip.Q8_ERR_ARG
    finally:
        ctx.close()


def test_bf16_conversion_matches_torch():
    """Non-NaN values: torch's round to nearest even, bit for bit.  NaN gives
    a quiet bf16 NaN (torch itself gives 0xFFFF on its vector path and 0x7FC0
    on its scalar path)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    f = np.concatenate([rng.standard_normal(1000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 1000),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.3895314e38, 1e-45],
                                 np.float32)]).astype(np.float32)
    info = ck.TensorInfo("n", "F32", [f.size], "", 0, 4 * f.size)
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = ck._to_bf16_bits(info, f)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7F80) == 0x7F80) and np.all(got[nan] & 0x7F)


def test_model_rejects_mismatched_checkpoint(tmp_path):
    """Q8Llama checks a packed file's layout, names and shapes before any
    device work (so this runs on a host-only context)."""
    from lama32_mojo_amd import model as gm
    cfg = gm.Config(64, 1, 2, 1, 32, 128, 50, 1e-5, 500000.0, 32.0, 1.0, 4.0, 8192.0,
                    tied=True, name="t")

    def write(path, bad=None, meta=None, drop=None):
        t = {}
        for name, sh in gm.tensor_shapes(cfg).items():
            if name == drop:
                continue
            if len(sh) == 2:
                n = sh[0] + (1 if name == bad else 0)
                t[name] = ck.Raw("F16", np.zeros((n, q8hip.rowstride_u16(sh[1])), np.uint16))
            else:
                t[name] = ck.Raw("BF16", np.zeros(sh, np.uint16))
        ck.save_file(t, str(path), meta)

    ctx = q8hip.Context(q8hip.Q8_DEVICE_NONE)
    try:
        cases = [("shape", dict(bad="model.embed_tokens.weight"), ValueError),
                 ("layout", dict(meta={ck.QUANT_GROUP_KEY: "32", ck.QUANT_SCALE_KEY: "f32"}),
                  ValueError),
                 ("missing", dict(drop="model.norm.weight"), KeyError)]
        for tag, kw, exc in cases:
            p = tmp_path / f"{tag}.safetensors"
            write(p, **kw)
            with ck.SafeTensors(str(p)) as st, pytest.raises(exc):
                gm.Q8Llama(ctx, cfg, 8, 64, "f16", weights=st)
    finally:
        ctx.close()


def test_read_of_a_file_cut_after_open_fails_at_once(tmp_path):
    """A file that ends inside a tensor (cut short after its header was
    read) is not a failure that can pass: the read fails on its first
    attempt, without the retries of a transient read error
    (src/resident.mojo:41-54 retries every failed read 15 times, 2 s apart;
    here only I/O errors, timeouts, stale handles and busy resources are
    retried)."""
    import time
    path = tmp_path / "m.safetensors"
    safetensors_numpy.save_file({"a": np.arange(64, dtype=np.float32)}, str(path))
    with ck.SafeTensors(str(path)) as st:
        assert np.array_equal(st.read("a"), np.arange(64, dtype=np.float32))
        with open(path, "r+b") as f:
            f.truncate(os.path.getsize(path) - 100)
        t0 = time.perf_counter()
        with pytest.raises(q8hip.Q8Error) as ei:
            st.read("a")
        assert time.perf_counter() - t0 < 1.0
        assert "ends inside the tensor" in ei.value.msg and "1 attempt" in ei.value.msg
