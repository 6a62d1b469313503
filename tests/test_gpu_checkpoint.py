"""Packed checkpoint files through the GPU (C ABI).

  * pack_checkpoint (quantize.py's main with q8_quantize_pack) writes the
    bytes quantize.py writes for the same bf16 / f16 / f32 source model: the
    expected file is the oracle's pack_q8 restatement (pinned by the
    reference's golden vectors) saved with the safetensors library's
    save_file, as qwen3_mojo/scripts/quantize.py:46-64 does.  Bit-exact.
  * a model loaded from a packed file (file -> device through pinned
    staging) gives the same logits bits as the same tensors uploaded from
    memory.
"""

import sys

import numpy as np
import pytest

from lama32_mojo_amd import checkpoint as ck
from oracle.q8_oracle import bf16_bits_to_f32, f32_to_bf16_bits, pack_q8_np, synth_weights_bf16

sys.path.insert(0, __file__.rsplit("/", 1)[0])
from test_gpu_layers import gpu_model, say  # noqa: E402
from test_model_oracle import tiny_model  # noqa: E402

pytestmark = pytest.mark.gpu


def source_model(torch):
    """A small mixed-dtype model as quantize.py would read it."""
    rng = np.random.default_rng(7)
    bits_a = synth_weights_bf16(16, 128, 1, 0.05)
    bits_b = synth_weights_bf16(24, 64, 2, 1e-3)
    c = (0.3 * rng.standard_normal((8, 256))).astype(np.float32)
    d = (0.7 * rng.standard_normal((4, 64))).astype(np.float16)
    norm = f32_to_bf16_bits((1 + 0.1 * rng.standard_normal(64)).astype(np.float32))
    bias = rng.standard_normal(7).astype(np.float32)
    t = {"model.layers.0.a.weight": torch.from_numpy(bits_a.view(np.int16)).view(torch.bfloat16),
         "model.layers.0.b.weight": torch.from_numpy(bits_b.view(np.int16)).view(torch.bfloat16),
         "model.c.weight": torch.from_numpy(c), "model.d.weight": torch.from_numpy(d),
         "model.norm.weight": torch.from_numpy(norm.view(np.int16)).view(torch.bfloat16),
         "model.bias": torch.from_numpy(bias)}
    f32 = {"model.layers.0.a.weight": bf16_bits_to_f32(bits_a),
           "model.layers.0.b.weight": bf16_bits_to_f32(bits_b),
           "model.c.weight": c, "model.d.weight": d.astype(np.float32)}
    return t, f32


def test_pack_checkpoint_writes_quantize_py_bytes(ctx, tmp_path):
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file as torch_save
    say("pack_checkpoint")
    src_t, f32 = source_model(torch)
    src = tmp_path / "model.safetensors"
    torch_save(src_t, str(src))
    out = tmp_path / "q8.safetensors"
    sizes = ck.pack_checkpoint(ctx, str(tmp_path), str(out), 64, "f16")
    want = {}
    for name, t in src_t.items():
        if t.dim() == 2:
            packed = pack_q8_np(f32[name], 64, "f16")
            want[name] = torch.from_numpy(packed.view(np.float16))
        else:
            want[name] = t.to(torch.bfloat16)
    exp = tmp_path / "expected.safetensors"
    torch_save(want, str(exp))
    assert out.read_bytes() == exp.read_bytes()
    assert sizes["raw_bytes"] == sum(t.numel() * 2 for t in src_t.values())
    # G = 32 with f32 scales: the same rows in that layout, and a layout tag
    out32 = tmp_path / "q8_g32.safetensors"
    ck.pack_checkpoint(ctx, str(src), str(out32), 32, "f32")
    with ck.SafeTensors(str(out32)) as st:
        assert ck.checkpoint_layout(st) == (32, "f32")
        for name, v in f32.items():
            assert np.array_equal(st.read(name).view(np.uint16), pack_q8_np(v, 32, "f32"))
        assert np.array_equal(st.read("model.norm.weight"),
                              src_t["model.norm.weight"].view(torch.int16).numpy().view(np.uint16))


@pytest.mark.parametrize("G,scale", [(64, "f16"), (32, "f32")])
def test_model_from_packed_file_equals_in_memory(ctx, tmp_path, G, scale):
    say("model from file", G, scale)
    spec, t, inv = tiny_model(seed=9, G=G, scale=scale)
    path = tmp_path / "tiny.safetensors"
    meta = None if (G, scale) == (64, "f16") else {ck.QUANT_GROUP_KEY: str(G),
                                                     ck.QUANT_SCALE_KEY: scale}
    ck.save_file({n: ck.Raw("F16" if a.ndim == 2 else "BF16", a) for n, a in t.items()},
                 str(path), meta)
    a = gpu_model(ctx, spec, t, 16)
    with ck.SafeTensors(str(path)) as st:
        b = gpu_model(ctx, spec, st, 16)
    try:
        la, lb = a.forward([4, 8, 15]), b.forward([4, 8, 15])
        assert np.all(np.isfinite(la)) and np.array_equal(la, lb)
        assert np.array_equal(a.forward([16]), b.forward([16]))
    finally:
        a.close()
        b.close()
