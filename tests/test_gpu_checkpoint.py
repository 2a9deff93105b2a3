"""safetensors checkpoint -> GPU quantizer -> on-disk format -> dequant-matmul."""

import numpy as np
import pytest

from oracle import quant_ref as ref

pytestmark = pytest.mark.gpu

lq = pytest.importorskip("locomp_amd")


def _write_checkpoint(path):
    import torch
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(0)
    t = {
        "model.layers.0.self_attn.q_proj.weight": torch.randn(576, 576, generator=g).to(torch.bfloat16),
        "model.layers.0.mlp.down_proj.weight": (0.02 * torch.randn(576, 1536, generator=g)).to(torch.float16),
        "model.layers.0.mlp.up_proj.weight": torch.randn(1536, 576, generator=g),
        "model.norm.weight": torch.ones(576),
        "model.embed_tokens.weight": torch.randn(100, 30, generator=g),   # K % 32 != 0: skipped
    }
    save_file(t, str(path))
    return {k: v.to(torch.float32).numpy() for k, v in t.items()}


def test_quantize_checkpoint_matches_reference_producer(tmp_path):
    src = tmp_path / "model.safetensors"
    w = _write_checkpoint(src)
    layers = lq.quantize_checkpoint(src, group_size=32, scale_dtype=np.float32)
    assert set(layers) == {"model.layers.0.self_attn.q_proj.weight",
                           "model.layers.0.mlp.down_proj.weight", "model.layers.0.mlp.up_proj.weight"}
    for name, layer in layers.items():
        p, s = ref.quantize_int4(w[name], 32)
        assert np.array_equal(layer.qweight.numpy(), p)
        assert np.array_equal(layer.scales.numpy().view(np.uint32), s.view(np.uint32))


def test_packed_file_round_trip_and_matvec(tmp_path):
    src = tmp_path / "model.safetensors"
    w = _write_checkpoint(src)
    layers = lq.quantize_checkpoint(src, group_size=32, scale_dtype=np.float16)
    dst = tmp_path / "model.int4.safetensors"
    lq.save_packed(dst, layers)
    back = lq.load_packed(dst)
    rng = np.random.default_rng(1)
    for name, layer in back.items():
        p, s = ref.quantize_int4(w[name], 32)
        assert np.array_equal(layer.qweight.numpy(), p)
        assert np.array_equal(layer.scales.numpy().view(np.uint16), s.astype(np.float16).view(np.uint16))
        x = rng.standard_normal((4, layer.K)).astype(np.float16)
        y = layer(x).astype(np.float32)
        want = ref.fast_numpy_matvec_int4(x, p, s.astype(np.float16), 32)
        np.testing.assert_allclose(y, want, rtol=1e-2, atol=1e-2 * max(1.0, float(np.abs(want).max()) / 100))


def test_default_scales_are_float32_and_fp16_overflow_is_an_error(tmp_path):
    import torch
    from safetensors.torch import save_file
    src = tmp_path / "m.safetensors"
    w = torch.zeros(64, 64)
    w[0, :32] = 1e6          # group amax 1e6 -> scale 1.4e5: beyond fp16
    w[1, :32] = 1e-12        # scale 1.4e-13: zero in fp16
    w[2:] = torch.randn(62, 64)
    save_file({"l.weight": w}, str(src))
    layers = lq.quantize_checkpoint(src, group_size=32)
    p, s = ref.quantize_int4(w.numpy(), 32)
    assert layers["l.weight"].scales.numpy().dtype == np.float32
    assert np.array_equal(layers["l.weight"].scales.numpy().view(np.uint32), s.view(np.uint32))
    with pytest.raises(ValueError, match="float16"):
        lq.quantize_checkpoint(src, group_size=32, scale_dtype=np.float16)
