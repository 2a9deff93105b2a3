"""The quantized on-disk format (host side: no GPU needed)."""

import numpy as np
import pytest

from locomp_amd import checkpoint as ck
from oracle import quant_ref as ref


def test_save_read_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    layers = {}
    for name, (N, K) in {"model.layers.0.mlp.up_proj": (96, 64), "lm_head": (40, 128)}.items():
        w = rng.standard_normal((N, K)).astype(np.float32)
        p, s = ref.quantize_int4(w, 32)
        layers[name] = (p, s.astype(np.float16))
    f = tmp_path / "q.safetensors"
    ck.save_packed(f, layers)
    back, gs = ck.read_packed(f)
    assert gs == 32 and set(back) == set(layers)
    for n, (p, s) in layers.items():
        assert np.array_equal(back[n][0], p) and back[n][0].dtype == np.uint8
        assert np.array_equal(back[n][1].view(np.uint16), s.view(np.uint16))


def test_read_rejects_other_files(tmp_path):
    from safetensors.numpy import save_file
    f = tmp_path / "plain.safetensors"
    save_file({"w": np.zeros((2, 2), np.float32)}, str(f))
    with pytest.raises(ValueError):
        ck.read_packed(f)
    g = tmp_path / "bad.safetensors"
    save_file({"a.qweight": np.zeros((4, 8), np.uint8), "a.scales": np.zeros((4, 3), np.float16)},
              str(g), metadata={"format": ck.FORMAT, "group_size": "32"})
    with pytest.raises(ValueError):
        ck.read_packed(g)


def test_save_rejects_mixed_groups(tmp_path):
    a = (np.zeros((2, 16), np.uint8), np.zeros((2, 1), np.float16))   # G = 32
    b = (np.zeros((2, 16), np.uint8), np.zeros((2, 2), np.float16))   # G = 16
    with pytest.raises(ValueError):
        ck.save_packed(tmp_path / "x.safetensors", {"a": a, "b": b})


def test_default_selection():
    sel = ck._default_select(32)
    assert sel("model.layers.0.self_attn.q_proj.weight", (576, 576))
    assert not sel("model.norm.weight", (576,))
    assert not sel("model.layers.0.mlp.down_proj.weight", (576, 1500))   # K % 32 != 0
    assert not sel("model.embed_tokens.bias", (10, 64))
