"""Drafter directory reading and writing (woodcock_amd/weights.py) on the CPU:
python/woodcock/drafter.py:310-330 (strict load), export.py:1-64 (manifest),
src/core/weights.cpp:64-122 (BF16 / F16 / F32 tensors, every .safetensors of
the directory)."""
import json

import pytest
import torch

from woodcock_amd.config import DrafterConfig
from woodcock_amd.synthetic import random_drafter
from woodcock_amd.weights import read_drafter_dir, write_drafter_dir


def _cfg():
    return DrafterConfig(hidden_size=64, num_layers=1, num_heads=2, num_kv_heads=1, head_dim=32,
                         intermediate_size=96, vocab_size=300, target_hidden_size=48, feature_layers=[2, 4, 5])


def test_round_trip_bit_exact(tmp_path):
    cfg = _cfg()
    w = random_drafter(cfg, seed=1)
    write_drafter_dir(tmp_path, cfg, w, target_name="Qwen/Qwen3-1.7B")
    cfg2, w2, man = read_drafter_dir(tmp_path)
    assert cfg2 == cfg
    assert set(w2) == set(w)
    for k in w:
        assert w2[k].dtype == torch.bfloat16 and torch.equal(w2[k].view(torch.int16), w[k].view(torch.int16))
    assert man["format"] == "woodcock-drafter" and man["version"] == 1
    assert man["target"]["name"] == "Qwen/Qwen3-1.7B"
    assert man["weights"]["num_params"] == sum(v.numel() for v in w.values())


def test_float32_and_float16_tensors_round_to_bf16(tmp_path):
    from safetensors.torch import save_file

    cfg = _cfg()
    w = random_drafter(cfg, seed=2)
    f32 = {k: v.float() + (1e-3 if v.dim() == 1 else 0.0) for k, v in w.items()}
    f32["fc.weight"] = f32["fc.weight"].half()
    cfg.save(tmp_path / "config.json")
    save_file(f32, str(tmp_path / "model.safetensors"))
    _, w2, man = read_drafter_dir(tmp_path)
    assert man is None
    for k, v in f32.items():
        assert torch.equal(w2[k].view(torch.int16), v.to(torch.bfloat16).view(torch.int16))


def test_weights_split_over_files(tmp_path):
    from safetensors.torch import save_file

    cfg = _cfg()
    w = random_drafter(cfg, seed=3)
    keys = sorted(w)
    cfg.save(tmp_path / "config.json")
    save_file({k: w[k] for k in keys[:5]}, str(tmp_path / "a.safetensors"))
    save_file({k: w[k] for k in keys[5:]}, str(tmp_path / "b.safetensors"))
    _, w2, _ = read_drafter_dir(tmp_path)
    assert set(w2) == set(w)


@pytest.mark.parametrize("case", ["missing", "extra", "shape"])
def test_strict_tensor_set(tmp_path, case):
    from safetensors.torch import save_file

    cfg = _cfg()
    w = random_drafter(cfg, seed=4)
    if case == "missing":
        del w["norm.weight"]
    elif case == "extra":
        w["layers.0.lowrank.weight"] = torch.zeros(4, 4, dtype=torch.bfloat16)
    else:
        w["fc.weight"] = w["fc.weight"][:, :-1].contiguous()
    cfg.save(tmp_path / "config.json")
    save_file(w, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError):
        read_drafter_dir(tmp_path)


@pytest.mark.parametrize("field,value", [("format", "other"), ("version", 2), ("sha256", "0" * 64),
                                         ("target_hidden", 49), ("num_layers", 2)])
def test_manifest_mismatches_are_rejected(tmp_path, field, value):
    cfg = _cfg()
    write_drafter_dir(tmp_path, cfg, random_drafter(cfg, seed=5))
    mf = tmp_path / "woodcock.json"
    m = json.loads(mf.read_text())
    if field in ("format", "version"):
        m[field] = value
    elif field == "sha256":
        m["weights"]["sha256"] = value
    elif field == "target_hidden":
        m["target"]["hidden_size"] = value
    else:
        m["drafter"]["num_layers"] = value
    mf.write_text(json.dumps(m))
    with pytest.raises(ValueError):
        read_drafter_dir(tmp_path)
    if field == "sha256":
        read_drafter_dir(tmp_path, verify_sha=False)  # the caller may skip hashing


def test_legacy_config_rejected_and_missing_files(tmp_path):
    cfg = _cfg()
    write_drafter_dir(tmp_path, cfg, random_drafter(cfg, seed=6))
    d = json.loads((tmp_path / "config.json").read_text())
    d["lowrank_rank"] = 8
    (tmp_path / "config.json").write_text(json.dumps(d))
    with pytest.raises(ValueError):
        read_drafter_dir(tmp_path)
    with pytest.raises(ValueError):
        read_drafter_dir(tmp_path / "absent")
