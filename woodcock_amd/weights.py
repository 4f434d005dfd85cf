"""Drafter weight files on local paths: the reference's drafter directory.

    <dir>/
      woodcock.json       manifest (optional): format, version, mode, target, drafter, tensor table, sha256
      config.json         DrafterConfig (legacy fields checked, config.py)
      model.safetensors   weights, names as in python/woodcock/drafter.py

Follows Drafter.save / Drafter.load (python/woodcock/drafter.py:310-330: a
strict load, every parameter present and nothing else), the export manifest
(python/woodcock/export.py:1-64) and the native reader's tensor handling
(src/core/weights.cpp:64-122: every *.safetensors of the directory, BF16 / F16 /
F32 tensors).  Weights are returned as bf16 CPU tensors (F16 / F32 rounded to
nearest even, the reference's `dtype` cast at load).  Nothing is fetched by
name: a missing file is an error.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import torch

from .config import DrafterConfig
from .synthetic import weight_shapes

FORMAT = "woodcock-drafter"
VERSION = 1
MODE = "woodcock-v1"
WEIGHTS_FILE = "model.safetensors"
_DTYPES = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def _sha256(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 24), b""):
            h.update(block)
    return h.hexdigest()


def _read_safetensors(files: list[Path]) -> dict[str, torch.Tensor]:
    from safetensors.torch import load_file

    out: dict[str, torch.Tensor] = {}
    for f in files:
        for k, v in load_file(str(f), device="cpu").items():
            if k in out:
                raise ValueError(f"tensor {k} appears in more than one weight file")
            if v.dtype not in _DTYPES:
                raise ValueError(f"unsupported dtype {v.dtype} for {k}")
            out[k] = v
    return out


def check_weights(cfg: DrafterConfig, weights: dict[str, torch.Tensor], where: str = "weights") -> None:
    """Strict: every parameter of the configuration with its shape, nothing else."""
    want = weight_shapes(cfg)
    missing = sorted(set(want) - set(weights))
    extra = sorted(set(weights) - set(want))
    if missing:
        raise ValueError(f"{where}: missing tensors {missing[:4]}{' ...' if len(missing) > 4 else ''}")
    if extra:
        raise ValueError(f"{where}: unexpected tensors {extra[:4]}{' ...' if len(extra) > 4 else ''}")
    for k, shape in want.items():
        if tuple(weights[k].shape) != tuple(shape):
            raise ValueError(f"{where}: {k} has shape {tuple(weights[k].shape)}, expected {tuple(shape)}")


def check_manifest(manifest: dict, cfg: DrafterConfig, weights: dict[str, torch.Tensor], weights_path: Path,
                   verify_sha: bool = True) -> None:
    """The manifest agrees with the configuration and the weight file."""
    if manifest.get("format") != FORMAT:
        raise ValueError(f"woodcock.json: format {manifest.get('format')!r}, expected {FORMAT!r}")
    if manifest.get("version") != VERSION:
        raise ValueError(f"woodcock.json: version {manifest.get('version')!r} is not supported (expected {VERSION})")
    t = manifest.get("target") or {}
    if t.get("hidden_size") != cfg.target_hidden_size or t.get("vocab_size") != cfg.vocab_size:
        raise ValueError("woodcock.json: target hidden size / vocabulary disagree with config.json")
    if t.get("feature_layers") is not None and list(t["feature_layers"]) != list(cfg.feature_layers):
        raise ValueError("woodcock.json: target feature layers disagree with config.json")
    dr = manifest.get("drafter") or {}
    for k in ("hidden_size", "num_layers", "post_norm", "window"):
        if k in dr and dr[k] != getattr(cfg, k):
            raise ValueError(f"woodcock.json: drafter {k} disagrees with config.json")
    w = manifest.get("weights") or {}
    if w.get("file", WEIGHTS_FILE) != weights_path.name:
        raise ValueError(f"woodcock.json: weight file {w.get('file')!r} is not {weights_path.name!r}")
    if verify_sha and w.get("sha256") and w["sha256"] != _sha256(weights_path):
        raise ValueError("woodcock.json: sha256 of the weight file does not match")
    for k, spec in (w.get("tensors") or {}).items():
        if k not in weights or list(weights[k].shape) != list(spec.get("shape", [])):
            raise ValueError(f"woodcock.json: tensor table entry {k} does not match the weight file")


def read_drafter_dir(path, verify_sha: bool = True):
    """(DrafterConfig, {name: bf16 CPU tensor}, manifest or None) from a local drafter directory."""
    p = Path(path)
    if not p.is_dir():
        raise ValueError(f"{p}: not a drafter directory")
    cfg_file = p / "config.json"
    if not cfg_file.is_file():
        raise ValueError(f"{p}: config.json missing")
    cfg = DrafterConfig.load(cfg_file)
    files = sorted(f for f in p.iterdir() if f.suffix == ".safetensors")
    if not files:
        raise ValueError(f"no .safetensors in {p}")
    raw = _read_safetensors(files)
    check_weights(cfg, raw, str(p))
    manifest = None
    mf = p / "woodcock.json"
    if mf.is_file():
        manifest = json.loads(mf.read_text())
        wname = (manifest.get("weights") or {}).get("file", WEIGHTS_FILE)
        check_manifest(manifest, cfg, raw, p / wname, verify_sha)
    weights = {k: (v if v.dtype == torch.bfloat16 else v.to(torch.bfloat16)).contiguous() for k, v in raw.items()}
    return cfg, weights, manifest


def write_drafter_dir(path, cfg: DrafterConfig, weights: dict[str, torch.Tensor], target_name: str | None = None,
                      training: dict | None = None) -> Path:
    """config.json + model.safetensors (bf16) + woodcock.json, as Drafter.save plus the
    export manifest (export.py:27-53)."""
    from safetensors.torch import save_file

    check_weights(cfg, weights, "write_drafter_dir")
    p = Path(path)
    p.mkdir(parents=True, exist_ok=True)
    cfg.save(p / "config.json")
    w = {k: v.detach().to("cpu", torch.bfloat16).contiguous() for k, v in weights.items()}
    wfile = p / WEIGHTS_FILE
    save_file(w, str(wfile), metadata={"format": "woodcock-drafter-v1"})
    manifest = {
        "format": FORMAT,
        "version": VERSION,
        "mode": MODE,
        "target": {"name": target_name, "hidden_size": cfg.target_hidden_size, "vocab_size": cfg.vocab_size,
                   "feature_layers": list(cfg.feature_layers)},
        "drafter": {"hidden_size": cfg.hidden_size, "num_layers": cfg.num_layers, "post_norm": cfg.post_norm,
                    "window": cfg.window},
        "weights": {"file": WEIGHTS_FILE, "sha256": _sha256(wfile), "num_params": sum(v.numel() for v in w.values()),
                    "tensors": {k: {"shape": list(v.shape), "dtype": _DTYPES[v.dtype]} for k, v in w.items()}},
        "training": training,
    }
    (p / "woodcock.json").write_text(json.dumps(manifest, indent=2))
    return p
