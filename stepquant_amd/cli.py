"""Command-line helpers the serving adapter imports (reference stepquant/cli.py).

Only ``fingerprint`` (cli.py:12-18) and ``save`` (cli.py:21-24) are on the
serving path: a plan artifact records the fingerprint of the checkpoint it
was calibrated on, and the adapter refuses a plan whose fingerprint differs.
Calibration and evaluation commands are outside this build.
"""
import hashlib
from pathlib import Path

import torch


def fingerprint(path):
    """SHA-256 over the bytes of ``config.json`` then
    ``model.safetensors.index.json`` of a checkpoint directory (files that do
    not exist are skipped; an empty directory gives the digest of nothing)."""
    root = Path(path)
    digest = hashlib.sha256()
    for name in ("config.json", "model.safetensors.index.json"):
        part = root / name
        if part.exists():
            digest.update(part.read_bytes())
    return digest.hexdigest()


def save(value, path):
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    torch.save(value, path)
