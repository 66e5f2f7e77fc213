"""Writes golden_vectors.safetensors: for every case in cases.py, its seeded
inputs ("<case>/in/<name>") and the CPU oracle's outputs ("<case>/out/<name>").

    python tests/golden/make_golden.py

Run it again only when a case or the oracle changes on purpose; the fixture
file is committed and tests/test_golden.py reads it.
"""
from __future__ import annotations

import os
import sys
import zlib

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
for p in (REPO, HERE):
    if p not in sys.path:
        sys.path.insert(0, p)

from cases import CASES  # noqa: E402

PATH = os.path.join(HERE, "golden_vectors.safetensors")


def seed_of(name: str) -> int:
    return zlib.crc32(name.encode())


def build_all():
    torch.set_num_threads(1)
    tensors = {}
    for name, c in CASES.items():
        g = torch.Generator().manual_seed(seed_of(name))
        inp = c.inputs(g)
        out = c.oracle({k: v.clone() for k, v in inp.items()})
        for k, v in inp.items():
            tensors[f"{name}/in/{k}"] = v.contiguous()
        for k, v in out.items():
            tensors[f"{name}/out/{k}"] = v.contiguous()
    return tensors


if __name__ == "__main__":
    t = build_all()
    save_file(t, PATH, metadata={"generator": "tests/golden/make_golden.py"})
    print(f"{PATH}: {len(t)} tensors, {os.path.getsize(PATH)} bytes")
