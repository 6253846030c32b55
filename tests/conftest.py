import json
import os
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PKG = ROOT / "streaming-attention_amd"
for p in (str(ROOT), str(PKG), str(ROOT / "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")


def has_gpu() -> bool:
    import torch

    return torch.cuda.is_available()


def pytest_collection_modifyitems(config, items):
    if has_gpu():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


class Golden(dict):
    """npz arrays plus the decoded meta dict."""

    meta: dict


def load_golden(name: str) -> Golden:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        g = Golden({k: z[k] for k in z.files})
    g.meta = json.loads(bytes(g.pop("meta_json")).decode())
    return g


@pytest.fixture
def golden():
    return load_golden
