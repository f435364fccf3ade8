import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "polarquant-kv_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libpqkv_hip.so on cuda:0)")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def golden_codebooks():
    with open(os.path.join(GOLDEN, "codebooks.json")) as f:
        books = json.load(f)["codebooks"]
    return {k: (np.asarray(v["centroids"], np.float32), np.asarray(v["boundaries"], np.float32))
            for k, v in books.items()}


@pytest.fixture(scope="session")
def golden_R():
    return {d: np.load(os.path.join(GOLDEN, f"R_d{d}_s42.npy")) for d in (64, 128)}


@pytest.fixture(scope="session")
def golden_P():
    out = {}
    for m, d, s in ((64, 64, 43), (128, 128, 43), (64, 128, 42)):
        out[(m, d, s)] = np.load(os.path.join(GOLDEN, f"P_m{m}_d{d}_s{s}.npy"))
    return out
