import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def lib():
    from lazyweights_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from lazyweights_amd import build
        build.build()
    return _lib.load_library()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    if not os.path.exists(oracle.LIB):
        oracle.build()
    return oracle


def golden_cases():
    out = []
    for f in sorted(os.listdir(GOLDEN)):
        if f.endswith(".npz") and f != "huffman_lengths.npz":
            out.append(f[:-4])
    return out


def load_golden(name):
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
