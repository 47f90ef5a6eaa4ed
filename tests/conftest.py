import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "meta-work_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: full-size model runs")


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return str(tmp_path_factory.mktemp("models"))


def synth_model(model_dir, cfg, name):
    import xjpipe as xp
    path = os.path.join(model_dir, name + ".gguf")
    if not os.path.exists(path):
        xp.write_model(path, cfg)
    return path


@pytest.fixture(scope="session")
def tiny_path(model_dir):
    import xjpipe as xp
    return synth_model(model_dir, xp.TINY, "tiny")


@pytest.fixture(scope="session")
def tiny_draft_path(model_dir):
    import xjpipe as xp
    return synth_model(model_dir, xp.TINY_DRAFT, "tiny_draft")
