import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def known():
    return json.loads((GOLDEN / "known_answers.json").read_text())


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN / "ref_vectors.npz", allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


@pytest.fixture(scope="session")
def reference():
    from oracle import kernels as K
    if not K.Reference.available():
        pytest.skip("reference library (oracle/_ref) not built here")
    return K.Reference()
