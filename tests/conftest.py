import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
GOLDEN = REPO / "tests" / "golden"
REFERENCE = Path("/root/reference")
for p in (REPO, REPO / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def int_models():
    from sigcomp_amd import model_io
    return {name: model_io.load_int_model(getattr(model_io, f"DEFAULT_QUANT_{name.upper()}_MODEL_PATH"))
            for name in ("lossless", "lossy")}


@pytest.fixture(scope="session")
def oracle_models(int_models, oracle_mod):
    return {k: oracle_mod.OracleModel(m) for k, m in int_models.items()}
