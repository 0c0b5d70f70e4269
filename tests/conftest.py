"""Shared test setup: the `gpu` marker, the package loader and golden data."""
import importlib.util
import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def load_package():
    """Import three-llm_amd/ (a directory name Python cannot spell) as `three_llm_amd`."""
    if "three_llm_amd" in sys.modules:
        return sys.modules["three_llm_amd"]
    pkg_dir = ROOT / "three-llm_amd"
    spec = importlib.util.spec_from_file_location("three_llm_amd", pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["three_llm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")


@pytest.fixture(scope="session")
def hf_fixture():
    with open(GOLDEN / "transformers-llama.json") as f:
        return json.load(f)
