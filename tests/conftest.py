"""Shared fixtures: the product package (loaded by path: its directory name
has a dot) and the oracle wrapper (test infrastructure)."""
import importlib.util
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def _load(name, path):
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def load_pkg():
    return _load("llamanyon_rs_amd", os.path.join(REPO, "llamanyon.rs_amd", "__init__.py"))


def load_oracle():
    return _load("swamp_oracle_py", os.path.join(REPO, "oracle", "oracle.py"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X / gfx950)")


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def orc():
    return load_oracle()


@pytest.fixture(scope="session")
def fixtures():
    import json
    with open(os.path.join(REPO, "tests", "golden", "fixtures.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def errlog():
    """record(case, err): print the normalized error a parity case reached
    and, when SWAMP_PARITY_LOG names a file, append it there as one JSON
    line, so the precision of each path is visible from run to run."""
    import json
    path = os.environ.get("SWAMP_PARITY_LOG")

    def record(case, err, **extra):
        print(f"[parity] {case}: max normalized error {err:.3e}", flush=True)
        if path:
            with open(path, "a") as f:
                f.write(json.dumps(dict(case=case, err=float(err), **extra)) + "\n")
        return err

    return record
