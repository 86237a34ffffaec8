"""Shared pytest set-up: the `gpu` marker, the golden fixtures, repo on sys.path."""
import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X; calls the HIP sampler through its C ABI")


def _num(x):
    if isinstance(x, str):
        return float(x)
    return x


def _walk(o):
    if isinstance(o, dict):
        return {k: _walk(v) for k, v in o.items()}
    if isinstance(o, list):
        return [_walk(v) for v in o]
    if isinstance(o, str) and o in ("nan", "inf", "-inf"):
        return float(o)
    return o


@pytest.fixture(scope="session")
def golden():
    with open(os.path.join(ROOT, "tests", "golden", "reference_cases.json")) as f:
        return _walk(json.load(f))


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.build()
    return o


def pytest_sessionstart(session):
    """Build what the tests load if nothing is built yet (the GPU box uses the
    prebuilt files that travel with the tree)."""
    from oracle import oracle as o
    o.build()
    from xwen_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from xwen_amd import build
        build.build()
