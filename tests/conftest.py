"""Shared test set-up.

GPU tests are marked ``gpu``; everything else runs on the CPU container.  The
product package lives in the directory ``paddleocr-vl-webgpu_amd`` (not an
identifier), so it is loaded by path through ``__graft_entry__.load_package``.
"""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for path in (REPO, TESTS):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden():
    import json

    with open(os.path.join(REPO, "tests", "golden", "reference_digests.json")) as f:
        return json.load(f)
