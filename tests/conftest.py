"""Shared pytest setup.

* registers the ``gpu`` marker (tests that need an MI355X; run with ``-m gpu``);
* puts the repo root on sys.path so ``oracle`` and ``_pkg`` import;
* exposes ``pkg`` — the product package, whose directory name carries a dash
  and therefore loads through importlib.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def pkg():
    import importlib

    return importlib.import_module("rwkv-megatron_amd")
