"""Shared fixtures: the product package (hyphenated directory name), the
CPU oracle (test infrastructure) and GPU gating."""
from __future__ import annotations

import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
ORACLE_DIR = os.path.join(ROOT, "oracle")
if ORACLE_DIR not in sys.path:
    sys.path.insert(0, ORACLE_DIR)

PKG_NAME = "micro-expert-router-ssd-streamed-moe-mer_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) GPU")


def load_pkg():
    return importlib.import_module(PKG_NAME)


@pytest.fixture(scope="session")
def mer():
    return load_pkg()


@pytest.fixture(scope="session")
def oracle():
    import mer_oracle

    mer_oracle.lib()
    return mer_oracle


@pytest.fixture(scope="session")
def gpu(mer):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    mer.init(0)
    return torch.device("cuda", 0)
