"""pytest configuration: the `gpu` marker and shared helpers.

`-m "not gpu"` runs the oracle, host-logic and ABI-export tests on any
machine; `-m gpu` runs the HIP parity tests on an MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def flush_print(*args):
    print(*args, flush=True)
