import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    oracle_so = os.path.join(ROOT, "oracle", "liboracle_pbmoe.so")
    if not os.path.exists(oracle_so):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def pytest_collection_modifyitems(config, items):
    # GPU tests run only where a GPU is present; they are selected with -m gpu
    pass
