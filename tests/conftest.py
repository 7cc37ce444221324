"""Shared fixtures. GPU tests are marked `gpu` and need a visible MI355X; the rest run on CPU."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_unconfigure(config):
    # a process still alive 60 s after the test session ended (stuck while exiting) prints every thread's Python stack
    # to stderr, so that the place it waits in is on record
    import faulthandler
    faulthandler.dump_traceback_later(60, exit=False, file=sys.__stderr__)


@pytest.fixture(scope="session")
def plugin():
    from ryft_amd import pjrt
    return pjrt.load_plugin()


@pytest.fixture(scope="session")
def compile_client(plugin):
    """A client that compiles programs to plans without touching a GPU."""
    return plugin.client({"compile_only": True})


@pytest.fixture(scope="session")
def gpu_client(plugin):
    c = plugin.client({"visible_devices": [0]})
    yield c
