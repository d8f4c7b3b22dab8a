import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


def pytest_sessionstart(session):
    try:
        import pyoracle

        pyoracle.lib.orc_set_threads(min(8, os.cpu_count() or 1))
    except Exception:
        pass
