import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)

# MANTLE_TEST_HIP_LIB: run the CPU tests against another build of libmantle_hip.so from the same
# sources (the host-sanitizer build that tests/sanitize_cpu.py makes); tests only.
if os.environ.get("MANTLE_TEST_HIP_LIB"):
    from mantle_amd import _lib as _mh_lib

    _mh_lib.LIB_PATH = os.environ["MANTLE_TEST_HIP_LIB"]


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP path")
