"""Test configuration: import paths and the `gpu` marker.

CPU tests (-m "not gpu") pin the oracle against the reference's fixtures and brute force, test the host symbolic
analysis and check that libpathpack_hip.so loads and exports its ABI.  GPU tests (-m gpu) compare the HIP path with
the oracle through the C ABI.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("pathpack.jl_amd", "oracle", os.path.join("tests", "golden")):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")
