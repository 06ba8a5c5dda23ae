import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "system1-omni_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


import pytest  # noqa: E402


@pytest.fixture
def forms():
    """Force GDN prep / scan kernel forms through the library's test hook for one test; the
    shape-based choice is restored afterwards. Call as forms(prep_wide=0, scan_halves=2, ...)."""
    from qwen3_5_native import hip

    state = {"prep_wide": -1, "prep_split": -1, "scan_halves": -1, "scan_osets": -1}

    def force(**kw):
        unknown = set(kw) - set(state)
        if unknown:
            raise TypeError(f"unknown forms {sorted(unknown)}")
        state.update(kw)
        hip.check(hip.api().q35_gdn_force_forms(state["prep_wide"], state["prep_split"], state["scan_halves"],
                                                state["scan_osets"]), "force forms")

    yield force
    hip.check(hip.api().q35_gdn_force_forms(-1, -1, -1, -1), "reset forms")
