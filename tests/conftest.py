import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def plan():
    """Planner overrides for one test (awq_set_plan_override), cleared before and after it."""
    from sglite_amd import ops

    class _Plan:
        def set(self, knob, value):
            ops.set_plan_override(knob, int(value))

    ops.clear_plan_overrides()
    yield _Plan()
    ops.clear_plan_overrides()
