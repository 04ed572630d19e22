import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run on the GPU box")


@pytest.fixture
def tune(ctx):
    """tune(key, value): a tuning override on the test module's context
    (mh_context_set_tuning), restored to its default after the test."""
    keys = []

    def set_(key, value):
        keys.append(key)
        ctx.set_tuning(key, value)

    yield set_
    for k in keys:
        ctx.set_tuning(k, None)
