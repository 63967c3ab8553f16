"""The graft entry's smoke() (one small call of each hot-path kernel checked
against the oracle) must pass as part of the GPU suite."""

import pytest

pytestmark = pytest.mark.gpu


def test_graft_smoke(dev):
    import __graft_entry__

    __graft_entry__.smoke()
