"""The device-layer tests of test_host_device.py, run on the MI355X.

test_host_device.py runs them over the host stand-in of the kernel library
where there is no GPU; collected here with the `gpu` mark they run the same
checks on the real gfx950 library (routing, autocast, OOM retry, pickling,
fused linear, cat/stack, the amsgrad state checks)."""

import pytest

from test_host_device import *  # noqa: F401,F403  (re-collect every test function here)

pytestmark = pytest.mark.gpu
