"""Status codes that need a device: allocation failure and a failed HIP call."""
from __future__ import annotations

import ctypes as C

import pytest

from qm38 import QmError, _check

pytestmark = pytest.mark.gpu


def test_out_of_memory_and_command_failed(rt, torch_dev):
    out = C.c_void_p()
    # 1 PiB: far beyond the card (288 GB), refused by the allocator.
    with pytest.raises(QmError, match="OUT_OF_MEMORY"):
        _check(rt.lib.qm_device_alloc(rt.handle, 1 << 50, C.byref(out)))
    # Freeing an address the allocator never returned: the HIP call fails
    # without touching device memory.
    with pytest.raises(QmError, match="COMMAND_FAILED"):
        _check(rt.lib.qm_device_free(rt.handle, C.c_void_p(0x7F0000001000)))
