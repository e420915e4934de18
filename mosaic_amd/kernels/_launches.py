"""Per-module kernel-launch counters with the reference's semantics.

Each reference kernel module keeps ``_LAUNCHES``: its operators add one per
kernel they launch, its MoE entry point resets it to 0 first, and
``last_launch_count()`` returns it (``kernels/skinny_fp4.py:18-22,133,274``,
``kernels/mxint.py:23-34,1460``, ``kernels/qpa_mma.py:40-59,698``,
``kernels/xsimt.py:20-32``, ``kernels/w4a16_grouped.py:12-16,165``).  Here an
operator adds the number of kernels the HIP library launched on this thread
during the call (``mosaic_launch_count``), so the count is the real one."""
from __future__ import annotations

from contextlib import contextmanager

from .. import _lib


class LaunchCounter:
    def __init__(self) -> None:
        self.n = 0

    def reset(self) -> None:
        self.n = 0

    @contextmanager
    def track(self):
        lib = _lib.lib()
        before = lib.mosaic_launch_count()
        try:
            yield
        finally:
            self.n += lib.mosaic_launch_count() - before
