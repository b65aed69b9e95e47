"""hipGraph capture and replay of one forward call.

The reference measures graph mode by capturing the kernel launch
``func(*args)`` in an NPUGraph and replaying it (``test_graph_mode.py:185-209``).
Here the whole device pipeline of a call (planner when no plan is given, row
resolution, attention, split combine) is captured natively through
``sas_graph_capture`` and replayed with ``sas_graph_launch``.  The captured
launches reference the tensors of the :class:`~dsv4_planb_amd.api.SasLaunch`,
which the graph keeps alive; refresh their contents in place between replays.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .api import SasLaunch


class SasGraph:
    def __init__(self, launch: SasLaunch):
        self.launch = launch
        self._exec = ctypes.c_void_p()
        lib = _lib.load()
        side = torch.cuda.Stream(device=launch.device)  # capture needs a non-default stream
        side.wait_stream(torch.cuda.current_stream(launch.device))
        with torch.cuda.stream(side):
            plan = None if launch.plan is None else ctypes.c_void_p(launch.plan.data_ptr())
            rc = lib.sas_graph_capture(ctypes.byref(launch.params), ctypes.byref(launch.tensors),
                                       plan, ctypes.c_void_p(launch.ws.data_ptr()),
                                       launch.ws.numel(), ctypes.c_void_p(side.cuda_stream),
                                       ctypes.byref(self._exec))
        torch.cuda.current_stream(launch.device).wait_stream(side)
        _lib.check(rc, "sas_graph_capture")

    def replay(self, stream: torch.cuda.Stream | None = None) -> None:
        s = stream if stream is not None else torch.cuda.current_stream(self.launch.device)
        _lib.check(_lib.load().sas_graph_launch(self._exec, ctypes.c_void_p(s.cuda_stream)),
                   "sas_graph_launch")

    def close(self) -> None:
        if self._exec:
            _lib.load().sas_graph_destroy(self._exec)
            self._exec = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass
