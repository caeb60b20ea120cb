"""CopyEngine -- copy-engine (SDMA) transfers for the tier on side streams.

Mirror of the reference ``tier/dma.py:77-140``: double-buffered side streams (default
priority) on which host-planned runs of pinned-pool pages are copied into hot slots with
hipMemcpy2DAsync (``amass_tier_dma``), so the host-link transfer does not hold compute
units and can overlap decode.  ``issue`` returns an event the consumer stream waits on.
"""
from __future__ import annotations

import torch

from .residency import Residency


class CopyEngine:
    def __init__(self, device=None, n_streams: int = 2):
        self.device = device
        self.streams = [torch.cuda.Stream(device=device) for _ in range(n_streams)]
        self._i = 0

    def next_stream(self) -> torch.cuda.Stream:
        s = self.streams[self._i]
        self._i = (self._i + 1) % len(self.streams)
        return s

    def issue(self, runs, stream=None, timing: bool = False) -> torch.cuda.Event:
        stream = stream or self.next_stream()
        stream.wait_stream(torch.cuda.current_stream(self.device))
        Residency.issue_dma_plan(runs, stream)
        ev = torch.cuda.Event(enable_timing=timing)
        ev.record(stream)
        return ev
