"""The shader clock the attention kernels run at, read inside them (mi_fa2_set_clock_probe).

Kernel times scale with the shader clock, and the clock under load differs from box to box and
from workload to workload (the part lowers it under heavy MFMA load and raises it again within
microseconds once the load ends, so a reading taken just before or just after a timed region does
not give the region's clock).  While a `ClockProbe` is active, the first work-group on each XCD of
every prefill, decode and general-kernel launch adds the shader cycles its CU counted and the
100 MHz real-time ticks it spent, start to end, to that XCD's sums; the ratio is the clock the
XCD ran those kernels at.  A region's shader cycles are then its time x that clock, which is what
its cost is on any box: time = cycles / clock.

    probe = ClockProbe()
    with probe:
        ... launches ...
    torch.cuda.synchronize()
    probe.result()   # {"ghz": median over XCDs, "min", "max", "xcds"} or None
"""
import statistics

import torch

from . import _lib

REALTIME_HZ = 100e6  # s_memrealtime's constant rate


class ClockProbe:
    def __init__(self, device=None):
        self.acc = torch.zeros(16, dtype=torch.int64,
                               device=torch.device(device if device is not None else "cuda"))

    def __enter__(self):
        _lib.check(_lib.load().mi_fa2_set_clock_probe(self.acc.data_ptr()))
        return self

    def __exit__(self, *exc):
        _lib.check(_lib.load().mi_fa2_set_clock_probe(None))
        return False

    def result(self):
        """The clock (GHz) the probed launches ran at; call after a synchronize."""
        v = self.acc.cpu().tolist()
        per = [v[2 * x] / v[2 * x + 1] * REALTIME_HZ / 1e9 for x in range(8) if v[2 * x + 1] > 0]
        if not per:
            return None
        return {"ghz": round(statistics.median(per), 4), "min": round(min(per), 4),
                "max": round(max(per), 4), "xcds": len(per),
                "ticks": sum(v[2 * x + 1] for x in range(8))}
