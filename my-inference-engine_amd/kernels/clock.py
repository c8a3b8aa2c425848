"""Shader clock around a timed region, read on the device (mi_fa2_clock_stamp).

Kernel times scale with the shader clock the part sustains under load, which differs by a few
percent between boxes.  `ClockStamp` takes a reading on the current stream right before and right
after a timed region.  In a reading every work-group of the stamp launch measures its own CU's
clock: its shader-cycle count over a spin of a few microseconds of the 100 MHz real-time counter
(the shader-cycle count is per CU and stops while the CU is clock-gated, so counts of different
work-groups are never compared).  The clock of the region is taken as the mean of the two
readings' medians; a region's shader cycles are its time x that clock, which is what its cost is
on any box: time = cycles / clock.
"""
import statistics

import torch

from . import _lib

REALTIME_HZ = 100e6  # s_memrealtime's constant rate
WORDS = 5            # per work-group: cycles0, ticks0, cycles1, ticks1, XCD id


class ClockStamp:
    def __init__(self, device=None, groups_per_xcd=2, spin_us=5.0):
        self.device = torch.device(device if device is not None else "cuda")
        plan = _lib.launch_plan()
        self.n_groups = max(1, plan["num_xcds"]) * groups_per_xcd
        self.spin_ticks = max(1, int(spin_us * 1e-6 * REALTIME_HZ))
        self.buf = torch.zeros((2, self.n_groups, WORDS), dtype=torch.int64, device=self.device)

    def _stamp(self, i):
        lib = _lib.load()
        with _lib.on_device(self.device) as stream:
            _lib.check(lib.mi_fa2_clock_stamp(self.buf[i].data_ptr(), self.n_groups,
                                              self.spin_ticks, stream))

    def before(self):
        self._stamp(0)

    def after(self):
        self._stamp(1)

    @staticmethod
    def _reading(rows):
        per = {}
        for c0, t0, c1, t1, x in rows:
            if t1 > t0 and c1 > c0:
                per.setdefault(x, []).append((c1 - c0) / (t1 - t0) * REALTIME_HZ / 1e9)
        return {x: statistics.median(v) for x, v in sorted(per.items())}

    def result(self):
        """The clock (GHz) around the stamped region; call after a synchronize."""
        b = self.buf.cpu().tolist()
        before, after = self._reading(b[0]), self._reading(b[1])
        if not before or not after:
            return None
        g0, g1 = statistics.median(before.values()), statistics.median(after.values())
        per_xcd = [round((before[x] + after[x]) / 2, 4) for x in before if x in after]
        return {"ghz": round((g0 + g1) / 2, 4), "before": round(g0, 4), "after": round(g1, 4),
                "min": min(per_xcd) if per_xcd else None, "max": max(per_xcd) if per_xcd else None,
                "xcds": len(per_xcd),
                "region_us": round((b[1][0][1] - b[0][0][3]) / REALTIME_HZ * 1e6, 1)}
