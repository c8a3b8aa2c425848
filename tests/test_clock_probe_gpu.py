"""The kernels' clock probe (mi_fa2_set_clock_probe): with it on, the first work-group on each XCD
of every attention launch counts its own shader cycles and real-time ticks; the outputs are
bitwise those of a launch without it, and the clock it reads is a shader clock (between 0.5 and
3 GHz: MI355X peaks at 2.4 GHz)."""
import pytest
import torch

import workloads as wl
from conftest import announce
from kernels import _lib
from kernels.clock import ClockProbe
from kernels.fa2 import FlashAttention2Function, fa2_paged

pytestmark = pytest.mark.gpu


def test_probe_reads_a_clock_and_leaves_outputs_unchanged():
    q, k, v = (t.cuda() for t in wl.prefill_single(1024, seed=4))
    qd, kp, vp, tables, lens = wl.decode_paged(n_rows=8, lo=100, hi=3000, seed=4)
    bt = wl.table_tensor(tables).cuda()
    lens_t = torch.tensor(lens, dtype=torch.int32, device="cuda")
    qd, kp, vp = qd.cuda(), kp.cuda(), vp.cuda()
    announce("[gpu] clock probe: prefill 1x12x1024 and an 8-row paged decode, probe off then on")
    want_p = FlashAttention2Function.apply(q, k, v, True, None)
    want_d = fa2_paged(qd, kp, vp, bt, lens_t)
    probe = ClockProbe()
    with probe:
        for _ in range(5):
            got_p = FlashAttention2Function.apply(q, k, v, True, None)
            got_d = fa2_paged(qd, kp, vp, bt, lens_t)
    after = FlashAttention2Function.apply(q, k, v, True, None)  # probe off again
    torch.cuda.synchronize()
    assert torch.equal(got_p, want_p) and torch.equal(got_d, want_d) and torch.equal(after, want_p)
    r = probe.result()
    assert r is not None
    assert r["xcds"] == min(8, _lib.launch_plan()["num_xcds"])
    assert 0.5 < r["min"] <= r["ghz"] <= r["max"] < 3.0, r
    # launches made after the probe was turned off add nothing
    ticks = r["ticks"]
    FlashAttention2Function.apply(q, k, v, True, None)
    torch.cuda.synchronize()
    assert probe.result()["ticks"] == ticks
