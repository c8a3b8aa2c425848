"""mi_fa2_fwd_paged_noalloc (the paged forward whose split-decode partials live in the library's
static scratch) against mi_fa2_fwd_paged (the same kernels over a caller workspace), through the C
ABI: bitwise the same outputs and LSE, on two calls in a row with the second smaller (the scratch
keeps the first call's contents), a prefill through it, and the oracle on a sample of rows."""
import ctypes
import math

import pytest
import torch

import workloads as wl
from conftest import announce
from kernels import _lib
from oracle import paged as opaged
from oracle import sdpa

pytestmark = pytest.mark.gpu


def _call(noalloc, q, kp, vp, bt, lens, max_kv, causal):
    lib = _lib.load()
    B, Hq, T, d = q.shape
    O = torch.full_like(q, float("nan"))
    L = torch.full((B, Hq, T), float("nan"), device=q.device)
    pool = (ctypes.c_int64 * 2)(*kp.stride()[:2])
    args = [0, q.data_ptr(), kp.data_ptr(), vp.data_ptr(), O.data_ptr(), L.data_ptr(),
            bt.data_ptr(), bt.stride(0), lens.data_ptr(), B, Hq, kp.shape[1], T, max_kv, d, 16,
            kp.shape[0] // 16, _lib.strides(q), pool, _lib.strides(O), _lib.strides(L),
            int(causal), 1.0 / math.sqrt(d)]
    with torch.cuda.device(q.device):
        if noalloc:
            _lib.check(lib.mi_fa2_fwd_paged_noalloc(*args, _lib.stream_of(q)))
        else:
            n = lib.mi_fa2_fwd_paged_workspace_size(B, Hq, kp.shape[1], T, max_kv, d)
            ws = torch.empty(max(n, 1), dtype=torch.uint8, device=q.device)
            _lib.check(lib.mi_fa2_fwd_paged(*args, ws.data_ptr(), n, _lib.stream_of(q)))
            torch.cuda.synchronize()
    return O, L


def test_noalloc_decode_equals_the_workspace_entry_point_on_two_calls():
    # the full 64-row decode (25.6 MB of the 32 MiB scratch), then a smaller one: 9 rows
    for n_rows, lo, hi, seed in ((64, 128, 8192, 0), (9, 16, 3000, 1)):
        q, kp, vp, tables, lens = wl.decode_paged(n_rows=n_rows, lo=lo, hi=hi, seed=seed)
        bt = wl.table_tensor(tables).cuda()
        lens_t = torch.tensor(lens, dtype=torch.int32, device="cuda")
        qd, kd, vd = q.cuda(), kp.cuda(), vp.cuda()
        max_kv = bt.shape[1] * 16
        announce(f"[gpu] no-alloc paged decode: {n_rows} rows, kv_len U[{lo},{hi}]")
        got, got_l = _call(True, qd, kd, vd, bt, lens_t, max_kv, False)
        torch.cuda.synchronize()
        want, want_l = _call(False, qd, kd, vd, bt, lens_t, max_kv, False)
        torch.cuda.synchronize()
        assert torch.equal(got, want) and torch.equal(got_l, want_l)
        # and the oracle on a sample of rows
        rows = list(range(0, n_rows, max(1, n_rows // 8)))
        S = max(lens[r] for r in rows)
        ref = sdpa.attention_ref(q[rows], opaged.gather_dense(kp, [tables[r] for r in rows], S, 16),
                                 opaged.gather_dense(vp, [tables[r] for r in rows], S, 16), False,
                                 [lens[r] for r in rows])
        err = (got[rows].float().cpu() - ref).abs()
        assert err.max().item() < 1e-2 and err.mean().item() < 1e-3


def test_noalloc_prefill_equals_the_workspace_entry_point():
    q, kp, vp, tables = wl.prefill_paged(700, seed=2)
    bt = wl.table_tensor(tables).cuda()
    lens = torch.tensor([700], dtype=torch.int32, device="cuda")
    announce("[gpu] no-alloc paged prefill: 1 x 12 x 700 causal")
    got, got_l = _call(True, q.cuda(), kp.cuda(), vp.cuda(), bt, lens, 700, True)
    want, want_l = _call(False, q.cuda(), kp.cuda(), vp.cuda(), bt, lens, 700, True)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(got_l, want_l)


def test_noalloc_decode_allocates_no_device_memory():
    # what the entry point is for: after a first call (which looks up the scratch's address once),
    # calls leave the device's free memory and torch's allocations unchanged
    q, kp, vp, tables, lens = wl.decode_paged(n_rows=16, lo=128, hi=4000, seed=3)
    bt = wl.table_tensor(tables).cuda()
    lens_t = torch.tensor(lens, dtype=torch.int32, device="cuda")
    qd, kd, vd = q.cuda(), kp.cuda(), vp.cuda()
    B, Hq, T, d = qd.shape
    O = torch.empty_like(qd)
    L = torch.empty((B, Hq, T), device="cuda")
    max_kv = bt.shape[1] * 16
    assert _lib.load().mi_fa2_fwd_paged_workspace_size(B, Hq, kd.shape[1], T, max_kv, d) > 0
    pool = (ctypes.c_int64 * 2)(*kd.stride()[:2])
    qs, os_, ls = _lib.strides(qd), _lib.strides(O), _lib.strides(L)
    stream = _lib.stream_of(qd)
    lib = _lib.load()

    def call():
        _lib.check(lib.mi_fa2_fwd_paged_noalloc(
            0, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), O.data_ptr(), L.data_ptr(),
            bt.data_ptr(), bt.stride(0), lens_t.data_ptr(), B, Hq, kd.shape[1], T, max_kv, d, 16,
            kd.shape[0] // 16, qs, pool, os_, ls, 0, 1.0 / math.sqrt(d), stream))

    announce("[gpu] no-alloc paged decode: device memory before and after")
    call()
    torch.cuda.synchronize()
    free0, alloc0 = torch.cuda.mem_get_info()[0], torch.cuda.memory_allocated()
    for _ in range(3):
        call()
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == alloc0
    assert torch.cuda.mem_get_info()[0] >= free0
    want, _ = _call(False, qd, kd, vd, bt, lens_t, max_kv, False)
    assert torch.equal(O, want)
