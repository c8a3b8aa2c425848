"""CPU checks of the drop-in boundary: libmi_fa2.so loads, exports exactly what include/mi_fa2.h
declares, validates its arguments before touching the GPU, and the Python mirror of
FlashAttention2Function (kernels/fa2.py:164-214) raises like the reference on bad inputs.
No kernel is launched here."""
import ctypes
import re

import pytest
import torch

from conftest import ROOT
from kernels import _lib, fa2

HEADER = ROOT / "include" / "mi_fa2.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"MI_FA2_API\s+[\w\s\*]+?\b(mi_fa2_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) == 19
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES)


def test_library_exports_nothing_else():
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted(line.split()[-1] for line in out.splitlines() if " T " in line)
    assert exported == declared_symbols()


def test_version_and_clean_error_state():
    lib = _lib.load()
    assert lib.mi_fa2_version().decode().startswith("mi_fa2 ")
    assert "gfx950" in lib.mi_fa2_version().decode()


@pytest.mark.parametrize("cus,xcds,mapped,paged,dense", [
    (256, 8, 8, 768, 512),   # MI355X: the tuned sizes
    (32, 1, 1, 96, 64),      # one XCD of it (a CPX partition)
    (64, 2, 2, 192, 128),
    (80, 3, 1, 240, 160),    # an XCD count that is not a power of two: no XCD mapping
])
def test_launch_plan_follows_the_device_topology(cus, xcds, mapped, paged, dense, monkeypatch):
    # the grid sizes and the XCD mapping come from the device's CU and XCD counts, not from
    # constants; the MI355X case keeps the sizes the kernels were tuned at
    monkeypatch.delenv("MI_FA2_DECODE_WGS", raising=False)
    pl = _lib.launch_plan(cus, xcds)
    assert pl == {"num_cus": cus, "num_xcds": xcds, "xcds_mapped": mapped,
                  "decode_work_groups_paged": paged, "decode_work_groups_dense": dense,
                  "prefill_one_stream_min_work_groups": 2 * cus,
                  "prefill_one_stream_max_keys": 4096}


def test_launch_plan_and_clock_probe_reject_bad_arguments():
    lib = _lib.load()
    assert lib.mi_fa2_launch_plan(256, 8, None) == 1
    assert "out is NULL" in lib.mi_fa2_last_error().decode()
    assert lib.mi_fa2_set_clock_probe(12) == 1
    assert "aligned" in lib.mi_fa2_last_error().decode()
    assert lib.mi_fa2_set_clock_probe(None) == 0


def test_workspace_sizes():
    lib = _lib.load()
    # prefill needs none
    assert lib.mi_fa2_fwd_workspace_size(1, 12, 2, 4096, 4096, 128) == 0
    # a decode step with long rows needs [B, Hq, splits] x (128 + 2) fp32 partials, one split per
    # 128 keys of the longest row, and an int32 partial count per (row, kv head)
    n = lib.mi_fa2_fwd_paged_workspace_size(64, 12, 2, 1, 8192, 128)
    assert n == 64 * 12 * (8192 // 128) * 130 * 4 + 64 * 2 * 4
    # a single short row fits in one split: no workspace
    assert lib.mi_fa2_fwd_workspace_size(1, 12, 2, 1, 100, 128) == 0
    # the sampler: one (score, index) partial per 8192-entry chunk of each row, none for one chunk
    assert lib.mi_fa2_sample_workspace_size(16, 151936) == 16 * 19 * 8
    assert lib.mi_fa2_sample_workspace_size(4, 8192) == 0


def _fwd(lib, **over):
    args = dict(dtype=0, q=16, k=16, v=16, o=16, lse=None, kv_lens=None, batch=1, heads_q=12,
                heads_kv=2, seqlen_q=8, seqlen_k=8, head_dim=128)
    args.update(over)
    st = (ctypes.c_int64 * 4)(8192, 1024, 128, 1)
    return lib.mi_fa2_fwd(args["dtype"], args["q"], args["k"], args["v"], args["o"], args["lse"],
                          args["kv_lens"], args["batch"], args["heads_q"], args["heads_kv"],
                          args["seqlen_q"], args["seqlen_k"], args["head_dim"],
                          over.get("q_strides", st), st, st, st, None, 1, 0.1, None, 0, None)


@pytest.mark.parametrize("over,status,msg", [
    (dict(head_dim=64), 2, "head_dim 64"),
    (dict(dtype=7), 2, "dtype"),
    (dict(heads_q=12, heads_kv=5), 1, "multiple"),
    (dict(q=None), 1, "q is NULL"),
    (dict(q=24), 1, "16-byte aligned"),
    (dict(seqlen_q=-1), 1, "bad lengths"),
    (dict(q_strides=(ctypes.c_int64 * 4)(8192, 1024, 100, 1)), 1, "multiple of 8"),
])
def test_c_abi_rejects_bad_arguments_before_any_launch(over, status, msg):
    lib = _lib.load()
    assert _fwd(lib, **over) == status
    assert msg in lib.mi_fa2_last_error().decode()


def _fwd_general(lib, **over):
    args = dict(dtype=2, q=16, k=16, v=16, o=16, batch=1, heads_q=4, heads_kv=2, seqlen_q=8,
                seqlen_k=8, head_dim=64, head_dim_v=32)
    args.update(over)
    st = (ctypes.c_int64 * 4)(2048, 512, 64, 1)
    return lib.mi_fa2_fwd_general(args["dtype"], args["q"], args["k"], args["v"], args["o"], None,
                                  None, args["batch"], args["heads_q"], args["heads_kv"],
                                  args["seqlen_q"], args["seqlen_k"], args["head_dim"],
                                  args["head_dim_v"], st, st, st, st, None, 1, 0.125, None)


@pytest.mark.parametrize("over,status,msg", [
    (dict(head_dim=8), 2, "power of two from 16 to 256"),
    (dict(head_dim_v=512), 2, "power of two from 16 to 256"),
    (dict(head_dim=48), 2, "power of two from 16 to 256"),
    (dict(dtype=3), 2, "dtype"),
    (dict(heads_q=6, heads_kv=4), 1, "bad sizes"),
    (dict(batch=70000), 2, "65535"),
    (dict(v=None), 1, "v is NULL"),
    (dict(o=40), 1, "16-byte aligned"),
])
def test_general_entry_point_rejects_bad_arguments_before_any_launch(over, status, msg):
    lib = _lib.load()
    assert _fwd_general(lib, **over) == status
    assert msg in lib.mi_fa2_last_error().decode()


def test_general_entry_point_zero_sized_calls_are_no_ops():
    lib = _lib.load()
    assert _fwd_general(lib, batch=0) == 0
    assert _fwd_general(lib, seqlen_q=0) == 0


def test_python_mirror_routes_the_wider_envelope_and_rejects_the_rest():
    # d and d_v powers of two (kernels/fa2.py:185) up to 256, bf16 / fp16 / fp32: accepted by the
    # envelope checks (no launch here: these are CPU tensors, so the is_cuda assert fires first
    # in apply; the envelope functions are checked directly).
    q = torch.empty(1, 4, 3, 64)
    fa2._general_envelope(q, torch.empty(1, 2, 5, 64), torch.empty(1, 2, 5, 256))
    with pytest.raises(AssertionError):
        fa2._general_envelope(torch.empty(1, 4, 3, 512), torch.empty(1, 2, 5, 512),
                              torch.empty(1, 2, 5, 512))
    with pytest.raises(AssertionError):
        fa2._general_envelope(q.double(), torch.empty(1, 2, 5, 64).double(),
                              torch.empty(1, 2, 5, 64).double())
    with pytest.raises(AssertionError):
        fa2._envelope(q.bfloat16(), q.bfloat16(), q.bfloat16())


def test_overlapping_key_rows_are_rejected():
    lib = _lib.load()
    st = (ctypes.c_int64 * 4)(8192, 1024, 128, 1)
    kst = (ctypes.c_int64 * 4)(8192, 1024, 64, 1)
    rc = lib.mi_fa2_fwd(0, 16, 16, 16, 16, None, None, 1, 12, 2, 8, 8, 128, st, kst, st, st, None,
                        1, 0.1, None, 0, None)
    assert rc == 1 and "below head_dim" in lib.mi_fa2_last_error().decode()
    ps = (ctypes.c_int64 * 2)(64, 128)
    rc = lib.mi_fa2_fwd_paged(0, 16, 16, 16, 16, None, 16, 8, 16, 1, 12, 2, 1, 64, 128, 16, 10,
                              st, ps, st, None, 0, 0.1, None, 0, None)
    assert rc == 1 and "below head_dim" in lib.mi_fa2_last_error().decode()


def test_prefill_rejects_key_strides_past_its_32_bit_load_extents():
    # the prefill kernel loads up to 64 K/V rows per buffer resource (rows x 2 bytes x stride in a
    # 32-bit extent): token strides of 2^24 elements or more are refused in every prefill entry
    # point, before anything touches a device
    lib = _lib.load()
    big = 1 << 24
    st = (ctypes.c_int64 * 4)(8192, 1024, 128, 1)
    kst = (ctypes.c_int64 * 4)(big * 8, big, big, 1)
    rc = lib.mi_fa2_fwd(0, 16, 16, 16, 16, None, None, 1, 12, 2, 8, 8, 128, st, kst, kst, st, None,
                        1, 0.1, None, 0, None)
    assert rc == 2 and "2^24" in lib.mi_fa2_last_error().decode()
    s2 = (ctypes.c_int64 * 2)(1536, 128)
    k2 = (ctypes.c_int64 * 2)(big, 128)
    cu = 16
    rc = lib.mi_fa2_fwd_varlen(0, 16, 16, 16, 16, None, cu, cu, 1, 12, 2, 8, 128, s2, k2, k2, s2,
                               None, 1, 0.1, None)
    assert rc == 2 and "2^24" in lib.mi_fa2_last_error().decode()
    rc = lib.mi_fa2_fwd_paged(0, 16, 16, 16, 16, None, 16, 8, 16, 1, 12, 2, 8, 64, 128, 16, 10,
                              st, k2, st, None, 1, 0.1, None, 0, None)
    assert rc == 2 and "2^24" in lib.mi_fa2_last_error().decode()
    rc = lib.mi_fa2_fwd_paged_varlen(0, 16, 16, 16, 16, None, cu, 16, 8, 16, 1, 12, 2, 8, 64, 128,
                                     16, 10, s2, k2, s2, None, 1, 0.1, None)
    assert rc == 2 and "2^24" in lib.mi_fa2_last_error().decode()
    # a decode (one query) keeps its own, looser bound (16-token runs: 2^26)
    rc = lib.mi_fa2_fwd_paged(0, 16, 16, 16, 16, None, 16, 8, 16, 1, 12, 2, 1, 64, 128, 16, 10,
                              st, (ctypes.c_int64 * 2)(1 << 26, 128), st, None, 0, 0.1, None, 0,
                              None)
    assert rc == 2 and "2^26" in lib.mi_fa2_last_error().decode()


def test_paged_rejects_bad_block_size():
    lib = _lib.load()
    st = (ctypes.c_int64 * 4)(1536, 128, 1536, 1)
    ps = (ctypes.c_int64 * 2)(256, 128)
    rc = lib.mi_fa2_fwd_paged(0, 16, 16, 16, 16, None, 16, 8, 16, 1, 12, 2, 1, 64, 128, 24, 10,
                              st, ps, st, None, 0, 0.1, None, 0, None)
    assert rc == 2 and "block_size" in lib.mi_fa2_last_error().decode()


def test_zero_sized_calls_are_no_ops():
    lib = _lib.load()
    assert _fwd(lib, batch=0) == 0
    assert _fwd(lib, seqlen_q=0) == 0


def test_python_mirror_asserts_like_the_reference():
    q = torch.randn(1, 12, 4, 128, dtype=torch.bfloat16)
    k = torch.randn(1, 2, 4, 128, dtype=torch.bfloat16)
    # CPU tensors: the reference asserts is_cuda (kernels/fa2.py:177)
    with pytest.raises(AssertionError):
        fa2.FlashAttention2Function.apply(q, k, k, True, None)


def test_stride_helper_gives_size_one_dims_their_contiguous_stride():
    # size-1 dims are indexed only at 0, but a token stride is also the row pitch of the kernels'
    # load extents: it must cover a whole row (a 0 made a single-token K read as zeros)
    t = torch.empty(3, 1, 5, 128)[:, :, :, :]
    assert list(fa2._strides(t)) == [640, 640, 128, 1]
    k = torch.empty(2, 2, 1, 128)
    assert list(fa2._strides(k)) == [256, 128, 128, 1]
    e = torch.empty(1, 2, 128).expand(1, 2, 128)
    assert list(fa2._strides(e.as_strided((1, 2, 128), (0, 128, 1)))) == [256, 128, 1]
    assert fa2._dims_ok(torch.empty(2, 12, 7, 128))
    assert not fa2._dims_ok(torch.empty(2, 12, 7, 128).transpose(-1, -2))


def _sample(lib, **over):
    a = dict(dtype=0, logits=16, row_stride=1000, batch=2, vocab=1000, temperature=1.0,
             tokens=16, ws=None, ws_bytes=0)
    a.update(over)
    return lib.mi_fa2_sample(a["dtype"], a["logits"], a["row_stride"], a["batch"], a["vocab"],
                             a["temperature"], 0, 0, a["tokens"], a["ws"], a["ws_bytes"], None)


@pytest.mark.parametrize("over,status,msg", [
    (dict(dtype=5), 2, "dtype"),
    (dict(logits=None), 1, "logits is NULL"),
    (dict(tokens=None), 1, "tokens is NULL"),
    (dict(dtype=2, logits=18), 1, "aligned"),
    (dict(row_stride=999), 1, "row_stride"),
    (dict(temperature=float("nan")), 1, "NaN"),
    (dict(vocab=0), 1, "bad sizes"),
    (dict(batch=70000), 2, "65535"),
    (dict(vocab=20000, row_stride=20000), 3, "workspace"),
])
def test_sampler_rejects_bad_arguments_before_any_launch(over, status, msg):
    lib = _lib.load()
    assert _sample(lib, **over) == status
    assert msg in lib.mi_fa2_last_error().decode()


def test_sampler_zero_rows_is_a_no_op():
    lib = _lib.load()
    assert _sample(lib, batch=0, logits=None, tokens=None) == 0


def test_model_ops_reject_bad_arguments():
    lib = _lib.load()
    assert lib.mi_fa2_add_rmsnorm(0, 16, 1536, None, 0, 16, None, 0, 16, 1536, 2, 1540, 1e-6,
                                  None) == 1
    assert "hidden" in lib.mi_fa2_last_error().decode()
    assert lib.mi_fa2_add_rmsnorm(0, 16, 8200, None, 0, 16, None, 0, 16, 8200, 2, 8200, 1e-6,
                                  None) == 1
    assert lib.mi_fa2_add_rmsnorm(0, 24, 1536, None, 0, 16, None, 0, 16, 1536, 2, 1536, 1e-6,
                                  None) == 1
    assert "aligned" in lib.mi_fa2_last_error().decode()
    assert lib.mi_fa2_add_rmsnorm(3, 16, 1536, None, 0, 16, None, 0, 16, 1536, 2, 1536, 1e-6,
                                  None) == 2
    assert lib.mi_fa2_silu_mul(0, 16, 100, 16, 64, 2, 64, None) == 1
    assert "gate_up" in lib.mi_fa2_last_error().decode()
    assert lib.mi_fa2_silu_mul(0, 16, 128, 16, 64, 0, 64, None) == 0     # no rows: no-op


def _combine(lib, **over):
    i64 = lambda *v: (ctypes.c_int64 * len(v))(*v)  # noqa: E731
    a = dict(out_dtype=0, part_o=16, part_lse=16, n_parts=None, n_rows=4, heads=12, max_parts=3,
             head_dim=128, po=i64(4 * 12 * 128, 12 * 128, 128), pl=i64(48, 12, 1), o=16,
             os=i64(12 * 128, 128), lse=None, ls=None)
    a.update(over)
    return lib.mi_fa2_combine(a["out_dtype"], a["part_o"], a["part_lse"], a["n_parts"],
                              a["n_rows"], a["heads"], a["max_parts"], a["head_dim"], a["po"],
                              a["pl"], a["o"], a["os"], a["lse"], a["ls"], None)


@pytest.mark.parametrize("over,code,msg", [
    (dict(out_dtype=5), 2, "out_dtype"),
    (dict(head_dim=64), 2, "head_dim"),
    (dict(n_rows=70000), 1, "65535"),
    (dict(o=None), 1, "NULL"),
    (dict(part_o=None), 1, "NULL"),
    (dict(lse=16), 1, "lse strides"),
    (dict(o=18), 1, "aligned"),
    (dict(part_o=20), 1, "aligned"),
    (dict(os=(ctypes.c_int64 * 2)(12 * 128, 129)), 1, "even"),
])
def test_combine_rejects_bad_arguments(over, code, msg):
    lib = _lib.load()
    assert _combine(lib, **over) == code
    assert msg in lib.mi_fa2_last_error().decode()


def test_combine_with_nothing_to_do_touches_nothing():
    lib = _lib.load()
    assert _combine(lib, n_rows=0, part_o=None, o=None) == 0
    assert _combine(lib, heads=0, part_o=None, o=None) == 0


def test_noalloc_paged_forward_refuses_more_than_its_scratch_before_launching():
    """mi_fa2_fwd_paged_noalloc holds 32 MiB of scratch: a decode needing more is refused with
    MI_FA2_ERR_WORKSPACE before anything touches a device (so this runs without a GPU)."""
    lib = _lib.load()
    i64 = lambda *v: (ctypes.c_int64 * len(v))(*v)  # noqa: E731
    # 64 rows x 12 heads at 16,384 keys need 128 splits x 130 x 4 B per (row, head): 51 MB
    need = lib.mi_fa2_fwd_paged_workspace_size(64, 12, 2, 1, 16384, 128)
    assert need > 32 << 20
    rc = lib.mi_fa2_fwd_paged_noalloc(0, 16, 16, 16, 16, None, 16, 1024, 16, 64, 12, 2, 1, 16384,
                                      128, 16, 65536, i64(1536, 128, 128), i64(256, 128),
                                      i64(1536, 128, 128), None, 0, 0.088, None)
    assert rc == 3
    msg = lib.mi_fa2_last_error().decode()
    assert "at most 33554432" in msg and str(need) in msg
