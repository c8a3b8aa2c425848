"""The prefill kernel in both of its work-group shapes, each forced on every prefill parity test.

A launch picks two key streams per work-group (8 waves, one work-group per CU) or one (4 waves,
two work-groups per CU) from its grid size; most test shapes are small and take the two-stream
shape, the large packed and batched ones the one-stream shape.  MI_FA2_PREFILL_STREAMS, read at
every launch, forces one of them, and this module runs the prefill tests of test_fa2_gpu and
test_fa2_sweep_gpu under each, against the same oracle and bars.  (Decode and general-kernel
tests do not launch the prefill kernel and are not repeated.)
"""
import math

import pytest
import torch

import test_fa2_gpu as base
import test_fa2_sweep_gpu as sweep
from conftest import announce
from kernels.fa2 import FlashAttention2Function, fa2_varlen
from oracle import sdpa
import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["1", "2"], ids=["one_stream", "two_streams"])
def streams(request, monkeypatch):
    monkeypatch.setenv("MI_FA2_PREFILL_STREAMS", request.param)
    return int(request.param)


test_reference_cases = base.test_reference_cases
test_lse_matches_oracle = base.test_lse_matches_oracle
test_prefill_seq4096_causal = base.test_prefill_seq4096_causal
test_growing_scores_rescale_the_running_state = base.test_growing_scores_rescale_the_running_state
test_ragged_varlen_prefill = base.test_ragged_varlen_prefill
test_varlen_every_tile_is_written_for_any_row_count = base.test_varlen_every_tile_is_written_for_any_row_count
test_varlen_with_longer_keys_than_queries = base.test_varlen_with_longer_keys_than_queries
test_paged_prefill_4096_equals_dense_prefill_bitwise = base.test_paged_prefill_4096_equals_dense_prefill_bitwise
test_paged_prefill_over_cached_context = base.test_paged_prefill_over_cached_context
test_paged_varlen_mixed_rows = base.test_paged_varlen_mixed_rows
test_paged_block_size_32 = base.test_paged_block_size_32
test_paged_prefill_rows_across_table_groups_equal_dense = base.test_paged_prefill_rows_across_table_groups_equal_dense
test_empty_rows_and_queries_without_keys_give_zero = base.test_empty_rows_and_queries_without_keys_give_zero
test_nan_padding_never_leaks = base.test_nan_padding_never_leaks
test_strided_inputs_like_model_py = base.test_strided_inputs_like_model_py
test_odd_query_counts = base.test_odd_query_counts
test_single_token_key_tensors = base.test_single_token_key_tensors
test_mha_and_other_group_sizes = base.test_mha_and_other_group_sizes
test_single_head_short_rows = base.test_single_head_short_rows
test_repeat_calls_are_bitwise_deterministic = base.test_repeat_calls_are_bitwise_deterministic
test_padded_forward = sweep.test_padded_forward
test_packed_forward = sweep.test_packed_forward
test_paged_forward = sweep.test_paged_forward
test_paged_packed_forward = sweep.test_paged_packed_forward


def test_batched_long_rows(streams):
    """4 causal rows of 2,048 tokens (768 work-groups: the default picks one stream here)."""
    announce(f"[gpu] streams {streams}: batched long rows 4 x 12q/2kv x 2048 causal")
    q, k, v = wl.prefill_single(2048, seed=7)
    q = torch.cat([q, q.flip(2)], 0).repeat(2, 1, 1, 1)
    k = torch.cat([k, k.flip(2)], 0).repeat(2, 1, 1, 1)
    v = torch.cat([v, v.flip(2)], 0).repeat(2, 1, 1, 1)
    out = FlashAttention2Function.apply(q.cuda(), k.cuda(), v.cuda(), True, None)
    torch.cuda.synchronize()
    base.check_close(out[:2], sdpa.attention_ref(q[:2], k[:2], v[:2], True), what="rows 0-1")
    assert torch.equal(out[:2], out[2:]), "equal rows must give equal outputs"


def test_ragged_varlen_lse(streams):
    """The 16-row ragged batch's LSE against the oracle's, row by row (natural log, [Hq, total])."""
    announce(f"[gpu] streams {streams}: ragged varlen LSE")
    q, k, v, lens, cu = wl.prefill_ragged(seed=3)
    cu_t = torch.tensor(cu, dtype=torch.int32, device="cuda")
    out, lse = fa2_varlen(q.cuda(), k.cuda(), v.cuda(), cu_t, cu_t, max(lens), is_causal=True,
                          return_lse=True)
    torch.cuda.synchronize()
    base.check_close(out, sdpa.varlen_ref(q, k, v, cu, cu, True), what="varlen")
    lse = lse.cpu()
    for b in range(len(lens)):
        s, e = cu[b], cu[b + 1]
        qb = q[s:e].transpose(0, 1).unsqueeze(0)
        kb = k[s:e].transpose(0, 1).unsqueeze(0)
        want = sdpa.lse_ref(qb, kb, True)[0]
        # bf16-rounded P in the row sum: within log(1 + 2^-8) of the exact LSE
        assert (lse[:, s:e] - want).abs().max().item() < math.log1p(2.0 ** -8) + 1e-4, f"row {b}"
