"""Host-side argument checks of the torch wrappers that need no GPU: they reject
metadata and plans that do not fit a call before anything is launched."""

import numpy as np
import pytest
import torch

from minisgl_hip import ops


def test_step_sizes_match_the_lengths():
    cached = np.array([0, 5, 99], dtype=np.int32)
    device = np.array([4, 6, 100], dtype=np.int32)
    ops.check_step_sizes(cached, device, 1, 6, 110)
    ops.check_step_sizes(cached, device, 16, 6, 1 + 1 + 7)
    with pytest.raises(ValueError, match="num_tokens"):  # one extend token short
        ops.check_step_sizes(cached, device, 1, 5, 110)
    with pytest.raises(ValueError, match="num_kv"):  # index capacity short by one slot
        ops.check_step_sizes(cached, device, 1, 6, 109)
    with pytest.raises(ValueError, match="num_kv"):  # page-level count, not token count
        ops.check_step_sizes(cached, device, 16, 6, 110)


def test_build_step_indices_rejects_undersized_capacities_before_launch():
    table = torch.zeros((4, 128), dtype=torch.int32)
    r = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="num_kv"):
        ops.build_step_indices(table, r, r, r, num_tokens=11, num_kv=10, page_size=1,
                               host_lens=(np.array([0, 0]), np.array([2, 9])))


def test_planned_decode_needs_a_plan_for_its_sizes():
    b, hq, hkv, d, splits = 4, 16, 8, 64, 4
    q = torch.zeros(b, hq, d)
    pool = torch.zeros(64, hkv, d)
    indptr = torch.arange(b + 1, dtype=torch.int32)
    indices = torch.zeros(b, dtype=torch.int32)
    ws = torch.empty(ops.decode_workspace_bytes(b, hq, hkv, d, splits), dtype=torch.uint8)
    with pytest.raises(ValueError, match="no plan"):  # never planned
        ops.paged_decode_attention(q, pool, pool, indptr, indices, 0.1, max_splits=splits, workspace=ws,
                                   planned=True)
    ws._msgl_decode_plan = (b, hkv, splits - 1)  # planned for another split bound
    with pytest.raises(ValueError, match="no plan"):
        ops.paged_decode_attention(q, pool, pool, indptr, indices, 0.1, max_splits=splits, workspace=ws,
                                   planned=True)


def test_planned_prefill_needs_a_plan_for_its_sizes():
    q = torch.zeros(8, 16, 64, dtype=torch.bfloat16)
    pool = torch.zeros(64, 8, 64, dtype=torch.bfloat16)
    qi = torch.tensor([0, 3, 8], dtype=torch.int32)
    ki = torch.tensor([0, 10, 20], dtype=torch.int32)
    kx = torch.zeros(20, dtype=torch.int32)
    ws = ops.prefill_workspace(2, 8, 5, 16, 8, 64, 2, "cpu")
    with pytest.raises(ValueError, match="no plan"):
        ops.prefill_ragged_attention(q, pool, pool, qi, ki, kx, None, 0.1, max_extend_len=5, max_seq_len=10,
                                     max_splits=2, workspace=ws, planned=True)


def test_scale_value_reads_cpu_tensors_and_floats():
    assert ops.scale_value(0.25) == 0.25
    assert ops.scale_value(torch.tensor([0.125])) == 0.125
    with pytest.raises(ValueError):
        ops.scale_value(torch.zeros(2))


def test_decode_split_choice_for_known_lengths():
    rng = np.random.default_rng(0)
    # near-uniform batch filling the device: the shared-head form (one launch, no merge)
    assert ops.decode_splits_for(np.full(128, 1144), 8) == 1
    assert ops.decode_splits_for(rng.integers(1000, 1200, size=96), 8) == 1
    # ragged lengths, too few (request, kv head) pairs, or more than 512 keys per wavefront: the split forms
    ragged = rng.integers(200, 2049, size=128)
    assert ops.decode_splits_for(ragged, 8) == ops.default_splits(128, 8, int(ragged.max()))
    assert ops.decode_splits_for(np.full(95, 1144), 8) != 1
    assert ops.decode_splits_for(np.full(128, 3000), 8) != 1


def test_validate_metadata_needs_lengths_with_pages():
    indptr = torch.tensor([0, 2], dtype=torch.int32)
    ids = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(ValueError, match="seq_lens"):
        ops.validate_metadata(indptr, ids, None, num_slots=64, page_size=16)
