"""Per-key mask / bias operands of the attention kernels (host logic, no launch).

The kernel reads a uint8 mask and an fp32 bias of B*Sk values.  ops.key_operands gives every
mask value the truth value the reference's ``key_mask.to(torch.bool)`` gives it
(kernels/fp8_attention.py:374), accepts one row shared by every batch item, and refuses
tensors of another device or size with ValueError before anything reaches the kernel.
"""
import pytest
import torch

from minimaxh3_amd import ops

CPU = torch.device("cpu")


def test_mask_truth_values_follow_to_bool():
    mask = torch.tensor([[0.0, 0.5, -2.0, 256.0, 1e-30, float("nan")]])
    km, kb = ops.key_operands(mask, None, 1, 6, CPU)
    assert kb is None and km.dtype == torch.uint8 and km.shape == (1, 6)
    assert km.tolist() == mask.to(torch.bool).to(torch.uint8).tolist() == [[0, 1, 1, 1, 1, 1]]
    ints = torch.tensor([[0, 256, 1, 512]], dtype=torch.int32)  # uint8 conversion would wrap 256 to 0
    km, _ = ops.key_operands(ints, None, 1, 4, CPU)
    assert km.tolist() == [[0, 1, 1, 1]]


def test_shared_row_is_broadcast_and_sizes_are_checked():
    km, kb = ops.key_operands(torch.tensor([True, False, True]), torch.tensor([[0.5, -1e9, 2.0]]), 2, 3, CPU)
    assert km.tolist() == [[1, 0, 1], [1, 0, 1]] and km.is_contiguous()
    assert kb.dtype == torch.float32 and kb.shape == (2, 3) and kb[1, 1] == -1e9
    with pytest.raises(ValueError, match="key_mask"):
        ops.key_operands(torch.ones(2, 4, dtype=torch.bool), None, 2, 3, CPU)
    with pytest.raises(ValueError, match="key_bias"):
        ops.key_operands(None, torch.zeros(5), 2, 3, CPU)


def test_operands_on_another_device_are_refused():
    with pytest.raises(ValueError, match="must be on"):
        ops.key_operands(torch.ones(1, 3, dtype=torch.bool), None, 1, 3, torch.device("meta"))
    with pytest.raises(ValueError, match="must be on"):
        ops.key_operands(None, torch.zeros(1, 3), 1, 3, torch.device("meta"))
